"""CPU-only checks of the boundary: the C ABI library loads and exports every
function declared in include/omo_mxfp4.h, argument validation runs (and
fails correctly) before any HIP call, and the Python layers apply the
reference's host checks. No call here reaches a kernel launch.
"""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from conftest import ROOT


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "omo_mxfp4.h")).read()
    return re.findall(r"OMO_API\s+(?:const\s+)?\w+\*?\s+(omo_hip_\w+)\s*\(", text)


def test_header_declares_the_reference_entry_points():
    names = set(declared_symbols())
    for n in ["omo_hip_per_token_group_quant_fp4", "omo_hip_per_token_Mxfp4ToBf16_dequant",
              "omo_hip_per_token_Mxfp4ToFp8", "omo_hip_per_token_Mxfp4ToBf16ToFp8",
              "omo_hip_per_token_Mxfp4ToFp8_col", "omo_hip_per_token_Mxfp4RowToBf16ToFp8Col",
              "omo_hip_per_token_Mxfp4RowToBf16ToFp8Col_msplit", "omo_hip_quant_mxfp4_dual",
              "omo_hip_quant_mxfp4_packed", "omo_hip_packed_Mxfp4ToBf16_dequant", "omo_hip_packed_Mxfp4ToFp8",
              "omo_hip_mxfp4_permute_rows", "omo_hip_permute_Mxfp4ToFp8", "omo_hip_quant_mxfp4_dual_grouped",
              "omo_hip_abi_version", "omo_hip_status_string", "omo_hip_last_error"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    from omo import _abi
    lib = ctypes.CDLL(_abi.LIB_PATH)
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert _abi.lib.omo_hip_abi_version() == 1
    assert _abi.lib.omo_hip_status_string(-1) == b"invalid argument"


def _lib():
    from omo import _abi
    return _abi.lib


def test_quant_validation_paths():
    lib = _lib()
    P = ctypes.c_void_p
    fake = P(0x1000)  # never dereferenced: every call below fails validation
    # numel % group_size
    assert lib.omo_hip_per_token_group_quant_fp4(fake, 40, fake, 20, fake, 1, 32, 1e-10, -6.0, 6.0, 0, None) == -1
    assert b"group_size" in lib.omo_hip_last_error()
    # unsupported modes
    assert lib.omo_hip_per_token_group_quant_fp4(fake, 64, fake, 32, fake, 2, 32, 1e-10, -6.0, 6.0, 1, None) == -2
    assert lib.omo_hip_per_token_group_quant_fp4(fake, 128, fake, 64, fake, 2, 64, 1e-10, -6.0, 6.0, 0, None) == -2
    # undersized outputs, null pointers, misalignment, bad constants
    assert lib.omo_hip_per_token_group_quant_fp4(fake, 64, fake, 31, fake, 2, 32, 1e-10, -6.0, 6.0, 0, None) == -1
    assert lib.omo_hip_per_token_group_quant_fp4(None, 64, fake, 32, fake, 2, 32, 1e-10, -6.0, 6.0, 0, None) == -1
    assert lib.omo_hip_per_token_group_quant_fp4(P(0x1002), 64, fake, 32, fake, 2, 32, 1e-10, -6.0, 6.0, 0, None) == -1
    assert lib.omo_hip_per_token_group_quant_fp4(fake, 64, fake, 32, fake, 2, 32, float("nan"), -6.0, 6.0, 0,
                                                 None) == -1
    assert lib.omo_hip_per_token_group_quant_fp4(fake, 64, fake, 32, fake, 2, 32, 1e-10, -6.0, 0.0, 0, None) == -1
    # empty input is a no-op success
    assert lib.omo_hip_per_token_group_quant_fp4(None, 0, None, 0, None, 0, 32, 1e-10, -6.0, 6.0, 0, None) == 0


def test_requant_validation_paths():
    lib = _lib()
    f = ctypes.c_void_p(0x1000)
    # dequant: numel % 128
    assert lib.omo_hip_per_token_Mxfp4ToBf16_dequant(f, 64, f, 4, f, 128, None, 0, 32, 1e-10, -6.0, 6.0, 0,
                                                     None) == -1
    # rowwise fp8: row bytes % 64, numel % 128
    assert lib.omo_hip_per_token_Mxfp4ToFp8(f, 4, 32, f, 8, f, 256, f, 2, 128, 1e-10, -6.0, 6.0, 0, None) == -1
    assert lib.omo_hip_per_token_Mxfp4ToFp8(f, 3, 64, f, 12, f, 384, f, 3, 128, 1e-10, -6.0, 6.0, 0, None) == -1
    assert lib.omo_hip_per_token_Mxfp4ToBf16ToFp8(f, 2, 64, f, 8, f, 255, f, 2, 128, 1e-10, -6.0, 6.0, 0,
                                                  None) == -1
    # col: whole 128x128-byte tiles only
    assert lib.omo_hip_per_token_Mxfp4ToFp8_col(f, 64, 128, f, 512, f, 16384, f, 128, 128, 1e-10, -6.0, 6.0, 0,
                                                None) == -1
    # row->col: the reference's shape checks
    assert lib.omo_hip_per_token_Mxfp4RowToBf16ToFp8Col(f, 4, 32, f, 4, 1, f, 64, 4, f, 1, 64, 1e-10, None) == -1
    assert lib.omo_hip_per_token_Mxfp4RowToBf16ToFp8Col(f, 4, 32, f, 4, 2, f, 4, 64, f, 1, 64, 1e-10, None) == -1
    # msplit: output too small
    assert lib.omo_hip_per_token_Mxfp4RowToBf16ToFp8Col_msplit(f, 4, 32, f, 8, f, 100, f, 64, f, f, f, 1, 4,
                                                               1e-10, None) == -1
    # dual: multiples of 32
    assert lib.omo_hip_quant_mxfp4_dual(f, 48, 32, f, 768, f, 48, f, 768, f, 48, 1e-10, None) == -1


def test_omo_binding_host_checks():
    import omo
    x = torch.zeros((2, 64), dtype=torch.bfloat16)
    q = torch.zeros((2, 32), dtype=torch.uint8)
    s = torch.zeros((2, 2), dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        omo.omo_per_token_group_quant_fp4(x, q, s, 32, 1e-10, -6.0, 6.0, False)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        omo.omo_per_token_Mxfp4ToBf16_dequant(q, s, x, torch.zeros(1, 1), 32, 1e-10, -6.0, 6.0, False)
    with pytest.raises(NotImplementedError):
        omo.omo_per_token_group_quant_fp4_fused_ToFp8(x, q, s, x, s, 32, 1e-10, -6.0, 6.0, False)
    # keyword names of the reference binding (code/kernel/ops.cu:28-41)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        omo.omo_per_token_group_quant_fp4(input=x, output_q=q, output_s=s, group_size=32, eps=1e-10, fp4_min=-6.0,
                                          fp4_max=6.0, scale_ue8m0=False)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        omo.omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit(input=q, input_s=s, output_q=q, output_s=s, m_splits=s,
                                                        split_offsets=s, scale_offsets=s, max_split_len=2, eps=1e-10)


def test_wrapper_host_helpers():
    from omo_python_api.mxfp4_dequant import pad_to_multiple, split_metadata, unpad_from_multiple
    x = torch.arange(2 * 70, dtype=torch.uint8).view(2, 70)
    p, w = pad_to_multiple(x, 64)
    assert p.shape == (2, 128) and w == 70 and torch.equal(p[:, :70], x) and int(p[:, 70:].sum()) == 0
    same, w2 = pad_to_multiple(x[:, :64].contiguous(), 64)
    assert same.shape == (2, 64) and w2 == 64
    assert unpad_from_multiple(p, 70).shape == (2, 70)
    lens, offs, soffs, mx, rows, srows = split_metadata([1, 127, 0, 128, 300], "cpu")
    assert lens.tolist() == [1, 127, 0, 128, 300]
    assert offs.tolist() == [0, 1, 128, 128, 256]
    assert soffs.tolist() == [0, 1, 2, 2, 3]
    assert (mx, rows, srows) == (300, 556, 6)
    assert lens.dtype == torch.int32


def test_bench_refuses_more_than_one_gpu():
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "exactly one GPU" in r.stdout


def test_last_error_is_per_thread():
    # the failure message belongs to the calling thread: two threads failing
    # different checks at once each read back their own message
    import threading
    lib = _lib()
    P = ctypes.c_void_p
    barrier = threading.Barrier(2)
    got = {}

    def fail_with(group_size, key):
        for _ in range(200):
            rc = lib.omo_hip_per_token_group_quant_fp4(P(1), 64, P(1), 32, P(1), 2, group_size, 1e-10, -6.0, 6.0, 0,
                                                       None)
            barrier.wait()
            msg = lib.omo_hip_last_error()
            barrier.wait()
            got.setdefault(key, set()).add((rc, msg))

    ts = [threading.Thread(target=fail_with, args=(0, "zero")), threading.Thread(target=fail_with, args=(64, "g64"))]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert len(got["zero"]) == 1 and len(got["g64"]) == 1
    (rc0, m0), = got["zero"]
    (rc1, m1), = got["g64"]
    assert b"positive" in m0 and b"must be 32" in m1 and rc0 != 0 and rc1 != 0


def test_bench_floor_library_exports_and_shape_checks():
    # the memory-only kernels bench.py times beside the codec kernels: exported,
    # and shapes they do not cover are refused on the host before any launch
    lib = ctypes.CDLL(os.path.join(ROOT, "mxfp4-hopper_amd", "lib", "libomo_ceiling.so"))
    for name in ["omo_ceiling_launch", "omo_floor_dual", "omo_floor_dual_variant", "omo_floor_rowcol", "omo_floor_msplit",
                 "omo_floor_msplit_band", "omo_floor_requant", "omo_floor_dequant", "omo_floor_dual_grouped"]:
        assert hasattr(lib, name), name
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    lib.omo_floor_dual.argtypes = [P, P, P, P, P, I64, I64, P]
    lib.omo_floor_rowcol.argtypes = [P, P, P, P, I64, I64, P]
    lib.omo_floor_msplit.argtypes = [P, P, P, P, I64, I64, P, P, P, I64, I64, I64, P]
    lib.omo_floor_requant.argtypes = [P, P, P, P, I64, I64, P]
    lib.omo_floor_dequant.argtypes = [P, P, P, I64, P]
    assert lib.omo_floor_dual(None, None, None, None, None, 7168, 18432 + 32, None) == -1
    assert lib.omo_floor_dual(None, None, None, None, None, 0, 256, None) == -1
    assert lib.omo_floor_rowcol(None, None, None, None, 4096 + 64, 7168, None) == -1
    assert lib.omo_floor_rowcol(None, None, None, None, 4096, 7168 + 128, None) == -1
    assert lib.omo_floor_msplit(None, None, None, None, 100, 7168 + 128, None, None, None, 2, 60, 2, None) == -1
    assert lib.omo_floor_msplit(None, None, None, None, 100, 7168, None, None, None, 2, 101, 2, None) == -1
    assert lib.omo_floor_msplit(None, None, None, None, 100, 7168, None, None, None, 0, 60, 2, None) == -1
    assert lib.omo_floor_requant(None, None, None, None, 4096, 3584 + 32, None) == -1
    assert lib.omo_floor_dequant(None, None, None, 0, None) == -1
    lib.omo_floor_dual_variant.argtypes = [ctypes.c_int, P, P, P, P, P, I64, I64, P]
    lib.omo_floor_msplit_band.argtypes = [P, P, P, P, I64, P, P, P, I64, I64, P]
    assert lib.omo_floor_dual_variant(0, None, None, None, None, None, 7168, 18432, None) == -1  # kinds 1..5
    assert lib.omo_floor_dual_variant(6, None, None, None, None, None, 7168, 18432, None) == -1
    # aligned groups need whole 8-band groups
    assert lib.omo_floor_dual_variant(5, None, None, None, None, None, 7168, 18432 + 256, None) == -1
    assert lib.omo_floor_dual_variant(1, None, None, None, None, None, 7168 + 64, 18432, None) == -1
    # the band schedule holds a whole split's band in LDS: longer splits and N % 64 are refused
    assert lib.omo_floor_msplit_band(None, None, None, None, 7168, None, None, None, 8, 4353, None) == -1
    assert lib.omo_floor_msplit_band(None, None, None, None, 7168 + 32, None, None, None, 8, 2000, None) == -1
    assert lib.omo_floor_msplit_band(None, None, None, None, 7168, None, None, None, 0, 2000, None) == -1
    # grouped: at most 32 items, each M % 64 == 0 and K % 256 == 0, scm 0 or 1
    lib.omo_floor_dual_grouped.argtypes = [ctypes.c_int, P, P, P, P, P, P, P, ctypes.c_int, P]
    ptrs = (ctypes.c_void_p * 2)(None, None)
    ms, ks = (ctypes.c_int64 * 2)(7168, 2048), (ctypes.c_int64 * 2)(2048, 7168)
    bad_m, bad_k = (ctypes.c_int64 * 2)(7168, 2048 + 32), (ctypes.c_int64 * 2)(2048, 7168 + 128)
    assert lib.omo_floor_dual_grouped(2, ptrs, ptrs, ptrs, ptrs, ptrs, ms, ks, 2, None) == -1
    assert lib.omo_floor_dual_grouped(0, ptrs, ptrs, ptrs, ptrs, ptrs, ms, ks, 0, None) == -1
    assert lib.omo_floor_dual_grouped(0, ptrs, ptrs, ptrs, ptrs, ptrs, ms, ks, 33, None) == -1
    assert lib.omo_floor_dual_grouped(0, ptrs, ptrs, ptrs, ptrs, ptrs, bad_m, ks, 2, None) == -1
    assert lib.omo_floor_dual_grouped(1, ptrs, ptrs, ptrs, ptrs, ptrs, ms, bad_k, 2, None) == -1


def test_payload_validation_paths():
    lib = _lib()
    f = ctypes.c_void_p(0x1000)
    # cols % 128 (payload rows must stay dword aligned)
    assert lib.omo_hip_quant_mxfp4_packed(f, 2, 96, f, 2 * 51, 1e-10, None) == -1
    assert b"multiple of 128" in lib.omo_hip_last_error()
    # undersized output, misaligned input, non-finite eps
    assert lib.omo_hip_quant_mxfp4_packed(f, 2, 128, f, 2 * 68 - 1, 1e-10, None) == -1
    assert lib.omo_hip_quant_mxfp4_packed(ctypes.c_void_p(0x1008), 2, 128, f, 136, 1e-10, None) == -1
    assert lib.omo_hip_quant_mxfp4_packed(f, 2, 128, f, 136, float("inf"), None) == -1
    assert lib.omo_hip_packed_Mxfp4ToBf16_dequant(f, 2, 128, f, 255, None) == -1
    assert lib.omo_hip_packed_Mxfp4ToBf16_dequant(ctypes.c_void_p(0x1002), 2, 128, f, 256, None) == -1
    assert lib.omo_hip_packed_Mxfp4ToFp8(f, 2, 128, f, 256, f, 1, None) == -1
    # empty payloads are no-op successes
    assert lib.omo_hip_quant_mxfp4_packed(None, 0, 7168, None, 0, 1e-10, None) == 0
    assert lib.omo_hip_packed_Mxfp4ToBf16_dequant(None, 0, 7168, None, 0, None) == 0
    assert lib.omo_hip_packed_Mxfp4ToFp8(None, 0, 7168, None, 0, None, 0, None) == 0


def test_payload_join_split_layout():
    """Payload rows are [H/2 code bytes | H/32 scale bytes]: join/split
    against byte-for-byte numpy placement, contiguous parts, shape errors."""
    from omo_python_api.ep_payload import hidden_of, join_payload, payload_width, split_payload
    g = torch.Generator().manual_seed(3)
    q = torch.randint(0, 256, (5, 3584), generator=g, dtype=torch.uint8)
    s = torch.randint(0, 256, (5, 224), generator=g, dtype=torch.uint8)
    p = join_payload(q, s)
    assert p.shape == (5, payload_width(7168)) == (5, 3808) and hidden_of(p) == 7168
    exp = np.zeros((5, 3808), np.uint8)
    for t in range(5):
        exp[t, :3584] = q[t].numpy()
        exp[t, 3584:] = s[t].numpy()
    np.testing.assert_array_equal(p.numpy(), exp)
    uq, us = split_payload(p)
    assert torch.equal(uq, q) and torch.equal(us, s) and uq.is_contiguous() and us.is_contiguous()
    with pytest.raises(ValueError, match="tokens"):
        join_payload(q, s[:4])
    with pytest.raises(ValueError, match="scale bytes"):
        join_payload(q, s[:, :200])
    with pytest.raises(ValueError, match="17/32"):
        split_payload(torch.zeros((2, 100), dtype=torch.uint8))
    with pytest.raises(ValueError, match="2-D"):
        split_payload(torch.zeros((), dtype=torch.uint8))


def test_make_row_id_map_expert_major():
    """Routed (token, expert) pairs in expert-major order, tokens ascending
    within an expert; padding rows -1; dest is the inverse map."""
    from omo_python_api.permutation import make_row_id_map
    rm = torch.tensor([[1, 0, 1],
                       [0, 1, 1],
                       [1, 1, 0],
                       [0, 0, 0]], dtype=torch.bool)
    src, m_splits, dest = make_row_id_map(rm, num_out_tokens=8)
    assert m_splits == [2, 2, 2]
    assert src.tolist() == [0, 2, 1, 2, 0, 1, -1, -1]
    assert dest.tolist() == [[0, -1, 4], [-1, 2, 5], [1, 3, -1], [-1, -1, -1]]
    with pytest.raises(ValueError):
        make_row_id_map(rm, num_out_tokens=5)


def test_permute_validation_paths():
    lib = _lib()
    f = ctypes.c_void_p(0x1000)
    # cols % 32; stride shorter than the row; undersized input; null indices
    assert lib.omo_hip_mxfp4_permute_rows(f, 1 << 20, 24, f, 1 << 20, 2, 4, 48, f, 4, f, 96, f, 8, None) == -1
    assert lib.omo_hip_mxfp4_permute_rows(f, 1 << 20, 32, f, 1 << 20, 4, 4, 128, f, 4, f, 256, f, 16, None) == -1
    assert lib.omo_hip_mxfp4_permute_rows(f, 100, 64, f, 1 << 20, 4, 4, 128, f, 4, f, 256, f, 16, None) == -1
    assert lib.omo_hip_mxfp4_permute_rows(f, 1 << 20, 64, f, 1 << 20, 4, 4, 128, None, 4, f, 256, f, 16,
                                          None) == -1
    # fused fp8: cols % 128, 4-byte rows, output size
    assert lib.omo_hip_permute_Mxfp4ToFp8(f, 1 << 20, 48, f, 1 << 20, 3, 4, 96, f, 4, f, 384, f, 4, None) == -1
    assert lib.omo_hip_permute_Mxfp4ToFp8(f, 1 << 20, 66, f, 1 << 20, 4, 4, 128, f, 4, f, 512, f, 4, None) == -1
    assert lib.omo_hip_permute_Mxfp4ToFp8(f, 1 << 20, 64, f, 1 << 20, 4, 4, 128, f, 4, f, 511, f, 4, None) == -1
    # nothing to do
    assert lib.omo_hip_permute_Mxfp4ToFp8(f, 1 << 20, 64, f, 1 << 20, 4, 4, 128, None, 0, None, 0, None, 0,
                                          None) == 0


def test_dual_grouped_validation_paths():
    from omo._abi import DualItem
    lib = _lib()
    f = 0x1000
    good = DualItem(f, 32, 32, f, 512, f, 32, f, 512, f, 32)
    bad = DualItem(f, 48, 32, f, 768, f, 48, f, 768, f, 48)  # rows % 32
    arr = (DualItem * 2)(good, bad)
    assert lib.omo_hip_quant_mxfp4_dual_grouped(arr, 2, 1e-10, None) == -1
    assert b"item 1" in lib.omo_hip_last_error()
    assert lib.omo_hip_quant_mxfp4_dual_grouped(arr, 1, float("nan"), None) == -1
    assert lib.omo_hip_quant_mxfp4_dual_grouped(None, 3, 1e-10, None) == -1
    assert lib.omo_hip_quant_mxfp4_dual_grouped(None, 0, 1e-10, None) == 0


def test_oversized_shapes_rejected():
    """Shapes whose byte counts overflow 64-bit arithmetic are refused before
    any size check could wrap (fake pointers, never dereferenced)."""
    lib = _lib()
    f = ctypes.c_void_p(0x1000)
    big = 1 << 62

    def refused(rc, what=b"too large"):
        assert rc == -1 and what in lib.omo_hip_last_error(), lib.omo_hip_last_error()

    refused(lib.omo_hip_per_token_Mxfp4ToBf16_dequant(f, big, f, big, f, big, None, 0, 32, 1e-10, -6.0, 6.0, 0, None))
    for fn in (lib.omo_hip_per_token_Mxfp4ToFp8, lib.omo_hip_per_token_Mxfp4ToBf16ToFp8,
               lib.omo_hip_per_token_Mxfp4ToFp8_col):
        refused(fn(f, 1 << 40, 1 << 30, f, big, f, big, f, big, 128, 1e-10, -6.0, 6.0, 0, None))
    # 2^34 x 2^31 bytes wraps to 0 in int64, a multiple of everything
    refused(lib.omo_hip_per_token_Mxfp4ToFp8(f, 1 << 33, 1 << 31, f, big, f, big, f, big, 128, 1e-10, -6.0, 6.0, 0,
                                             None))
    refused(lib.omo_hip_per_token_Mxfp4RowToBf16ToFp8Col(f, 1 << 40, 1 << 30, f, 1 << 40, 1 << 26, f, 1 << 31,
                                                         1 << 40, f, 1 << 33, 1 << 31, 1e-10, None))
    refused(lib.omo_hip_per_token_Mxfp4RowToBf16ToFp8Col(f, 1, big, f, 1, 1, f, 1, 1, f, 1, 1, 1e-10, None))
    refused(lib.omo_hip_per_token_Mxfp4RowToBf16ToFp8Col_msplit(f, 1 << 40, 1 << 30, f, big, f, big, f, big, f, f, f,
                                                                1, 1 << 40, 1e-10, None))
    refused(lib.omo_hip_quant_mxfp4_dual(f, 1 << 40, 1 << 40, f, big, f, big, f, big, f, big, 1e-10, None),
            b"too many tiles")
    refused(lib.omo_hip_mxfp4_permute_rows(f, big, 1 << 61, f, big, 4, 4, 128, f, 4, f, 256, f, 16, None))
    refused(lib.omo_hip_mxfp4_permute_rows(f, big, 1 << 40, f, big, 1 << 40, 1 << 30, 128, f, 4, f, 256, f, 16,
                                           None))
    refused(lib.omo_hip_permute_Mxfp4ToFp8(f, 1 << 20, 1 << 40, f, 1 << 20, 1 << 36, 1, 1 << 40, f, 1 << 30, f, big,
                                           f, big, None))
