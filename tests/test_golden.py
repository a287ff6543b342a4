"""Golden fixtures (tests/golden/*.json) against the CPU oracle and the HIP kernels.

The fixtures come from tests/golden/make_golden.py, a second restatement of
the reference rules in exact rational arithmetic that shares no code with
oracle/mxfp4_oracle.c (the reference itself ships no golden vectors). The
CPU tests pin the oracle to them; the GPU tests run the same vectors through
the C ABI.
"""
import base64
import json
import os

import numpy as np
import pytest
import torch

from helpers import bits_u16, bits_u8, from_u16

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def quant_vectors():
    g = _load("quant_blocks.json")
    x = np.concatenate([np.frombuffer(bytes.fromhex(b["x"]), np.uint16) for b in g["blocks"]])
    scales = np.array([b["scale"] for b in g["blocks"]], np.uint8)
    codes = np.concatenate([np.frombuffer(bytes.fromhex(b["codes"]), np.uint8) for b in g["blocks"]])
    return g["eps"], x, scales, codes


def dequant_vectors():
    """Codes: byte n | n << 4 for n = 0..15 (both nibbles n), 8 blocks per scale
    byte; expected bf16 bits per element (None where unpinned)."""
    t = _load("dequant_table.json")["table"]
    q = np.zeros(256 * 128, np.uint8)
    for s in range(256):
        q[s * 128: s * 128 + 16] = np.arange(16) | (np.arange(16) << 4)
    sc = np.repeat(np.arange(256, dtype=np.uint8), 8)  # 128 code bytes = 256 elements = 8 blocks
    return q, sc, t


def fp8_vectors():
    g = _load("fp8_rowwise_groups.json")["groups"]
    codes = np.stack([np.frombuffer(bytes.fromhex(x["codes"]), np.uint8) for x in g])
    scales = np.array([x["scales"] for x in g], np.uint8)
    fp8 = np.stack([np.frombuffer(bytes.fromhex(x["fp8"]), np.uint8) for x in g])
    sbits = np.array([x["scale_bits"] for x in g], np.uint32)
    return codes, scales, fp8, sbits


def row_to_col_vectors(kind):
    """Dense or per-split row -> col FP8 cases: dicts with codes [M, N/2],
    scales [M, N/32], expected fp8 bytes and scale-row bit patterns."""
    cases = []
    for c in _load("row_to_col_fp8.json")[kind]:
        N = c["N"]
        M = c["M"] if kind == "dense" else sum(c["splits"])
        b = {k: np.frombuffer(base64.b64decode(c[k]), np.uint8) for k in ("codes", "scales", "fp8")}
        cases.append({"M": M, "N": N, "eps": c["eps"], "splits": c.get("splits"),
                      "codes": b["codes"].reshape(M, N // 2), "scales": b["scales"].reshape(M, N // 32),
                      "fp8": b["fp8"], "scale_bits": np.array(c["scale_bits"], np.uint32).reshape(-1, N)})
    return cases


def _check_dequant(out_bits, table):
    checked = 0
    for s in range(256):
        for n in range(16):
            e = table[str(s)][n]
            if e is None:
                continue
            base = s * 256 + 2 * n
            assert int(out_bits[base]) == e and int(out_bits[base + 1]) == e, (s, n, hex(out_bits[base]), hex(e))
            checked += 2
    return checked


# ------------------------------------------------------------------ CPU: oracle
def test_golden_quant_oracle(oracle):
    eps, x, scales, codes = quant_vectors()
    q, s = oracle.quant_mxfp4(x, eps=eps)
    np.testing.assert_array_equal(s, scales)
    np.testing.assert_array_equal(q, codes)


def test_golden_dequant_oracle(oracle):
    q, sc, table = dequant_vectors()
    assert _check_dequant(oracle.dequant_bf16(q, sc), table) == 256 * 32 - 2 * 2


def test_golden_fp8_rowwise_oracle(oracle):
    codes, scales, fp8, sbits = fp8_vectors()
    o, os_ = oracle.mxfp4_to_fp8(codes, scales)
    np.testing.assert_array_equal(o, fp8)
    np.testing.assert_array_equal(os_.view(np.uint32)[0], sbits)


def test_golden_row_to_col_oracle(oracle):
    for c in row_to_col_vectors("dense"):
        o, os_ = oracle.row_to_fp8_col(c["codes"], c["scales"], eps=c["eps"])
        np.testing.assert_array_equal(o.reshape(-1), c["fp8"], err_msg=f"{c['M']}x{c['N']} eps {c['eps']}")
        np.testing.assert_array_equal(os_.view(np.uint32), c["scale_bits"])


def test_golden_msplit_oracle(oracle):
    for c in row_to_col_vectors("msplit"):
        o, os_ = oracle.row_to_fp8_col_msplit(c["codes"], c["scales"], c["splits"], eps=c["eps"])
        np.testing.assert_array_equal(o, c["fp8"], err_msg=f"{c['splits']} {c['N']} eps {c['eps']}")
        np.testing.assert_array_equal(os_.view(np.uint32), c["scale_bits"])


# ------------------------------------------------------------------ GPU: HIP path
@pytest.mark.gpu
def test_golden_quant_gpu(dev):
    import omo
    eps, x, scales, codes = quant_vectors()
    xt = from_u16(x, dev)
    q = torch.empty(x.size // 2, dtype=torch.uint8, device=dev)
    s = torch.empty((1, x.size // 32), dtype=torch.uint8, device=dev)  # the reference checks a 2-D scale tensor
    omo.omo_per_token_group_quant_fp4(xt, q, s, 32, eps, -6.0, 6.0, False)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits_u8(s).reshape(-1), scales)
    np.testing.assert_array_equal(bits_u8(q), codes)


@pytest.mark.gpu
def test_golden_dequant_gpu(dev):
    import omo
    q, sc, table = dequant_vectors()
    out = torch.empty(q.size * 2, dtype=torch.bfloat16, device=dev)
    omo.omo_per_token_Mxfp4ToBf16_dequant(torch.from_numpy(q).to(dev), torch.from_numpy(sc).to(dev), out,
                                          torch.empty((1, 1), device=dev), 32, 1e-10, -6.0, 6.0, False)
    torch.cuda.synchronize()
    assert _check_dequant(bits_u16(out).reshape(-1), table) == 256 * 32 - 2 * 2


@pytest.mark.gpu
def test_golden_fp8_rowwise_gpu(dev):
    import omo
    codes, scales, fp8, sbits = fp8_vectors()
    G = codes.shape[0]
    out = torch.empty((G, 128), dtype=torch.float8_e4m3fn, device=dev)
    outs = torch.empty((1, G), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4ToFp8(torch.from_numpy(codes).to(dev), torch.from_numpy(scales).to(dev), out, outs, 128,
                                 1e-10, -6.0, 6.0, False)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits_u8(out), fp8)
    np.testing.assert_array_equal(outs.cpu().numpy().view(np.uint32)[0], sbits)


@pytest.mark.gpu
def test_golden_row_to_col_gpu(dev):
    import omo
    for c in row_to_col_vectors("dense"):
        M, N = c["M"], c["N"]
        out = torch.empty((N, M), dtype=torch.float8_e4m3fn, device=dev)
        outs = torch.empty(((M + 127) // 128, N), dtype=torch.float32, device=dev)
        omo.omo_per_token_Mxfp4RowToBf16ToFp8Col(torch.from_numpy(c["codes"].copy()).to(dev),
                                                torch.from_numpy(c["scales"].copy()).to(dev), out, outs, c["eps"])
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits_u8(out).reshape(-1), c["fp8"], err_msg=f"{M}x{N} eps {c['eps']}")
        np.testing.assert_array_equal(outs.cpu().numpy().view(np.uint32), c["scale_bits"])


@pytest.mark.gpu
def test_golden_msplit_gpu(dev):
    from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4RowToBf16ToFp8Col_msplit_wrapper
    for c in row_to_col_vectors("msplit"):
        ys, ss = omo_per_token_mxfp4RowToBf16ToFp8Col_msplit_wrapper(
            torch.from_numpy(c["codes"].copy()).to(dev), torch.from_numpy(c["scales"].copy()).to(dev), c["splits"],
            eps=c["eps"])
        torch.cuda.synchronize()
        got = np.concatenate([bits_u8(y).reshape(-1) for y in ys])
        np.testing.assert_array_equal(got, c["fp8"], err_msg=f"{c['splits']} {c['N']} eps {c['eps']}")
        np.testing.assert_array_equal(torch.cat(ss).cpu().numpy().view(np.uint32), c["scale_bits"])
