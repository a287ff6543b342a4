"""ctypes front end of the CPU oracle (``liboracle_mxfp4.so``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, never by the product path. Every
function here returns numpy arrays computed by the C restatement of the
reference kernels in ``mxfp4_oracle.c`` (each C function cites the reference
file:line it follows).

Inputs and outputs are raw bit patterns: bf16 as ``uint16``, FP8 E4M3 and
E2M1/E8M0 bytes as ``uint8``, fp32 scales as ``float32``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_mxfp4.so")
_lib = None


def build() -> str:
    """Compile the oracle with its Makefile (gcc only); returns the .so path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P, I64, F, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int
        sig = {
            "oracle_quant_mxfp4": [P, I64, F, F, F, P, P, I],
            "oracle_dequant_bf16": [P, P, I64, P, I],
            "oracle_mxfp4_to_fp8": [P, P, I64, I64, P, P, I],
            "oracle_mxfp4_to_fp8_col": [P, P, I64, I64, F, P, P, I],
            "oracle_row_to_fp8_col": [P, P, I64, I64, F, P, P, I],
            "oracle_row_to_fp8_col_msplit": [P, P, I64, P, P, P, I64, I64, F, P, P, I],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        L.oracle_e2m1_from_f32.argtypes = [F]
        L.oracle_e2m1_from_f32.restype = ctypes.c_uint8
        L.oracle_e8m0_scale_from_amax.argtypes = [F, F]
        L.oracle_e8m0_scale_from_amax.restype = ctypes.c_uint8
        L.oracle_f32_to_e4m3.argtypes = [F]
        L.oracle_f32_to_e4m3.restype = ctypes.c_uint8
        L.oracle_f32_to_bf16.argtypes = [F]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_e2m1_to_bf16_bits.argtypes = [ctypes.c_uint8]
        L.oracle_e2m1_to_bf16_bits.restype = ctypes.c_uint16
        L.oracle_te_pow2_scale.argtypes = [F, F]
        L.oracle_te_pow2_scale.restype = F
        _lib = L
    return _lib


def _threads(n):
    return n if n else min(16, os.cpu_count() or 1)


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _check(rc, name):
    if rc != 0:
        raise ValueError(f"{name}: invalid arguments (rc={rc})")


def quant_mxfp4(x_bits, eps=1e-10, fp4_min=-6.0, fp4_max=6.0, nthreads=0):
    """BF16 (uint16 bits, any shape, numel % 32 == 0) -> (codes uint8 [numel/2],
    scales uint8 [numel/32]) in flat group order."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16).reshape(-1)
    codes = np.empty(x.size // 2, np.uint8)
    scales = np.empty(x.size // 32, np.uint8)
    _check(lib().oracle_quant_mxfp4(_p(x), x.size, eps, fp4_min, fp4_max, _p(codes), _p(scales),
                                    _threads(nthreads)), "quant")
    return codes, scales


def dequant_bf16(codes, scales, nthreads=0):
    """Flat codes (nbytes % 128 == 0) + flat scales -> bf16 bits [2*nbytes]."""
    q = np.ascontiguousarray(codes, dtype=np.uint8).reshape(-1)
    s = np.ascontiguousarray(scales, dtype=np.uint8).reshape(-1)
    assert s.size >= q.size // 16
    out = np.empty(q.size * 2, np.uint16)
    _check(lib().oracle_dequant_bf16(_p(q), _p(s), q.size, _p(out), _threads(nthreads)), "dequant")
    return out


def mxfp4_to_fp8(codes, scales, nthreads=0):
    """codes [M, Kb] (Kb % 64 == 0), scales [M, Kb/16] -> (fp8 [M, 2Kb], fp32 [Kb/64, M])."""
    q = np.ascontiguousarray(codes, dtype=np.uint8)
    M, Kb = q.shape
    s = np.ascontiguousarray(scales, dtype=np.uint8).reshape(-1)
    assert s.size >= M * Kb // 16
    out = np.empty((M, 2 * Kb), np.uint8)
    outs = np.empty((Kb // 64, M), np.float32)
    _check(lib().oracle_mxfp4_to_fp8(_p(q), _p(s), M, Kb, _p(out), _p(outs), _threads(nthreads)), "to_fp8")
    return out, outs


def mxfp4_to_fp8_col(codes, scales, eps=1e-10, nthreads=0):
    """codes [M, Kb] (M, Kb % 128 == 0) -> (fp8 [2Kb, M], fp32 [M/128, 2Kb])."""
    q = np.ascontiguousarray(codes, dtype=np.uint8)
    M, Kb = q.shape
    s = np.ascontiguousarray(scales, dtype=np.uint8).reshape(-1)
    assert s.size >= M * Kb // 16
    out = np.empty((2 * Kb, M), np.uint8)
    outs = np.empty((M // 128, 2 * Kb), np.float32)
    _check(lib().oracle_mxfp4_to_fp8_col(_p(q), _p(s), M, Kb, eps, _p(out), _p(outs), _threads(nthreads)),
           "to_fp8_col")
    return out, outs


def row_to_fp8_col(codes, scales, eps=1e-10, nthreads=0):
    """codes [M, N/2], scales [M, ceil(N/32)] -> (fp8 [N, M], fp32 [ceil(M/128), N])."""
    q = np.ascontiguousarray(codes, dtype=np.uint8)
    M, half = q.shape
    N = 2 * half
    s = np.ascontiguousarray(scales, dtype=np.uint8).reshape(-1)
    out = np.empty((N, M), np.uint8)
    outs = np.empty(((M + 127) // 128, N), np.float32)
    _check(lib().oracle_row_to_fp8_col(_p(q), _p(s), M, N, eps, _p(out), _p(outs), _threads(nthreads)),
           "row_to_fp8_col")
    return out, outs


def split_metadata(m_splits):
    """Exclusive prefix sums used by the grouped kernel: (lens, row offsets,
    scale-row offsets, max split length), all int32 except the last."""
    lens = np.asarray(m_splits, dtype=np.int32)
    offs = np.zeros_like(lens)
    soffs = np.zeros_like(lens)
    if lens.size:
        offs[1:] = np.cumsum(lens)[:-1]
        soffs[1:] = np.cumsum((lens + 127) // 128)[:-1]
    mx = int(lens.max()) if lens.size else 0
    return lens, offs, soffs, mx


def row_to_fp8_col_msplit(codes, scales, m_splits, eps=1e-10, nthreads=0, max_split_len=None):
    """Grouped variant. Returns (flat fp8 [sum(M) * N], fp32 [sum(ceil(len/128)), N])."""
    q = np.ascontiguousarray(codes, dtype=np.uint8)
    Mt, half = q.shape
    N = 2 * half
    s = np.ascontiguousarray(scales, dtype=np.uint8).reshape(-1)
    lens, offs, soffs, mx = split_metadata(m_splits)
    if max_split_len is not None:
        mx = max_split_len
    out = np.zeros(Mt * N, np.uint8)
    outs = np.zeros((int(((lens + 127) // 128).sum()), N), np.float32)
    _check(lib().oracle_row_to_fp8_col_msplit(_p(q), _p(s), N, _p(lens), _p(offs), _p(soffs), lens.size, mx,
                                              eps, _p(out), _p(outs), _threads(nthreads)), "msplit")
    return out, outs


def e2m1_from_f32(q: float) -> int:
    return int(lib().oracle_e2m1_from_f32(float(q)))


def e8m0_scale_from_amax(amax: float, fp4_max: float = 6.0) -> int:
    return int(lib().oracle_e8m0_scale_from_amax(float(amax), float(fp4_max)))


def f32_to_e4m3(f: float) -> int:
    return int(lib().oracle_f32_to_e4m3(float(f)))


def f32_to_bf16(f: float) -> int:
    return int(lib().oracle_f32_to_bf16(float(f)))


def e2m1_to_bf16_bits(nib: int) -> int:
    return int(lib().oracle_e2m1_to_bf16_bits(nib))


def te_pow2_scale(amax: float, eps: float = 1e-10) -> float:
    return float(lib().oracle_te_pow2_scale(float(amax), float(eps)))
