"""GPU parity on seeded random shapes, byte for byte against the CPU oracle:
the entry points whose kernels choose paths by shape (one-tile or four-tile
dual layout, full or ragged row tiles, two-phase or one-pass quantize). Each
case prints its shape before it runs.
"""
import numpy as np
import pytest
import torch

from helpers import bits_u16, bits_u8

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn
RNG = np.random.default_rng(20261201)
DUAL_SHAPES = [(32 * int(RNG.integers(1, 40)), 32 * int(RNG.integers(1, 40))) for _ in range(10)] + \
              [(64 * int(RNG.integers(1, 20)), 256 * int(RNG.integers(1, 6))) for _ in range(6)]
ROWCOL_SHAPES = [(int(RNG.integers(1, 700)), 32 * int(RNG.integers(1, 50))) for _ in range(10)]
MSPLIT_CASES = [([int(v) for v in RNG.integers(0, 400, size=int(RNG.integers(1, 12)))], 128 * int(RNG.integers(1, 8)))
                for _ in range(8)]
QUANT_SHAPES = [(int(RNG.integers(1, 3000)), 32 * int(RNG.integers(1, 300))) for _ in range(8)]
# row counts whole (multiple of 128) and ragged, N a multiple of 256 (the 256-column tiles)
RNG_W = np.random.default_rng(20261202)
ROWCOL_WIDE_SHAPES = [(int(v), 256 * int(RNG_W.integers(1, 12))) for v in
                      list(128 * RNG_W.integers(1, 12, size=3)) + list(RNG_W.integers(1, 1500, size=5))]
MSPLIT_WIDE_CASES = [([int(v) for v in RNG_W.integers(0, 700, size=int(RNG_W.integers(1, 10)))],
                      256 * int(RNG_W.integers(1, 8))) for _ in range(5)]


def _say(*a):
    print("[case]", *a, flush=True)


def _x(M, K, seed, std=1.0):
    return (torch.randn((M, K), generator=torch.Generator().manual_seed(seed)) * std).to(torch.bfloat16)


def _payload(M, K, seed):
    import oracle as o
    q, s = o.quant_mxfp4(bits_u16(_x(M, K, seed)).reshape(-1))
    return q.reshape(M, K // 2), s.reshape(M, K // 32)


@pytest.mark.parametrize("M,K", DUAL_SHAPES)
def test_dual_random(oracle, dev, M, K):
    from omo_python_api.mxfp4 import omo_per_token_group_quant_mxfp4_dual
    _say("dual random", M, K)
    x = _x(M, K, M * 7 + K)
    rq, rs, cq, cs = omo_per_token_group_quant_mxfp4_dual(x.to(dev))
    torch.cuda.synchronize()
    xb = bits_u16(x)
    eq, es = oracle.quant_mxfp4(xb.reshape(-1))
    np.testing.assert_array_equal(bits_u8(rq).reshape(-1), eq)
    np.testing.assert_array_equal(bits_u8(rs).reshape(-1), es)
    eqt, est = oracle.quant_mxfp4(np.ascontiguousarray(xb.T).reshape(-1))
    np.testing.assert_array_equal(bits_u8(cq).reshape(-1), eqt)
    np.testing.assert_array_equal(bits_u8(cs).reshape(-1), est)


def test_dual_grouped_random(oracle, dev):
    from omo_python_api.mxfp4 import omo_per_token_group_quant_mxfp4_dual_grouped
    _say("dual grouped random", DUAL_SHAPES)
    xs = [_x(M, K, i) for i, (M, K) in enumerate(DUAL_SHAPES)]
    outs = omo_per_token_group_quant_mxfp4_dual_grouped([x.to(dev) for x in xs])
    torch.cuda.synchronize()
    for x, (rq, rs, cq, cs) in zip(xs, outs):
        xb = bits_u16(x)
        eq, es = oracle.quant_mxfp4(xb.reshape(-1))
        np.testing.assert_array_equal(bits_u8(rq).reshape(-1), eq)
        np.testing.assert_array_equal(bits_u8(rs).reshape(-1), es)
        eqt, est = oracle.quant_mxfp4(np.ascontiguousarray(xb.T).reshape(-1))
        np.testing.assert_array_equal(bits_u8(cq).reshape(-1), eqt)
        np.testing.assert_array_equal(bits_u8(cs).reshape(-1), est)


@pytest.mark.parametrize("M,N", ROWCOL_SHAPES)
def test_row_to_fp8_col_random(oracle, dev, M, N):
    import omo
    _say("row->col random", M, N)
    q, s = _payload(M, N, M + N)
    out = torch.full((N, M), 0xAB, dtype=torch.uint8, device=dev).view(FP8)
    outs = torch.full(((M + 127) // 128, N), float("nan"), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), out, outs, 1e-10)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col(q, s)
    np.testing.assert_array_equal(bits_u8(out), eo)
    np.testing.assert_array_equal(outs.cpu().numpy().view(np.uint32), es.view(np.uint32))


@pytest.mark.parametrize("splits,N", MSPLIT_CASES)
def test_msplit_random(oracle, dev, splits, N):
    import omo
    from omo_python_api.mxfp4_dequant import split_metadata
    M = sum(splits)
    _say("msplit random", splits, N)
    if M == 0:
        pytest.skip("all splits empty")
    q, s = _payload(M, N, M % 1000)
    lens, offs, soffs, max_len, rows, srows = split_metadata(splits, dev)
    out_q = torch.full((M * N,), 0xAB, dtype=torch.uint8, device=dev).view(FP8)
    out_s = torch.full((max(srows, 1), N), float("nan"), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), out_q,
                                                    out_s, lens, offs, soffs, max_len, 1e-10)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col_msplit(q, s, splits)
    np.testing.assert_array_equal(bits_u8(out_q), eo)
    np.testing.assert_array_equal(out_s.cpu().numpy().view(np.uint32)[:srows], es.view(np.uint32))


@pytest.mark.parametrize("M,K", QUANT_SHAPES)
def test_quant_dequant_random(oracle, dev, M, K):
    import omo
    _say("quant/dequant random", M, K)
    x = _x(M, K, M ^ K, std=3.0)
    q = torch.empty((M, K // 2), dtype=torch.uint8, device=dev)
    s = torch.empty((M, K // 32), dtype=torch.uint8, device=dev)
    omo.omo_per_token_group_quant_fp4(x.to(dev), q, s, 32, 1e-10, -6.0, 6.0, False)
    torch.cuda.synchronize()
    xb = bits_u16(x).reshape(-1)
    eq, es = oracle.quant_mxfp4(xb)
    np.testing.assert_array_equal(bits_u8(q).reshape(-1), eq)
    np.testing.assert_array_equal(bits_u8(s).reshape(-1), es)
    if (M * K) % 256 == 0:  # the dequant's codes come in whole 128-byte groups
        y = torch.empty(M * K, dtype=torch.bfloat16, device=dev)
        unused = torch.empty((1, 1), dtype=torch.float32, device=dev)
        omo.omo_per_token_Mxfp4ToBf16_dequant(q.view(-1), s.view(-1), y, unused, 32, 1e-10, -6.0, 6.0, False)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits_u16(y).reshape(-1), oracle.dequant_bf16(eq, es))


@pytest.mark.parametrize("M,N", ROWCOL_WIDE_SHAPES)
def test_row_to_fp8_col_wide_random(oracle, dev, M, N):
    import omo
    _say("row->col wide random", M, N)
    q, s = _payload(M, N, M * 3 + N)
    out = torch.full((N, M), 0xAB, dtype=torch.uint8, device=dev).view(FP8)
    outs = torch.full(((M + 127) // 128, N), float("nan"), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), out, outs, 1e-10)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col(q, s)
    np.testing.assert_array_equal(bits_u8(out), eo)
    np.testing.assert_array_equal(outs.cpu().numpy().view(np.uint32), es.view(np.uint32))


@pytest.mark.parametrize("splits,N", MSPLIT_WIDE_CASES)
def test_msplit_wide_random(oracle, dev, splits, N):
    import omo
    from omo_python_api.mxfp4_dequant import split_metadata
    M = sum(splits)
    _say("msplit wide random", splits, N)
    if M == 0:
        pytest.skip("all splits empty")
    q, s = _payload(M, N, M % 997)
    lens, offs, soffs, max_len, rows, srows = split_metadata(splits, dev)
    out_q = torch.full((M * N,), 0xAB, dtype=torch.uint8, device=dev).view(FP8)
    out_s = torch.full((max(srows, 1), N), float("nan"), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), out_q,
                                                    out_s, lens, offs, soffs, max_len, 1e-10)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col_msplit(q, s, splits)
    np.testing.assert_array_equal(bits_u8(out_q), eo)
    np.testing.assert_array_equal(out_s.cpu().numpy().view(np.uint32)[:srows], es.view(np.uint32))
