"""GPU parity at the benchmark configurations' full sizes, byte for byte
against the CPU oracle on the same inputs: the cfg3 dual layout (the
columnwise half equal to the rowwise quantize of the transpose), the cfg5
expert weights in one grouped launch, the cfg5 per-split row->col FP8 over the
routed rows, the dense row->col FP8 at cfg4's shape, and the quantize at the
cfg5 activation shapes (which take the one-pass kernel), and the transposed FP8
requant at cfg4's shape.
"""
import numpy as np
import pytest
import torch

from helpers import bits_u16, bits_u8

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


def _wl():
    import omo_workloads as wl
    return wl


def _check_dual(oracle, xb, rq, rs, cq, cs):
    eq, es = oracle.quant_mxfp4(xb.reshape(-1))
    np.testing.assert_array_equal(bits_u8(rs).reshape(-1), es)
    np.testing.assert_array_equal(bits_u8(rq).reshape(-1), eq)
    eqt, est = oracle.quant_mxfp4(np.ascontiguousarray(xb.T).reshape(-1))
    np.testing.assert_array_equal(bits_u8(cs).reshape(-1), est)
    np.testing.assert_array_equal(bits_u8(cq).reshape(-1), eqt)


def test_dual_cfg3_full(oracle, dev):
    """cfg3: 7168 x 18432 heavy-tailed weights, both layouts in one launch."""
    from omo_python_api.mxfp4 import omo_per_token_group_quant_mxfp4_dual
    _say("dual cfg3 7168x18432")
    x = _wl().heavy_tail_weights(7168, 18432, seed=3, device="cpu")
    rq, rs, cq, cs = omo_per_token_group_quant_mxfp4_dual(x.to(dev))
    torch.cuda.synchronize()
    _check_dual(oracle, bits_u16(x), rq, rs, cq, cs)


def test_dual_grouped_cfg5_weights(oracle, dev):
    """cfg5: gate/up [7168, 2048] and down [2048, 7168] of 8 local experts,
    24 tensors in one grouped launch."""
    from omo_python_api.mxfp4 import omo_per_token_group_quant_mxfp4_dual_grouped
    c5 = _wl().CFG5
    shapes = [(c5["hidden"], c5["ffn"]), (c5["hidden"], c5["ffn"]), (c5["ffn"], c5["hidden"])] * c5["local_experts"]
    _say("dual grouped cfg5 weights", len(shapes))
    xs = [_wl().heavy_tail_weights(M, K, seed=100 + i, device="cpu") for i, (M, K) in enumerate(shapes)]
    outs = omo_per_token_group_quant_mxfp4_dual_grouped([x.to(dev) for x in xs])
    torch.cuda.synchronize()
    for x, (rq, rs, cq, cs) in zip(xs, outs):
        _check_dual(oracle, bits_u16(x), rq, rs, cq, cs)


def test_msplit_cfg5_routed_rows(oracle, dev):
    """cfg5: the 16431 rows routed to experts 0..7 (ragged splits of 1965..2133
    rows), H = 7168, MXFP4 codes from the oracle's quantize of activations."""
    from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4RowToBf16ToFp8Col_msplit_wrapper
    wl = _wl()
    c5 = wl.CFG5
    splits = wl.moe_routing(c5["tokens"], c5["n_experts"], c5["topk"], range(c5["local_experts"]), seed=5)
    R, H = sum(splits), c5["hidden"]
    _say("msplit cfg5", R, H, splits)
    xb = bits_u16(wl.activations_with_outliers(R, H, seed=55, device="cpu")).reshape(-1)
    q, s = oracle.quant_mxfp4(xb)
    q, s = q.reshape(R, H // 2), s.reshape(R, H // 32)
    ys, ss = omo_per_token_mxfp4RowToBf16ToFp8Col_msplit_wrapper(torch.from_numpy(q).to(dev),
                                                                 torch.from_numpy(s).to(dev), splits)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col_msplit(q, s, splits)
    np.testing.assert_array_equal(np.concatenate([bits_u8(y).reshape(-1) for y in ys]), eo)
    np.testing.assert_array_equal(torch.cat(ss).cpu().numpy().view(np.uint32), es.view(np.uint32))


def test_row_to_fp8_col_cfg4_full(oracle, dev):
    """cfg4 shape: 4096 x 7168 rowwise MXFP4 -> FP8 columnwise (dense)."""
    import omo
    wl = _wl()
    M, N = 4096, 7168
    _say("row->col cfg4", M, N)
    xb = bits_u16(wl.activations_with_outliers(M, N, seed=44, device="cpu")).reshape(-1)
    q, s = oracle.quant_mxfp4(xb)
    q, s = q.reshape(M, N // 2), s.reshape(M, N // 32)
    out = torch.empty((N, M), dtype=torch.float8_e4m3fn, device=dev)
    outs = torch.empty((M // 128, N), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), out, outs,
                                             1e-10)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col(q, s)
    np.testing.assert_array_equal(bits_u8(out), eo)
    np.testing.assert_array_equal(outs.cpu().numpy().view(np.uint32), es.view(np.uint32))


@pytest.mark.parametrize("K", [2048, 4096, 7168])
def test_quant_cfg5_activation_shapes(oracle, dev, K):
    """cfg5's activation and gradient quantizes: 16431 rows x {2048, 4096, 7168}."""
    import omo
    R = 16431
    _say("quant cfg5", R, K)
    x = _wl().activations_with_outliers(R, K, seed=K, device="cpu")
    xb = bits_u16(x).reshape(-1)
    q = torch.empty((R, K // 2), dtype=torch.uint8, device=dev)
    s = torch.empty((R, K // 32), dtype=torch.uint8, device=dev)
    omo.omo_per_token_group_quant_fp4(x.to(dev), q, s, 32, 1e-10, -6.0, 6.0, False)
    torch.cuda.synchronize()
    eq, es = oracle.quant_mxfp4(xb)
    np.testing.assert_array_equal(bits_u8(s).reshape(-1), es)
    np.testing.assert_array_equal(bits_u8(q).reshape(-1), eq)


def test_to_fp8_col_cfg4_full(oracle, dev):
    """cfg4 shape: 4096 x 7168 MXFP4 -> FP8 transposed [7168, 4096] with the
    fp32 scale rows."""
    import omo
    wl = _wl()
    M, N = 4096, 7168
    _say("to_fp8_col cfg4", M, N)
    xb = bits_u16(wl.activations_with_outliers(M, N, seed=45, device="cpu")).reshape(-1)
    q, s = oracle.quant_mxfp4(xb)
    q, s = q.reshape(M, N // 2), s.reshape(M, N // 32)
    out = torch.empty((N, M), dtype=torch.float8_e4m3fn, device=dev)
    outs = torch.empty((M // 128, N), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4ToFp8_col(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), out, outs, 128, 1e-10,
                                     -6.0, 6.0, False)
    torch.cuda.synchronize()
    eo, es = oracle.mxfp4_to_fp8_col(q, s, eps=1e-10)
    np.testing.assert_array_equal(bits_u8(out), eo)
    np.testing.assert_array_equal(outs.cpu().numpy().view(np.uint32), es.view(np.uint32))
