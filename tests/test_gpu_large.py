"""GPU parity past 2^31 elements: a bf16 tensor of 264,192 x 8,192 = 2^31 +
2^24 elements (4.3 GB) quantized, requantized to FP8 and dequantized back on
the GPU. Its chunk indices pass 2^28, the FP8 output 2^31 bytes and the bf16
output 2^32 bytes, so every 32-bit index the kernels could have left would
show. The kernels are row-local, so the oracle checks 32-row windows at the
start, across element 2^31 and at the end, and the whole tensor is checked
on the GPU for the value idempotence of dequantize∘quantize.
"""
import numpy as np
import pytest
import torch

from helpers import bits_u16, bits_u8

pytestmark = pytest.mark.gpu

ROWS, K = 2**31 // 8192 + 2048, 8192


def _say(*a):
    print("[case]", *a, flush=True)


def test_quant_requant_dequant_past_2_31(oracle, dev):
    import omo
    numel = ROWS * K
    assert numel == 2**31 + 2**24
    _say("quantize / FP8 requant / dequant", ROWS, K)
    g = torch.Generator(device=dev).manual_seed(2031)
    x = torch.randn((ROWS, K), generator=g, device=dev, dtype=torch.bfloat16)
    q = torch.full((ROWS, K // 2), 0xAB, dtype=torch.uint8, device=dev)
    s = torch.full((ROWS, K // 32), 0xAB, dtype=torch.uint8, device=dev)
    omo.omo_per_token_group_quant_fp4(x, q, s, 32, 1e-10, -6.0, 6.0, False)
    f8 = torch.empty((ROWS, K), dtype=torch.float8_e4m3fn, device=dev)
    f8s = torch.empty((K // 128, ROWS), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4ToFp8(q, s, f8, f8s, 128, 1e-10, -6.0, 6.0, False)
    y = torch.empty((ROWS, K), dtype=torch.bfloat16, device=dev)
    unused = torch.empty((1, 1), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4ToBf16_dequant(q, s, y, unused, 32, 1e-10, -6.0, 6.0, False)
    torch.cuda.synchronize()

    first_past = 2**31 // K  # row holding element 2^31
    for r0 in (0, first_past - 16, ROWS - 32):
        sl = slice(r0, r0 + 32)
        xb = bits_u16(x[sl]).reshape(-1)
        eq, es = oracle.quant_mxfp4(xb)
        np.testing.assert_array_equal(bits_u8(q[sl]).reshape(-1), eq)
        np.testing.assert_array_equal(bits_u8(s[sl]).reshape(-1), es)
        eo, eos = oracle.mxfp4_to_fp8(eq.reshape(32, K // 2), es)
        np.testing.assert_array_equal(bits_u8(f8[sl]), eo)
        np.testing.assert_array_equal(f8s[:, sl].cpu().numpy().view(np.uint32), eos.view(np.uint32))
        np.testing.assert_array_equal(bits_u16(y[sl]).reshape(-1), oracle.dequant_bf16(eq, es))

    # every element: dequantize(quantize(y)) == y for y already on the MXFP4 grid
    q2 = torch.empty_like(q)
    s2 = torch.empty_like(s)
    omo.omo_per_token_group_quant_fp4(y, q2, s2, 32, 1e-10, -6.0, 6.0, False)
    y2 = torch.empty_like(y)
    omo.omo_per_token_Mxfp4ToBf16_dequant(q2, s2, y2, unused, 32, 1e-10, -6.0, 6.0, False)
    torch.cuda.synchronize()
    assert torch.equal(y2.view(torch.int16), y.view(torch.int16))


def _gpu_codes(dev, M, N, seed):
    """MXFP4 codes and scales of a seeded N(0,1) bf16 [M, N] tensor, quantized
    on the GPU (the quantize is checked past 2^31 elements above)."""
    import omo
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn((M, N), generator=g, device=dev, dtype=torch.bfloat16)
    q = torch.empty((M, N // 2), dtype=torch.uint8, device=dev)
    s = torch.empty((M, N // 32), dtype=torch.uint8, device=dev)
    omo.omo_per_token_group_quant_fp4(x, q, s, 32, 1e-10, -6.0, 6.0, False)
    del x
    return q, s


def test_row_to_fp8_col_past_2_31(oracle, dev):
    """Dense row->col FP8 over 300,032 x 7168 codes (2.15e9 elements): the
    output [N, M] passes 2^31 bytes; 128-row tiles at the start, middle and
    end against the oracle on those rows."""
    import omo
    M, N = 300032, 7168
    assert M * N > 2**31
    _say("row->col dense", M, N)
    q, s = _gpu_codes(dev, M, N, 31)
    out = torch.empty((N, M), dtype=torch.float8_e4m3fn, device=dev)
    outs = torch.empty((M // 128, N), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col(q, s, out, outs, 1e-10)
    torch.cuda.synchronize()
    for r0 in (0, M // 256 * 128, M - 128):
        eo, es = oracle.row_to_fp8_col(bits_u8(q[r0:r0 + 128]), bits_u8(s[r0:r0 + 128]))
        np.testing.assert_array_equal(bits_u8(out[:, r0:r0 + 128]), eo)
        np.testing.assert_array_equal(outs[r0 // 128:r0 // 128 + 1].cpu().numpy().view(np.uint32),
                                      es.view(np.uint32))


def test_row_to_fp8_col_msplit_past_2_31(oracle, dev):
    """Per-split row->col FP8 over 8 ragged splits totalling 300,001 rows x
    7168 (2.15e9 elements): the last split's output block ends past 2^31
    bytes; the first and the last split against the oracle."""
    from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4RowToBf16ToFp8Col_msplit_wrapper
    splits = [37463, 37511, 37553, 37429, 37529, 37500, 37487, 37529]
    R, N = sum(splits), 7168
    assert R * N > 2**31 and (R - splits[-1]) * N < 2**31
    _say("row->col msplit", R, N, splits)
    q, s = _gpu_codes(dev, R, N, 32)
    ys, ss = omo_per_token_mxfp4RowToBf16ToFp8Col_msplit_wrapper(q, s, splits)
    torch.cuda.synchronize()
    for i in (0, len(splits) - 1):
        r0 = sum(splits[:i])
        sl = slice(r0, r0 + splits[i])
        eo, es = oracle.row_to_fp8_col_msplit(bits_u8(q[sl]), bits_u8(s[sl]), [splits[i]])
        np.testing.assert_array_equal(bits_u8(ys[i]).reshape(-1), eo)
        np.testing.assert_array_equal(ss[i].cpu().numpy().view(np.uint32), es.view(np.uint32))


def test_dual_past_2_31(oracle, dev):
    """Dual-layout quantize of 16384 x 133120 bf16 (2.18e9 elements, 4.4 GB):
    rowwise outputs of rows at both ends and columnwise outputs of columns at
    both ends against the oracle's quantize of those rows and of those
    columns' transpose."""
    from omo_python_api.mxfp4 import omo_per_token_group_quant_mxfp4_dual
    M, K = 16384, 133120
    assert M * K > 2**31
    _say("dual", M, K)
    g = torch.Generator(device=dev).manual_seed(33)
    x = torch.randn((M, K), generator=g, device=dev, dtype=torch.bfloat16)
    rq, rs, cq, cs = omo_per_token_group_quant_mxfp4_dual(x)
    torch.cuda.synchronize()
    for r0 in (0, M - 32):
        eq, es = oracle.quant_mxfp4(bits_u16(x[r0:r0 + 32]).reshape(-1))
        np.testing.assert_array_equal(bits_u8(rq[r0:r0 + 32]).reshape(-1), eq)
        np.testing.assert_array_equal(bits_u8(rs[r0:r0 + 32]).reshape(-1), es)
    for c0 in (0, K - 256):
        xt = np.ascontiguousarray(bits_u16(x[:, c0:c0 + 256]).T)
        eq, es = oracle.quant_mxfp4(xt.reshape(-1))
        np.testing.assert_array_equal(bits_u8(cq[c0:c0 + 256]).reshape(-1), eq)
        np.testing.assert_array_equal(bits_u8(cs[c0:c0 + 256]).reshape(-1), es)


def _msplit_gpu(dev, q, s, splits):
    import omo
    from omo_python_api.mxfp4_dequant import split_metadata
    R, N = q.size(0), q.size(1) * 2
    lens, offs, soffs, mx, _, srows = split_metadata(splits, dev)
    out = torch.empty(R * N, dtype=torch.float8_e4m3fn, device=dev)
    outs = torch.empty((srows, N), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit(q, s, out, outs, lens, offs, soffs, mx, 1e-10)
    torch.cuda.synchronize()
    return out, outs


@pytest.mark.parametrize("empty_tail", [0, 255])
def test_msplit_more_row_tiles_than_grid_y(oracle, dev, empty_tail):
    """A split of 8,400,037 rows has 65,626 row tiles, past the 65,536 that
    grid y holds: with two splits the flat grid covers them, and with 255
    empty splits appended (257 splits, past the flat grid's 128) the 3-D
    launch is split over row-tile ranges. Row windows at the start, across tile
    65,535 and at the end against the oracle."""
    splits, N = [8_400_037, 300] + [0] * empty_tail, 256
    R = sum(splits)
    _say("msplit long split", splits, N)
    q, s = _gpu_codes(dev, R, N, 34)
    out, outs = _msplit_gpu(dev, q, s, splits)
    ys = out[:splits[0] * N].view(N, splits[0])
    for r0, w in ((0, 256), (65535 * 128 - 256, 512), (65624 * 128, splits[0] - 65624 * 128)):
        eo, es = oracle.row_to_fp8_col_msplit(bits_u8(q[r0:r0 + w]), bits_u8(s[r0:r0 + w]), [w])
        np.testing.assert_array_equal(bits_u8(ys[:, r0:r0 + w]).reshape(-1), eo)
        t0 = r0 // 128
        np.testing.assert_array_equal(outs[t0:t0 + es.shape[0]].cpu().numpy().view(np.uint32), es.view(np.uint32))
    eo, es = oracle.row_to_fp8_col_msplit(bits_u8(q[splits[0]:]), bits_u8(s[splits[0]:]), splits[1:])
    np.testing.assert_array_equal(bits_u8(out[splits[0] * N:]), eo)
    np.testing.assert_array_equal(outs[-es.shape[0]:].cpu().numpy().view(np.uint32), es.view(np.uint32))


@pytest.mark.parametrize("N,empty_tail,shift", [(65536 * 256 + 256, 0, 0), (65536 * 256 + 256, 255, 0),
                                                (65536 * 128 + 128, 0, 4), (65536 * 128 + 128, 125, 4),
                                                (65536 * 128 + 128, 0, 0)])
def test_msplit_more_column_bands_than_grid_z(oracle, dev, N, empty_tail, shift):
    """Rows of 16.8M (256-column bands, the wide kernel: on the flat grid,
    and with 255 empty splits appended on the 3-D grid) or 8.4M columns
    (128-column bands of the general kernel, which codes 4 bytes past a 16 B
    boundary take) have more than the 65,536 column bands grid z holds:
    column windows at the start and across the last band boundaries against
    the oracle on those columns. With 125 empty splits appended (128 splits,
    the flat grid's limit) the 128-column flat grid would need 128 x 65,537
    workgroups of 512 lanes, past the 2^32 - 1 work-items a launch holds
    along x, so the 3-D grid takes it. The same 8.4M columns with aligned
    codes take the 256-column bands with a partial last band."""
    splits = [128, 1, 77] + [0] * empty_tail
    R = sum(splits)
    _say("msplit wide rows", splits, N, shift)
    q, s = _gpu_codes(dev, R, N, 35)
    if shift:
        flat = torch.empty(q.numel() + 16, dtype=torch.uint8, device=dev)
        qm = flat[shift:shift + q.numel()].view(q.shape)
        qm.copy_(q)
        del q
        q = qm
    out, outs = _msplit_gpu(dev, q, s, splits)
    for c0, w in ((0, 256), (N - 768, 768)):
        eo, es = oracle.row_to_fp8_col_msplit(bits_u8(q[:, c0 // 2:(c0 + w) // 2]), bits_u8(s[:, c0 // 32:(c0 + w) // 32]),
                                              splits)
        got, o = [], 0
        for m in splits:
            got.append(bits_u8(out[o * N:(o + m) * N].view(N, m)[c0:c0 + w]).reshape(-1))
            o += m
        np.testing.assert_array_equal(np.concatenate(got), eo)
        np.testing.assert_array_equal(outs[:, c0:c0 + w].cpu().numpy().view(np.uint32), es.view(np.uint32))
