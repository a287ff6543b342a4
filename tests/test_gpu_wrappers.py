"""GPU parity of the reference's Python wrappers on the paths the other GPU
tests do not take: the padding branches of the FP8 requant wrappers, the
``ToBf16ToFp8`` and ``_col`` wrappers, and the generic quantize ``warpper``
entry points with their oversized scale buffer.

Each expected value is the oracle applied to exactly what the reference
wrapper hands its kernel (zero-padded codes and scales), then sliced and
split the way the wrapper does (code/kernel/api/mxfp4_dequant.py:15-33,
79-121, 122-187, 189-237; code/kernel/api/mxfp4.py:17-115).
"""
import numpy as np
import pytest
import torch

from helpers import bits_u16, bits_u8

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


def ragged_payload(M, W, seed, spread=16):
    """Random code bytes [M, W] (20% zeros) and E8M0 scale bytes [M, W/16];
    the scales of each run of four blocks (one FP8 group of 128 elements)
    spread over `spread` values below a random base, so the requant's wrap
    cases (zero code with s <= max-7) occur. W need not be a multiple of 64."""
    assert W % 16 == 0
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 256, size=(M, W), dtype=np.uint8)
    q[rng.random((M, W)) < 0.2] = 0
    nb = W // 16
    base = rng.integers(8, 256, size=(M, (nb + 3) // 4))
    s = base.repeat(4, axis=1)[:, :nb] - rng.integers(0, spread, size=(M, nb))
    return q, np.clip(s, 0, 255).astype(np.uint8)


def pad_cols(a, multiple):
    """Zero-pad the last dim to a multiple (the reference's pad_to_multiple)."""
    pad = (-a.shape[1]) % multiple
    return np.pad(a, ((0, 0), (0, pad))) if pad else a


def f32_bits(t):
    return t.detach().cpu().contiguous().numpy().view(np.uint32)


# H = 96, 1056 and 7104 give code rows of 48, 528 and 3552 bytes, none a
# multiple of 64, so the wrapper pads codes to 64, 576 and 3584 bytes and the
# scale rows from 3, 33 and 222 to 4, 36 and 224 columns.
@pytest.mark.parametrize("H,splits,seed", [(96, [5, 0, 60, 1], 1), (1056, [100, 0, 200], 2),
                                          (7104, [37, 219], 3), (7168, [64], 4), (192, [], 5)])
def test_to_fp8_wrapper_padding(oracle, dev, H, splits, seed):
    from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4ToFp8_wrapper
    _say("ToFp8 wrapper padding", H, splits)
    M, W = sum(splits), H // 2
    q, s = ragged_payload(M, W, seed)
    qt, st = torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev)
    xs, ss = omo_per_token_mxfp4ToFp8_wrapper(qt, st, splits)
    torch.cuda.synchronize()
    qp, sp = pad_cols(q, 64), pad_cols(s, 4)
    assert qp.shape[1] // 16 == sp.shape[1]
    Wp = qp.shape[1]
    if M > 0:
        eo, es = oracle.mxfp4_to_fp8(qp, sp)
    else:
        eo, es = np.empty((0, 2 * Wp), np.uint8), np.empty((Wp // 64, 0), np.float32)
    eo = eo[:, :H]
    es = es[:H // 32, :]          # every row: H/32 >= Wp/64 (mxfp4_dequant.py:173)
    assert len(xs) == len(splits) and len(ss) == len(splits)
    o = 0
    for m, x, sc in zip(splits, xs, ss):
        assert x.shape == (m, H) and x.dtype == torch.float8_e4m3fn
        assert sc.shape == (Wp // 64, m) and sc.dtype == torch.float32
        np.testing.assert_array_equal(bits_u8(x), eo[o:o + m])
        np.testing.assert_array_equal(f32_bits(sc), es[:, o:o + m].view(np.uint32))
        o += m
    # the inputs the caller passed are untouched by the padding
    assert np.array_equal(bits_u8(qt), q) and np.array_equal(bits_u8(st), s)


@pytest.mark.parametrize("M,H,seed", [(2, 128, 1), (130, 7168, 2), (64, 1152, 3)])
def test_to_bf16_to_fp8_wrapper(oracle, dev, M, H, seed):
    from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4ToBf16ToFp8_wrapper
    _say("ToBf16ToFp8 wrapper", M, H)
    q, s = ragged_payload(M, H // 2, seed)
    x_q, x_s = omo_per_token_mxfp4ToBf16ToFp8_wrapper(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev))
    torch.cuda.synchronize()
    eo, es = oracle.mxfp4_to_fp8(q, s)
    assert x_q.shape == (M, H) and x_s.shape == (H // 128, M)
    np.testing.assert_array_equal(bits_u8(x_q), eo)
    np.testing.assert_array_equal(f32_bits(x_s), es.view(np.uint32))


@pytest.mark.parametrize("H", [96, 160, 1056])
def test_to_bf16_to_fp8_wrapper_refuses_partial_groups(dev, H):
    """Code rows padded to 16 bytes but not a multiple of 64 leave a partial
    128-element group whose fp32 scale row the wrapper's [2Wp/128, M] buffer
    does not hold; the binding raises instead of launching."""
    from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4ToBf16ToFp8_wrapper
    _say("ToBf16ToFp8 wrapper refusal", H)
    q, s = ragged_payload(4, H // 2, 7)
    with pytest.raises(RuntimeError):
        omo_per_token_mxfp4ToBf16ToFp8_wrapper(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev))
    torch.cuda.synchronize()


# M and the code-row bytes H/2 are multiples of 128 (the tile the reference
# kernel indexes without bounds checks). The wrapper slices the transposed
# output's last dim (M) to 2*W, as the reference does (mxfp4_dequant.py:236),
# which cuts rows when M > H.
@pytest.mark.parametrize("M,H,seed", [(128, 256, 1), (384, 256, 2), (256, 7168, 3)])
def test_to_fp8_col_wrapper(oracle, dev, M, H, seed):
    from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4ToFp8_col_wrapper
    _say("ToFp8_col wrapper", M, H)
    q, s = ragged_payload(M, H // 2, seed, spread=40)
    x_q, x_s = omo_per_token_mxfp4ToFp8_col_wrapper(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev))
    torch.cuda.synchronize()
    eo, es = oracle.mxfp4_to_fp8_col(q, s, eps=1e-10)
    assert x_q.shape == (H, min(M, H)) and x_s.shape == (M // 128, H)
    np.testing.assert_array_equal(bits_u8(x_q), eo[..., :H])
    np.testing.assert_array_equal(f32_bits(x_s), es.view(np.uint32))


@pytest.mark.parametrize("M,H", [(100, 256), (128, 96)])
def test_to_fp8_col_wrapper_refuses_partial_tiles(dev, M, H):
    from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4ToFp8_col_wrapper
    _say("ToFp8_col wrapper refusal", M, H)
    q, s = ragged_payload(M, H // 2, 8)
    with pytest.raises(RuntimeError):
        omo_per_token_mxfp4ToFp8_col_wrapper(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev))
    torch.cuda.synchronize()


SENTINEL = 0xA5


@pytest.mark.parametrize("entry", ["omo_per_token_group_quant_fp4_warpper", "omo_per_token_group_quant_4bit_warpper"])
@pytest.mark.parametrize("M,K,seed", [(1, 32, 1), (33, 7168, 2), (512, 96, 3)])
def test_generic_warpper_oversized_scales(oracle, dev, monkeypatch, entry, M, K, seed):
    """The generic warppers size the scale tensor from the code shape,
    [M, K/2] (mxfp4.py:62-72), 16x what the quantize writes. The kernel fills
    exactly the first M*K/32 bytes in flat block order and leaves the rest:
    the allocation is wrapped to pre-fill a sentinel, which must survive."""
    import omo_python_api.mxfp4 as api
    _say("generic warpper", entry, M, K)
    real = api.create_per_token_group_quant_fp8_output_scale
    made = []

    def prefilled(*a, **kw):
        t = real(*a, **kw)
        t.fill_(SENTINEL)
        made.append(t)
        return t

    monkeypatch.setattr(api, "create_per_token_group_quant_fp8_output_scale", prefilled)
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn((M, K), generator=g) * 3).to(torch.bfloat16)
    xd = x.to(dev)
    fn = getattr(api, entry)
    if entry.endswith("4bit_warpper"):
        x_q, x_s = fn(xd, 32, torch.uint8)
    else:
        x_q, x_s = fn(xd, 32)
    torch.cuda.synchronize()
    assert len(made) == 1 and x_s.data_ptr() == made[0].data_ptr()
    assert x_q.shape == (M, K // 2) and x_s.shape == (M, K // 2) and x_s.dtype == torch.uint8
    eq, es = oracle.quant_mxfp4(bits_u16(x).reshape(-1))
    flat = bits_u8(x_s).reshape(-1)
    np.testing.assert_array_equal(bits_u8(x_q).reshape(-1), eq)
    np.testing.assert_array_equal(flat[:es.size], es)
    assert (flat[es.size:] == SENTINEL).all(), "the quantize wrote past numel/32 scale bytes"
