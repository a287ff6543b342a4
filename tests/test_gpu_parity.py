"""GPU parity: every HIP entry point against the CPU oracle, bit for bit.

Inputs are generated on the host (seeded), copied to the device, run through
the `omo` binding (the C ABI of libomo_mxfp4.so) and compared byte for byte
with oracle/mxfp4_oracle.c on the same bytes.
"""
import numpy as np
import pytest
import torch

from helpers import bits_u16, bits_u8, from_u16

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


def _say(*a):
    print("[case]", *a, flush=True)


def _omo():
    import omo
    return omo


# ----------------------------------------------------------------- inputs
def domain_blocks():
    """Every finite bf16 value v with |v| <= 6*2^c, for every reachable scale
    exponent c in [-33, 126], placed after an anchor element that fixes the
    block's scale to c. Returns (bf16 bits, expected scale bytes)."""
    vals, scales = [], []
    for c in range(-33, 127):
        anchor = 0x7F7F if c == 126 else 0x40C0 + (c << 7)
        mags = np.arange(anchor + 1, dtype=np.uint32)
        v = np.concatenate([mags, mags | 0x8000]).astype(np.uint16)
        nblk = -(-v.size // 31)
        pad = np.zeros(nblk * 31, np.uint16)
        pad[: v.size] = v
        blk = np.empty((nblk, 32), np.uint16)
        blk[:, 0] = anchor
        blk[:, 1:] = pad.reshape(nblk, 31)
        vals.append(blk.reshape(-1))
        scales.append(np.full(nblk, c + 127, np.uint8))
    return np.concatenate(vals), np.concatenate(scales)


def special_blocks():
    """Blocks exercising the reference's special cases."""
    inf, ninf, qnan, snan, nqnan = 0x7F80, 0xFF80, 0x7FC0, 0x7F81, 0xFFC0
    one, six, half = 0x3F80, 0x40C0, 0x3F00
    rows = [
        [0] * 32,                                    # all zero -> scale 94
        [0x8000] * 32,                               # all -0
        [1, 0x8001, 0x007F, 0x807F] + [0] * 28,      # denormals only
        [qnan] + [one] * 31,                         # NaN ignored by amax, NaN -> 0xF
        [snan, nqnan] + [six] * 30,                  # signalling / negative NaN
        [qnan] * 32,                                 # NaN only: amax = eps
        [inf] + [one, 0x8000 | one, 0, 0x8000] * 7 + [one, one, ninf],  # inf: scale 126
        [ninf] * 32,
        [inf, qnan] + [half] * 30,                   # inf and NaN together
        [0x7F7F] + [0x0001] * 31,                    # max finite with denormals
        [0x7F40] + [one] * 31,                       # 1.5*2^127: exact power-of-two quotient
        [0x40C1] + [0x3E80, 0x3F40, 0x3FA0, 0x3FE0, 0x4020, 0x4060, 0x40A0, 0x40B0] * 3 + [0] * 7,
        [0x40C0] + [0x3E80, 0x3F40, 0x3FA0, 0x3FE0, 0x4020, 0x4060, 0x40A0, 0x40B0] * 3 + [0] * 7,
        [0x2F00] * 32,                               # below eps*6: eps dominates
        [0x3040] + [0x2FFF] * 31,                    # 6*2^-33 anchor
        [0x40C8, snan] + [one] * 30,                 # sNaN after the max, same 8-element group
        [one] * 5 + [0xC0C8, 0xFF81, half] + [one] * 24,
        [0x40C8, qnan, snan, nqnan] + [half] * 28,
    ]
    return np.array(rows, dtype=np.uint16).reshape(-1)


def run_quant(x_bits, dev, eps=1e-10, fmin=-6.0, fmax=6.0, shape=None):
    omo = _omo()
    x = from_u16(x_bits, dev)
    if shape is not None:
        x = x.view(shape)
    M = x.shape[0] if x.dim() > 1 else 1
    q = torch.empty(x.numel() // 2, dtype=torch.uint8, device=dev)
    s = torch.empty((M, x.numel() // 32 // M), dtype=torch.uint8, device=dev)
    omo.omo_per_token_group_quant_fp4(x, q, s, 32, eps, fmin, fmax, False)
    torch.cuda.synchronize()
    return bits_u8(q), bits_u8(s).reshape(-1)


# ----------------------------------------------------------------- quantize
@pytest.mark.parametrize("shape,std,seed", [
    ((1, 32), 1.0, 1), ((3, 64), 1.0, 2), ((128, 256), 3.0, 3), ((257, 7168), 1.0, 4),
    ((64, 1056), 1e-3, 5), ((2, 8192 * 4 + 96), 1e4, 6), ((1000, 96), 1e-30, 7),
])
def test_quant_seeded(oracle, dev, shape, std, seed):
    _say("quant seeded", shape, std, seed)
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(shape, generator=g) * std).to(torch.bfloat16)
    xb = bits_u16(x).reshape(-1)
    q, s = run_quant(xb, dev, shape=shape)
    eq, es = oracle.quant_mxfp4(xb)
    np.testing.assert_array_equal(s, es)
    np.testing.assert_array_equal(q, eq)


def test_quant_special_values(oracle, dev):
    _say("quant specials")
    xb = special_blocks()
    q, s = run_quant(xb, dev)
    eq, es = oracle.quant_mxfp4(xb)
    np.testing.assert_array_equal(s, es)
    np.testing.assert_array_equal(q, eq)
    assert s[0] == 94 and s[6] == 126


def test_quant_full_domain(oracle, dev):
    """All bf16 values under every reachable scale exponent, through the
    production kernel (fast path for every block)."""
    _say("quant full domain")
    xb, exp_s = domain_blocks()
    q, s = run_quant(xb, dev)
    eq, es = oracle.quant_mxfp4(xb)
    np.testing.assert_array_equal(es, exp_s)
    np.testing.assert_array_equal(s, es)
    np.testing.assert_array_equal(q, eq)


@pytest.mark.parametrize("eps,fmin,fmax", [
    (1e-10, -4.0, 4.0), (1e-10, -6.5, 6.5), (0.0, -6.0, 6.0), (1e-3, -6.0, 6.0), (1.0, -6.0, 6.0),
    (-1.0, -6.0, 6.0), (3e-38, -6.0, 6.0), (1e-10, -1.0, 6.0), (1e-10, -6.0, 0.7),
])
def test_quant_parameters(oracle, dev, eps, fmin, fmax):
    _say("quant params", eps, fmin, fmax)
    g = torch.Generator().manual_seed(11)
    x = (torch.randn((64, 512), generator=g) * torch.logspace(-3, 3, 512)).to(torch.bfloat16)
    xb = np.concatenate([bits_u16(x).reshape(-1), special_blocks()])
    q, s = run_quant(xb, dev, eps=eps, fmin=fmin, fmax=fmax)
    eq, es = oracle.quant_mxfp4(xb, eps=eps, fp4_min=fmin, fp4_max=fmax)
    np.testing.assert_array_equal(s, es)
    np.testing.assert_array_equal(q, eq)


def test_quant_cfg2_north_star(oracle, dev):
    """8192 x 7168 activations with outlier channels (the benchmark input),
    quantized and then dequantized back to bf16 on the GPU: codes, scale
    bytes and the round-tripped bf16 bits all equal the oracle's."""
    import omo_workloads as wl
    _say("quant cfg2 8192x7168 + dequant back")
    x = wl.activations_with_outliers(8192, 7168, seed=2026, device="cpu")
    xb = bits_u16(x).reshape(-1)
    q, s = run_quant(xb, dev, shape=(8192, 7168))
    eq, es = oracle.quant_mxfp4(xb)
    np.testing.assert_array_equal(s, es)
    np.testing.assert_array_equal(q, eq)
    # dequant of the GPU's own codes (equal to the oracle's, checked above)
    np.testing.assert_array_equal(run_dequant(q, s, dev), oracle.dequant_bf16(eq, es))


def test_cfg1_round_trip(oracle, dev):
    """cfg1: a seeded 4096 x 4096 N(0,1) bf16 tensor quantized on the GPU
    through the reference wrapper and dequantized back on the GPU through the
    dequant wrapper; every stage bit-exact against the oracle."""
    import omo_workloads as wl
    from omo_python_api.mxfp4 import omo_per_token_group_quant_mxfp4
    from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4ToBf16_dequant_wrapper
    _say("cfg1 4096x4096 quant + dequant round trip")
    x = wl.cfg1_input(device="cpu")
    xb = bits_u16(x).reshape(-1)
    q, s = omo_per_token_group_quant_mxfp4(x.to(dev))
    y = omo_per_token_mxfp4ToBf16_dequant_wrapper(q, s, torch.bfloat16)
    torch.cuda.synchronize()
    assert q.shape == (4096, 2048) and s.shape == (4096, 128) and y.shape == (4096, 4096)
    eq, es = oracle.quant_mxfp4(xb)
    np.testing.assert_array_equal(bits_u8(s).reshape(-1), es)
    np.testing.assert_array_equal(bits_u8(q).reshape(-1), eq)
    ey = oracle.dequant_bf16(eq, es)
    np.testing.assert_array_equal(bits_u16(y).reshape(-1), ey)
    # the round trip is a projection: quantizing its output reproduces it
    q2, s2 = omo_per_token_group_quant_mxfp4(y)
    y2 = omo_per_token_mxfp4ToBf16_dequant_wrapper(q2, s2, torch.bfloat16)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits_u16(y2).reshape(-1), ey)


@pytest.mark.parametrize("case", ["domain_tiled", "partial_last_workgroup", "steps_below_95", "few_partial_steps"])
def test_quant_two_phase_path(oracle, dev, case):
    """Shapes around the two-phase kernel (one LDS round per CU, then 16 B
    stores; taken when a CU's share is one round of at least 6144 chunks
    that fills its 2048-chunk steps to 95% or takes at most four of them).
    On a 256-CU device: every bf16 value under every scale exponent plus
    the special blocks in exactly 2 steps per CU; a share of 7 steps whose
    last workgroup ends early with a scale-byte tail that is not a multiple
    of 16; a share of 8.03 steps, which takes the one-pass kernel; and a
    share of 3.5 steps (2048 x 7168), whose last step is half full. Outputs
    start as a sentinel, so every byte must be written."""
    _say("quant two-phase", case)
    if case == "domain_tiled":
        dom, _ = domain_blocks()
        unit = np.concatenate([dom, special_blocks()])
        xb = np.tile(unit, -(-(1 << 23) // unit.size))[: 1 << 23]
        shape = (xb.size // 2048, 2048)
    elif case == "partial_last_workgroup":
        shape = (5, 5865632)  # 3,666,020 chunks: 255 shares of 14,336 and one of 10,340
        g = torch.Generator().manual_seed(32)
        xb = bits_u16((torch.randn(shape, generator=g) * 1e-3).to(torch.bfloat16)).reshape(-1)
    elif case == "steps_below_95":
        shape = (16431, 2048)
        g = torch.Generator().manual_seed(31)
        xb = bits_u16((torch.randn(shape, generator=g) * 5).to(torch.bfloat16)).reshape(-1)
    else:
        shape = (2048, 7168)
        g = torch.Generator().manual_seed(33)
        xb = bits_u16((torch.randn(shape, generator=g) * 0.3).to(torch.bfloat16)).reshape(-1)
    omo = _omo()
    x = from_u16(xb, dev).view(shape)
    q = torch.full((xb.size // 2,), 0xAB, dtype=torch.uint8, device=dev)
    s = torch.full((shape[0], xb.size // 32 // shape[0]), 0xAB, dtype=torch.uint8, device=dev)
    omo.omo_per_token_group_quant_fp4(x, q, s, 32, 1e-10, -6.0, 6.0, False)
    torch.cuda.synchronize()
    eq, es = oracle.quant_mxfp4(xb)
    np.testing.assert_array_equal(bits_u8(s).reshape(-1), es)
    np.testing.assert_array_equal(bits_u8(q), eq)


def test_quant_wrapper_and_determinism(oracle, dev):
    from omo_python_api.mxfp4 import omo_per_token_group_quant_mxfp4
    _say("quant wrapper")
    x = torch.randn((96, 7168), generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(dev)
    q1, s1 = omo_per_token_group_quant_mxfp4(x)
    q2, s2 = omo_per_token_group_quant_mxfp4(x)
    assert q1.shape == (96, 3584) and s1.shape == (96, 224)
    assert q1.dtype == torch.uint8 and s1.dtype == torch.uint8
    assert torch.equal(q1, q2) and torch.equal(s1, s2)
    eq, es = oracle.quant_mxfp4(bits_u16(x).reshape(-1))
    np.testing.assert_array_equal(bits_u8(q1).reshape(-1), eq)
    np.testing.assert_array_equal(bits_u8(s1).reshape(-1), es)
    q0, s0 = omo_per_token_group_quant_mxfp4(x[:0])
    assert q0.shape == (0, 3584) and s0.shape == (0, 224)


# ------------------------------------------------------------------ dequant
def run_dequant(q, s, dev):
    omo = _omo()
    qt = torch.from_numpy(q).to(dev)
    st = torch.from_numpy(s).to(dev)
    out = torch.empty(q.size * 2, dtype=torch.bfloat16, device=dev)
    unused = torch.empty((1, 1), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4ToBf16_dequant(qt, st, out, unused, 32, 1e-10, -6.0, 6.0, False)
    torch.cuda.synchronize()
    return bits_u16(out).reshape(-1)


def test_dequant_all_bytes_all_scales(oracle, dev):
    _say("dequant 256 bytes x 256 scales")
    q = np.tile(np.arange(256, dtype=np.uint8), 256 * 16)  # each scale covers 16 bytes
    s = np.repeat(np.arange(256, dtype=np.uint8), 256)
    got = run_dequant(q, s, dev)
    np.testing.assert_array_equal(got, oracle.dequant_bf16(q, s))


@pytest.mark.parametrize("M,K,seed", [(4, 128, 1), (4096, 4096, 2), (4096, 7168, 3), (33, 1024, 4)])
def test_dequant_roundtrip_seeded(oracle, dev, M, K, seed):
    _say("dequant seeded", M, K)
    x = torch.randn((M, K), generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)
    q, s = oracle.quant_mxfp4(bits_u16(x).reshape(-1))
    got = run_dequant(q, s, dev)
    np.testing.assert_array_equal(got, oracle.dequant_bf16(q, s))


def test_dequant_wrapper_dtypes(oracle, dev):
    from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4ToBf16_dequant_wrapper
    _say("dequant wrapper")
    x = torch.randn((64, 512), generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    q, s = oracle.quant_mxfp4(bits_u16(x).reshape(-1))
    qt = torch.from_numpy(q).view(64, 256).to(dev)
    st = torch.from_numpy(s).view(64, 16).to(dev)
    ref = oracle.dequant_bf16(q, s)
    y = omo_per_token_mxfp4ToBf16_dequant_wrapper(qt, st, torch.bfloat16)
    assert y.shape == (64, 512) and y.dtype == torch.bfloat16
    np.testing.assert_array_equal(bits_u16(y).reshape(-1), ref)
    y32 = omo_per_token_mxfp4ToBf16_dequant_wrapper(qt, st, torch.float32)
    assert y32.dtype == torch.float32
    assert torch.equal(y32.cpu(), from_u16(ref).view(64, 512).float())


# ---------------------------------------------------------- FP8 requant rows
def scale_spread_payload(M, Kb, seed, spread=16):
    """Random codes with block scales spread wide within each 128-group, so
    the wrap cases (zero code with s <= max-7, max < 6) occur."""
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 256, size=(M, Kb), dtype=np.uint8)
    q[rng.random((M, Kb)) < 0.2] = 0
    base = rng.integers(0, 256, size=(M, Kb // 64, 1))
    s = np.clip(base + rng.integers(-spread, 1, size=(M, Kb // 64, 4)), 0, 255).astype(np.uint8)
    return q, s.reshape(M, Kb // 16)


def run_to_fp8(q, s, dev, fn="omo_per_token_Mxfp4ToFp8"):
    omo = _omo()
    M, Kb = q.shape
    qt = torch.from_numpy(q).to(dev)
    st = torch.from_numpy(np.ascontiguousarray(s)).to(dev)
    out = torch.empty((M, 2 * Kb), dtype=FP8, device=dev)
    outs = torch.empty((Kb // 64, M), dtype=torch.float32, device=dev)
    getattr(omo, fn)(qt, st, out, outs, 128, 1e-10, -6.0, 6.0, False)
    torch.cuda.synchronize()
    return bits_u8(out), outs.cpu().numpy()


@pytest.mark.parametrize("fn", ["omo_per_token_Mxfp4ToFp8", "omo_per_token_Mxfp4ToBf16ToFp8"])
@pytest.mark.parametrize("M,Kb,seed,spread", [(2, 64, 1, 16), (130, 3584, 2, 16), (64, 640, 3, 255), (8, 192, 4, 3)])
def test_to_fp8_rowwise(oracle, dev, fn, M, Kb, seed, spread):
    _say(fn, M, Kb, spread)
    q, s = scale_spread_payload(M, Kb, seed, spread)
    out, outs = run_to_fp8(q, s, dev, fn)
    eo, es = oracle.mxfp4_to_fp8(q, s)
    np.testing.assert_array_equal(out, eo)
    np.testing.assert_array_equal(outs.view(np.uint32), es.view(np.uint32))


def test_to_fp8_rowwise_rejects_reference_invalid_shapes(dev):
    """The reference host checks input.numel() % 128 == 0
    (code/kernel/per_token_Mxfp4ToFp8.cu:259); the binding raises RuntimeError."""
    _say("to_fp8 invalid shapes")
    q, s = scale_spread_payload(7, 192, 1)
    with pytest.raises(RuntimeError):
        run_to_fp8(q, s, dev)


def test_quant_binding_rejects_bad_arguments(dev):
    """Host checks before any launch: group_size zero, a numel that is not a
    multiple of group_size (code/kernel/per_token_quant_mxfp4.cu:396), a group
    size other than 32, and undersized outputs raise; the outputs are untouched."""
    import omo
    _say("quant binding bad arguments")
    x = torch.ones((4, 64), dtype=torch.bfloat16, device=dev)
    q = torch.full((4, 32), 0xAB, dtype=torch.uint8, device=dev)
    s = torch.full((4, 2), 0xCD, dtype=torch.uint8, device=dev)
    with pytest.raises(RuntimeError, match="group_size must be positive"):
        omo.omo_per_token_group_quant_fp4(x, q, s, 0, 1e-10, -6.0, 6.0, False)
    with pytest.raises(RuntimeError):
        omo.omo_per_token_group_quant_fp4(x[:, :40].contiguous(), q, s, 64, 1e-10, -6.0, 6.0, False)
    with pytest.raises((RuntimeError, NotImplementedError)):
        omo.omo_per_token_group_quant_fp4(x, q, s, 64, 1e-10, -6.0, 6.0, False)
    with pytest.raises(RuntimeError):
        omo.omo_per_token_group_quant_fp4(x, q[:2], s, 32, 1e-10, -6.0, 6.0, False)
    torch.cuda.synchronize()
    assert bool((q == 0xAB).all()) and bool((s == 0xCD).all())


def test_to_fp8_rowwise_cfg4(oracle, dev):
    _say("to_fp8 cfg4 4096x7168")
    x = torch.randn((4096, 7168), generator=torch.Generator().manual_seed(44)).to(torch.bfloat16)
    q, s = oracle.quant_mxfp4(bits_u16(x).reshape(-1))
    q = q.reshape(4096, 3584)
    out, outs = run_to_fp8(q, s, dev)
    eo, es = oracle.mxfp4_to_fp8(q, s)
    np.testing.assert_array_equal(out, eo)
    np.testing.assert_array_equal(outs.view(np.uint32), es.view(np.uint32))


def every_gap_payload():
    """Rows 0..119: block 0 of each 128-group holds scale 255, block b > 0
    holds 255 - a with a = n % 256 for the group's n-th such block overall,
    and its 16 code bytes are 16 * ((n // 256) % 16) + 0..15, so every gap
    max(s) - s_i in 0..255 meets every code byte. Rows 120..127 take group
    maxima 0..5 (the wrapped g = max(s) - 6) with gaps up to the maximum.
    Read as (codes [128, 1024], scales [128, 64], pairs seen)."""
    M, Kb = 128, 1024
    q = np.zeros((M, Kb), np.uint8)
    s = np.zeros((M, Kb // 16), np.uint8)
    seen = set()
    n = 0
    for r in range(M):
        for g in range(Kb // 64):
            m = 255 if r < 120 else (r * 16 + g) % 6
            s[r, 4 * g] = m
            q[r, 64 * g:64 * g + 16] = np.arange(16) * 7
            for b in range(1, 4):
                a = n % 256 if r < 120 else n % (m + 1)
                s[r, 4 * g + b] = m - a
                lo = 16 * ((n // 256) % 16)
                q[r, 64 * g + 16 * b:64 * g + 16 * b + 16] = np.arange(lo, lo + 16)
                if r < 120:
                    seen.update((a, int(c)) for c in range(lo, lo + 16))
                n += 1
    return q, s, seen


def test_to_fp8_rowwise_every_gap(oracle, dev):
    """Every (max(s) - s_i, code byte) pair of the fast path (gaps 0..11) and
    the restated path (12..255), and group maxima below 6, against the oracle;
    the plain requant and the gathered one (reversed rows plus padding rows)."""
    _say("to_fp8 rowwise every gap")
    q, s, seen = every_gap_payload()
    assert seen == {(a, c) for a in range(256) for c in range(256)}
    out, outs = run_to_fp8(q, s, dev)
    eo, es = oracle.mxfp4_to_fp8(q, s)
    np.testing.assert_array_equal(out, eo)
    np.testing.assert_array_equal(outs.view(np.uint32), es.view(np.uint32))
    omo = _omo()
    M, Kb = q.shape
    src = np.concatenate([np.arange(M - 1, -1, -1), [-1, M, -5]]).astype(np.int32)
    N = src.size
    gq = np.zeros((N, Kb), np.uint8)
    gs = np.zeros((N, Kb // 16), np.uint8)
    gq[:M], gs[:M] = q[::-1], s[::-1]
    eo2, es2 = oracle.mxfp4_to_fp8(gq, gs)
    o8 = torch.empty((N, 2 * Kb), dtype=FP8, device=dev)
    o8s = torch.empty((Kb // 64, N), dtype=torch.float32, device=dev)
    omo.omo_permute_Mxfp4ToFp8(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev),
                               torch.from_numpy(src).to(dev), o8, o8s)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits_u8(o8), eo2)
    np.testing.assert_array_equal(o8s.cpu().numpy().view(np.uint32), es2.view(np.uint32))


def test_to_fp8_wrapper_split(oracle, dev):
    from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4ToFp8_wrapper
    _say("to_fp8 wrapper with m_splits")
    q, s = scale_spread_payload(300, 3584, 7)
    qt, st = torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev)
    xs, ss = omo_per_token_mxfp4ToFp8_wrapper(qt, st, [100, 0, 200])
    eo, es = oracle.mxfp4_to_fp8(q, s)
    assert [t.shape for t in xs] == [(100, 7168), (0, 7168), (200, 7168)]
    assert [t.shape for t in ss] == [(56, 100), (56, 0), (56, 200)]
    np.testing.assert_array_equal(bits_u8(torch.cat(xs)), eo)
    np.testing.assert_array_equal(torch.cat(ss, 1).cpu().numpy().view(np.uint32), es.view(np.uint32))


# ------------------------------------------------------- FP8 requant columns
@pytest.mark.parametrize("M,Kb,seed,spread,eps", [(128, 128, 1, 16, 1e-10), (256, 3584, 2, 255, 1e-10),
                                                  (384, 256, 3, 8, 200.0)])
def test_to_fp8_col(oracle, dev, M, Kb, seed, spread, eps):
    _say("to_fp8_col", M, Kb, spread, eps)
    omo = _omo()
    q, s = scale_spread_payload(M, Kb, seed, spread)
    qt, st = torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev)
    out = torch.empty((2 * Kb, M), dtype=FP8, device=dev)
    outs = torch.empty((M // 128, 2 * Kb), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4ToFp8_col(qt, st, out, outs, 128, eps, -6.0, 6.0, False)
    torch.cuda.synchronize()
    eo, es = oracle.mxfp4_to_fp8_col(q, s, eps=eps)
    np.testing.assert_array_equal(bits_u8(out), eo)
    np.testing.assert_array_equal(outs.cpu().numpy().view(np.uint32), es.view(np.uint32))


def test_to_fp8_col_every_adjust(oracle, dev):
    """Every (uint8)(g - s_row) value 0..255 meets every code byte. Row 0 of
    each 128-row tile holds scale 255 (so g = 249 with eps = 1e-10); row r > 0
    of tile k, MX column c holds 249 - a with a = (127 k + r - 1 + 37 c) mod 256,
    so the adjust values of tiles 0..3 run through all 256 values. The code
    bytes of a row run through all 256 values over two rows. The test asserts
    the coverage before comparing with the oracle."""
    _say("to_fp8_col every adjust value")
    omo = _omo()
    M, Kb = 512, 128
    r = np.arange(M)
    q = ((r[:, None] * 128 + np.arange(Kb)[None, :]) & 0xFF).astype(np.uint8)
    k, rr = r // 128, r % 128
    c = np.arange(Kb // 16)
    a = (127 * k[:, None] + rr[:, None] - 1 + 37 * c[None, :]) % 256
    s = np.where(rr[:, None] == 0, 255, (249 - a) % 256).astype(np.uint8)
    adj_seen = set()
    for k in range(M // 128):
        blk = s[128 * k:128 * (k + 1)].astype(np.int64)
        g = (blk.max(axis=0) - 6) & 0xFF
        for cc in range(Kb // 16):
            adj_seen.update(((g[cc] - blk[:, cc]) & 0xFF).tolist())
    assert adj_seen == set(range(256))
    qt, st = torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev)
    out = torch.empty((2 * Kb, M), dtype=FP8, device=dev)
    outs = torch.empty((M // 128, 2 * Kb), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4ToFp8_col(qt, st, out, outs, 128, 1e-10, -6.0, 6.0, False)
    torch.cuda.synchronize()
    eo, es = oracle.mxfp4_to_fp8_col(q, s)
    np.testing.assert_array_equal(bits_u8(out), eo)
    np.testing.assert_array_equal(outs.cpu().numpy().view(np.uint32), es.view(np.uint32))


# ------------------------------------------------------- row -> col (dense)
def payload_from_normal(M, K, seed, std=1.0):
    import oracle as o
    x = (torch.randn((M, K), generator=torch.Generator().manual_seed(seed)) * std).to(torch.bfloat16)
    q, s = o.quant_mxfp4(bits_u16(x).reshape(-1))
    return q.reshape(M, K // 2), s.reshape(M, K // 32)


# (128, 128) takes the 256-column tiles with a partial band (128 columns) and
# (1, 64) its ragged form; (256, 256), (512, 7168), (1024, 2048) and (128,
# 768) the whole 256-column tiles; (300, 7168), (129, 4096) and (1000, 2048)
# their ragged form.
@pytest.mark.parametrize("M,N,seed", [(128, 128, 1), (300, 7168, 2), (1, 64, 3), (129, 4096, 4), (1000, 2048, 5),
                                      (256, 256, 6), (512, 7168, 7), (1024, 2048, 8), (128, 768, 9)])
def test_row_to_fp8_col_dense(oracle, dev, M, N, seed):
    _say("row_to_fp8_col", M, N)
    from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4RowToBf16ToFp8Col_wrapper
    q, s = payload_from_normal(M, N, seed)
    out, outs = omo_per_token_mxfp4RowToBf16ToFp8Col_wrapper(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev))
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col(q, s)
    assert out.shape == (N, M) and outs.shape == ((M + 127) // 128, N)
    np.testing.assert_array_equal(bits_u8(out), eo)
    np.testing.assert_array_equal(outs.cpu().numpy().view(np.uint32), es.view(np.uint32))


@pytest.mark.parametrize("M,N", [(1, 256), (17, 512), (300, 512), (4001, 2048), (4000, 7168)])
def test_row_to_fp8_col_dense_ragged_sentinel(oracle, dev, M, N):
    """Row counts that leave the last 128-row tile partial (and output
    columns at any byte alignment for odd M), on the 256-column tiles, into
    outputs pre-filled with a sentinel so that a byte the kernel fails to
    write cannot pass."""
    _say("row_to_fp8_col ragged sentinel", M, N)
    omo = _omo()
    q, s = payload_from_normal(M, N, M + 3)
    out = torch.full((N, M), 0xAB, dtype=torch.uint8, device=dev).view(FP8)
    outs = torch.full(((M + 127) // 128, N), float("nan"), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), out, outs, 1e-10)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col(q, s)
    np.testing.assert_array_equal(bits_u8(out), eo)
    np.testing.assert_array_equal(outs.cpu().numpy().view(np.uint32), es.view(np.uint32))


@pytest.mark.parametrize("M,N,eps", [(256, 512, 1e3), (300, 640, 1e3), (256, 512, 3.0)])
def test_row_to_fp8_col_dense_eps(oracle, dev, M, N, eps):
    """eps above (1e3) or among (3.0) the column maxima: the maximum seeded
    with eps, on whole tiles and ragged ones."""
    _say("row_to_fp8_col eps", M, N, eps)
    omo = _omo()
    q, s = payload_from_normal(M, N, 11)
    out = torch.empty((N, M), dtype=FP8, device=dev)
    outs = torch.empty(((M + 127) // 128, N), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), out, outs, eps)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col(q, s, eps=eps)
    np.testing.assert_array_equal(bits_u8(out), eo)
    np.testing.assert_array_equal(outs.cpu().numpy().view(np.uint32), es.view(np.uint32))


def test_row_to_fp8_col_wide_scales(oracle, dev):
    """Random codes and scale bytes over the full 0..255 range (inf / NaN /
    subnormal dequantized values)."""
    _say("row_to_fp8_col wide scales")
    omo = _omo()
    rng = np.random.default_rng(3)
    M, N = 256, 512
    q = rng.integers(0, 256, size=(M, N // 2), dtype=np.uint8)
    s = rng.integers(0, 256, size=(M, N // 32), dtype=np.uint8)
    out = torch.empty((N, M), dtype=FP8, device=dev)
    outs = torch.empty((2, N), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), out, outs, 1e-10)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col(q, s)
    np.testing.assert_array_equal(bits_u8(out), eo)
    np.testing.assert_array_equal(outs.cpu().numpy().view(np.uint32), es.view(np.uint32))


@pytest.mark.parametrize("N,shift", [(512, 0), (384, 0), (384, 4)])
@pytest.mark.parametrize("eps", [-1.0, -0.0, 1e-10])
def test_row_to_fp8_col_nan_lane_groups(oracle, dev, N, shift, eps):
    """Lanes whose values are all NaN: codes 0 with scale byte 255 (0 * inf)
    over whole 16-row lane groups, so that with eps negative a lane's column
    maximum stays eps (< 0) and the kernels reduce the maxima with fmaxf
    rather than as integers; eps -0.0 keeps -0.0 maxima. N = 512 takes the
    256-column tiles, N = 384 the same with a partial band, and N = 384 with
    codes 4 bytes past a 16 B boundary the 128-column ones."""
    _say("row_to_fp8_col nan lane groups", N, shift, eps)
    omo = _omo()
    rng = np.random.default_rng(N)
    M = 256
    q = rng.integers(0, 256, size=(M, N // 2), dtype=np.uint8)
    s = rng.integers(100, 140, size=(M, N // 32)).astype(np.uint8)
    q[16:32, 0:16] = 0      # rows 16..31, element columns 0..31: codes 0
    s[16:32, 0] = 255       # ... with scale 2^128 (inf): every value NaN
    q[128:256, 32:48] = 0   # a whole tile's rows for element columns 64..95
    s[128:256, 2] = 255
    out = torch.empty((N, M), dtype=FP8, device=dev)
    outs = torch.empty((M // 128, N), dtype=torch.float32, device=dev)
    qd = _misaligned(dev, q, shift) if shift else torch.from_numpy(q).to(dev)
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col(qd, torch.from_numpy(s).to(dev), out, outs, eps)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col(q, s, eps=eps)
    np.testing.assert_array_equal(bits_u8(out), eo)
    np.testing.assert_array_equal(outs.cpu().numpy().view(np.uint32), es.view(np.uint32))


@pytest.mark.parametrize("lo,hi", [(1, 4), (250, 254), (1, 252), (0, 3)])
def test_row_to_fp8_col_scale_edges(oracle, dev, lo, hi):
    """Scale bytes at the ends of the range: subnormal products (1..4), the
    last bytes before overflow (250..254), and byte 0 (value 0)."""
    _say("row_to_fp8_col scale edges", lo, hi)
    omo = _omo()
    rng = np.random.default_rng(lo * 1000 + hi)
    M, N = 384, 1024
    q = rng.integers(0, 256, size=(M, N // 2), dtype=np.uint8)
    s = rng.integers(lo, hi + 1, size=(M, N // 32)).astype(np.uint8)
    for fn, outs_rows in (("dense", (M + 127) // 128), ("msplit", None)):
        if fn == "dense":
            out = torch.empty((N, M), dtype=FP8, device=dev)
            outs = torch.empty((outs_rows, N), dtype=torch.float32, device=dev)
            omo.omo_per_token_Mxfp4RowToBf16ToFp8Col(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), out,
                                                     outs, 1e-10)
            torch.cuda.synchronize()
            eo, es = oracle.row_to_fp8_col(q, s)
            np.testing.assert_array_equal(bits_u8(out), eo)
            np.testing.assert_array_equal(outs.cpu().numpy().view(np.uint32), es.view(np.uint32))
        else:
            from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4RowToBf16ToFp8Col_msplit_wrapper
            splits = [100, 284]
            ys, ss = omo_per_token_mxfp4RowToBf16ToFp8Col_msplit_wrapper(torch.from_numpy(q).to(dev),
                                                                         torch.from_numpy(s).to(dev), splits)
            torch.cuda.synchronize()
            eo, es = oracle.row_to_fp8_col_msplit(q, s, splits)
            np.testing.assert_array_equal(np.concatenate([bits_u8(y).reshape(-1) for y in ys]), eo)
            np.testing.assert_array_equal(torch.cat(ss).cpu().numpy().view(np.uint32), es.view(np.uint32))


# ------------------------------------------------------- row -> col (msplit)
@pytest.mark.parametrize("splits,N", [([1, 127, 128, 300], 256), ([0, 5, 0, 2048, 129], 7168), ([128], 128),
                                      ([2000, 1800, 2300, 2100], 2048)])
def test_row_to_fp8_col_msplit(oracle, dev, splits, N):
    _say("msplit", splits, N)
    from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4RowToBf16ToFp8Col_msplit_wrapper
    M = sum(splits)
    q, s = payload_from_normal(M, N, sum(splits) % 97)
    ys, ss = omo_per_token_mxfp4RowToBf16ToFp8Col_msplit_wrapper(torch.from_numpy(q).to(dev),
                                                                 torch.from_numpy(s).to(dev), splits)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col_msplit(q, s, splits)
    off, soff = 0, 0
    for i, m in enumerate(splits):
        assert ys[i].shape == (N, m)
        assert ss[i].shape == ((m + 127) // 128, N)
        np.testing.assert_array_equal(bits_u8(ys[i]).reshape(-1), eo[off * N:(off + m) * N])
        nb = (m + 127) // 128
        np.testing.assert_array_equal(ss[i].cpu().numpy().view(np.uint32), es[soff:soff + nb].view(np.uint32))
        off += m
        soff += nb


# Lengths 17i (i = 1..15) end a tile's column piece after every count 1..15
# of bytes of a 16-row block, on whole 256-column bands (N = 256) and with a
# partial last band (N = 384). Lengths that are multiples of 128 among ragged
# ones (N = 512) mix line-aligned tiles (non-temporal stores) with the others.
@pytest.mark.parametrize("splits,N", [([211, 97, 300, 5, 256, 130], 7168), ([2083, 17, 1965], 1024),
                                      ([129, 255, 383, 1, 16, 144], 384), ([17 * i for i in range(1, 16)], 256),
                                      ([17 * i for i in range(1, 16)], 384), ([256, 100, 128, 0, 384, 17, 640], 512)])
def test_row_to_fp8_col_msplit_every_byte(oracle, dev, splits, N):
    """Ragged splits (column runs at every byte alignment, pieces that end
    inside a 16 B block) into outputs pre-filled with a sentinel, so a byte
    the kernel fails to write cannot pass by holding an earlier result."""
    import omo
    from omo_python_api.mxfp4_dequant import split_metadata
    _say("msplit every byte", splits, N)
    M = sum(splits)
    q, s = payload_from_normal(M, N, M % 89)
    lens, offs, soffs, max_len, rows, srows = split_metadata(splits, dev)
    out_q = torch.full((M * N,), 0xAB, dtype=torch.uint8, device=dev).view(FP8)
    out_s = torch.full((srows, N), float("nan"), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), out_q,
                                                    out_s, lens, offs, soffs, max_len, 1e-10)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col_msplit(q, s, splits)
    np.testing.assert_array_equal(bits_u8(out_q), eo)
    np.testing.assert_array_equal(out_s.cpu().numpy().view(np.uint32), es.view(np.uint32))


def _msplit_sentinel_run(dev, q, s, splits, N, max_len=None):
    import omo
    from omo_python_api.mxfp4_dequant import split_metadata
    M = sum(splits)
    lens, offs, soffs, ml, rows, srows = split_metadata(splits, dev)
    out_q = torch.full((M * N,), 0xAB, dtype=torch.uint8, device=dev).view(FP8)
    out_s = torch.full((srows, N), float("nan"), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), out_q,
                                                    out_s, lens, offs, soffs, ml if max_len is None else max_len, 1e-10)
    torch.cuda.synchronize()
    return bits_u8(out_q), out_s.cpu().numpy().view(np.uint32)


def _misaligned(dev, a, shift):
    """A device copy of a at a byte address `shift` past a 256 B boundary."""
    flat = torch.empty(a.size + 256, dtype=torch.uint8, device=dev)
    v = flat[shift:shift + a.size].view(a.shape)
    v.copy_(torch.from_numpy(a))
    assert v.data_ptr() % 16 == shift % 16
    return v


# Widths that are multiples of 32 but not of 256 take the 256-column tiles
# with a partial last band (N - 256 * (N // 256) columns) and scale rows read
# byte by byte; outputs pre-filled with a sentinel.
@pytest.mark.parametrize("M,N", [(300, 7040), (128, 2880), (1, 96), (257, 160), (512, 1056), (4096, 7040)])
def test_row_to_fp8_col_partial_band(oracle, dev, M, N):
    omo = _omo()
    _say("row_to_fp8_col partial band", M, N)
    q, s = payload_from_normal(M, N, M + N)
    out = torch.full((N, M), 0xAB, dtype=torch.uint8, device=dev).view(FP8)
    outs = torch.full(((M + 127) // 128, N), float("nan"), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), out, outs, 1e-10)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col(q, s)
    np.testing.assert_array_equal(bits_u8(out), eo)
    np.testing.assert_array_equal(outs.cpu().numpy().view(np.uint32), es.view(np.uint32))


@pytest.mark.parametrize("nsplits,N,seed", [(8, 7040, 1), (5, 2880, 2), (3, 160, 3), (100, 2880, 4), (200, 1056, 5),
                                            (1, 96, 6)])
def test_row_to_fp8_col_msplit_partial_band(oracle, dev, nsplits, N, seed):
    """Per split on the 256-column tiles with a partial last band: the flat
    grid at up to 64 splits (band walk) and up to 128, the 3-D grid past 128."""
    rng = np.random.default_rng(seed)
    splits = [int(v) for v in rng.choice([0, 1, 17, 127, 128, 129, 300, 700, 2050], size=nsplits)]
    if sum(splits) == 0:
        splits[-1] = 129
    _say("msplit partial band", nsplits, N, sum(splits))
    q, s = payload_from_normal(sum(splits), N, seed)
    got, got_s = _msplit_sentinel_run(dev, q, s, splits, N)
    eo, es = oracle.row_to_fp8_col_msplit(q, s, splits)
    np.testing.assert_array_equal(got, eo)
    np.testing.assert_array_equal(got_s, es.view(np.uint32))


# Up to 64 splits the flat grid hands rows of at most 16 bands (4096
# columns) out in contiguous ranges and wider ones in band-walk order: both
# sides of that boundary, whole and partial last bands.
@pytest.mark.parametrize("nsplits,N,seed", [(8, 4096, 1), (20, 4128, 2), (8, 4352, 3), (64, 4384, 4), (3, 4064, 5)])
def test_row_to_fp8_col_msplit_order_boundary(oracle, dev, nsplits, N, seed):
    rng = np.random.default_rng(seed)
    splits = [int(v) for v in rng.choice([0, 1, 17, 128, 129, 300, 1100], size=nsplits)]
    if sum(splits) == 0:
        splits[-1] = 129
    _say("msplit order boundary", nsplits, N, sum(splits))
    q, s = payload_from_normal(sum(splits), N, seed)
    got, got_s = _msplit_sentinel_run(dev, q, s, splits, N)
    eo, es = oracle.row_to_fp8_col_msplit(q, s, splits)
    np.testing.assert_array_equal(got, eo)
    np.testing.assert_array_equal(got_s, es.view(np.uint32))


# Widths that are not multiples of 32 (row_bytes = N / 2 any, scales
# [M, ceil(N / 32)]) take the 128-column tiles with byte-wise code loads.
@pytest.mark.parametrize("M,N", [(300, 100), (129, 2050), (1, 2), (256, 7166)])
def test_row_to_fp8_col_odd_width(oracle, dev, M, N):
    omo = _omo()
    _say("row_to_fp8_col odd width", M, N)
    rng = np.random.default_rng(M + N)
    q = rng.integers(0, 256, size=(M, N // 2), dtype=np.uint8)
    s = rng.integers(110, 140, size=(M, (N + 31) // 32)).astype(np.uint8)
    out = torch.full((N, M), 0xAB, dtype=torch.uint8, device=dev).view(FP8)
    outs = torch.full(((M + 127) // 128, N), float("nan"), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), out, outs, 1e-10)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col(q, s)
    np.testing.assert_array_equal(bits_u8(out), eo)
    np.testing.assert_array_equal(outs.cpu().numpy().view(np.uint32), es.view(np.uint32))


@pytest.mark.parametrize("splits,N", [([129, 0, 300, 17], 100), ([5] * 70 + [260], 1026)])
def test_row_to_fp8_col_msplit_odd_width(oracle, dev, splits, N):
    _say("msplit odd width", len(splits), N)
    M = sum(splits)
    rng = np.random.default_rng(M + N)
    q = rng.integers(0, 256, size=(M, N // 2), dtype=np.uint8)
    s = rng.integers(110, 140, size=(M, (N + 31) // 32)).astype(np.uint8)
    got, got_s = _msplit_sentinel_run(dev, q, s, splits, N)
    eo, es = oracle.row_to_fp8_col_msplit(q, s, splits)
    np.testing.assert_array_equal(got, eo)
    np.testing.assert_array_equal(got_s, es.view(np.uint32))


# Code rows at an address that is not 16 B aligned take the 128-column
# kernels (byte-wise code loads); the scales at an odd address too.
@pytest.mark.parametrize("M,N,shift", [(300, 7168, 4), (128, 384, 8), (1, 64, 1), (700, 2048, 12)])
def test_row_to_fp8_col_misaligned_codes(oracle, dev, M, N, shift):
    omo = _omo()
    _say("row_to_fp8_col misaligned codes", M, N, shift)
    q, s = payload_from_normal(M, N, M * 5 + N)
    out = torch.full((N, M), 0xAB, dtype=torch.uint8, device=dev).view(FP8)
    outs = torch.full(((M + 127) // 128, N), float("nan"), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col(_misaligned(dev, q, shift), _misaligned(dev, s, 3), out, outs, 1e-10)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col(q, s)
    np.testing.assert_array_equal(bits_u8(out), eo)
    np.testing.assert_array_equal(outs.cpu().numpy().view(np.uint32), es.view(np.uint32))


@pytest.mark.parametrize("splits,N,shift", [([129, 255, 17], 384, 4), ([5, 300, 128, 0, 1], 7168, 8),
                                            ([1] * 70 + [300], 512, 2)])
def test_row_to_fp8_col_msplit_misaligned_codes(oracle, dev, splits, N, shift):
    import omo
    from omo_python_api.mxfp4_dequant import split_metadata
    _say("msplit misaligned codes", len(splits), N, shift)
    M = sum(splits)
    q, s = payload_from_normal(M, N, M % 61)
    lens, offs, soffs, ml, rows, srows = split_metadata(splits, dev)
    out_q = torch.full((M * N,), 0xAB, dtype=torch.uint8, device=dev).view(FP8)
    out_s = torch.full((srows, N), float("nan"), dtype=torch.float32, device=dev)
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit(_misaligned(dev, q, shift), _misaligned(dev, s, 1), out_q, out_s,
                                                    lens, offs, soffs, ml, 1e-10)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col_msplit(q, s, splits)
    np.testing.assert_array_equal(bits_u8(out_q), eo)
    np.testing.assert_array_equal(out_s.cpu().numpy().view(np.uint32), es.view(np.uint32))


@pytest.mark.parametrize("nsplits,N,seed", [(100, 256, 1), (256, 128, 2), (300, 128, 3), (9, 1056, 4), (5, 96, 5)])
def test_row_to_fp8_col_msplit_many_splits(oracle, dev, nsplits, N, seed):
    """Many splits (the grid's first dimension), N % 128 != 0 (a partial
    column tile), and empty, one-row, whole-tile and ragged splits, into
    sentinel-filled outputs."""
    rng = np.random.default_rng(seed)
    splits = [int(v) for v in rng.choice([0, 1, 17, 128, 129, 200, 255, 256, 300], size=nsplits)]
    _say("msplit many splits", nsplits, N, sum(splits))
    M = sum(splits)
    q, s = payload_from_normal(M, N, seed)
    got, got_s = _msplit_sentinel_run(dev, q, s, splits, N)
    eo, es = oracle.row_to_fp8_col_msplit(q, s, splits)
    np.testing.assert_array_equal(got, eo)
    np.testing.assert_array_equal(got_s, es.view(np.uint32))


@pytest.mark.parametrize("nsplits,seed,N", [(1, 11, 512), (2, 12, 512), (7, 13, 512), (16, 14, 512), (33, 15, 512),
                                            (64, 16, 512), (65, 17, 512), (128, 18, 512), (129, 19, 512),
                                            (256, 20, 512), (16, 21, 384), (100, 22, 384), (129, 23, 384)])
def test_row_to_fp8_col_msplit_uneven_split_counts(oracle, dev, nsplits, seed, N):
    """Split counts on both sides of 64 (one split per lane on the flat grid)
    and of 128 (the flat grid's limit; 129 and 256 take the 3-D grid) with
    very uneven lengths (empty, one-row, ragged and long splits), into
    sentinel-filled outputs: N = 512 (two 256-column bands), N = 384 (a
    whole band and a partial one)."""
    rng = np.random.default_rng(seed)
    splits = [int(v) for v in rng.choice([0, 1, 17, 127, 128, 129, 300, 700, 1500], size=nsplits)]
    if sum(splits) == 0:
        splits[-1] = 129
    _say("msplit uneven split counts", nsplits, sum(splits))
    q, s = payload_from_normal(sum(splits), N, seed)
    got, got_s = _msplit_sentinel_run(dev, q, s, splits, N)
    eo, es = oracle.row_to_fp8_col_msplit(q, s, splits)
    np.testing.assert_array_equal(got, eo)
    np.testing.assert_array_equal(got_s, es.view(np.uint32))


@pytest.mark.parametrize("N,extra,shift", [(512, 0, 0), (512, 66, 0), (512, 260, 0), (384, 0, 0), (384, 0, 4),
                                           (384, 260, 4)])
def test_row_to_fp8_col_msplit_skips_bad_metadata(oracle, dev, N, extra, shift):
    """Split metadata is read on the device, so the kernels skip tiles whose
    rows or scale rows fall outside the buffers: a split running past the
    last row, one whose scale rows start past output_s, and one with a
    negative row offset leave nothing written, and the valid splits around
    them convert normally. Every buffer is a view inside a larger sentinel-
    filled allocation, so a tile that were not skipped would land in the
    padding (checked untouched) instead of outside the allocation. N = 512
    takes the flat grid (extra empty splits: two splits per lane at 66, the
    3-D grid at 260), N = 384 a partial band, and N = 384 with the codes 4
    bytes past a 16 B boundary the 128-column kernel (flat, and 3-D at 260)."""
    import omo
    _say("msplit bad metadata", N, extra, shift)
    valid = [300, 129]
    M = sum(valid)
    srows = sum((m + 127) // 128 for m in valid)
    lens = [300, 200, 129, 128, 64] + [0] * extra
    offs = [0, M - 100, 300, 0, -5] + [0] * extra
    soffs = [0, 0, 3, srows, 0] + [0] * extra
    q, s = payload_from_normal(M, N, 5)
    pad = 256
    big_q = torch.zeros(((M + 2 * pad) * (N // 2) + 16,), dtype=torch.uint8, device=dev)
    big_q = big_q[shift:shift + (M + 2 * pad) * (N // 2)].view(M + 2 * pad, N // 2)
    big_s = torch.full((M + 2 * pad, N // 32), 127, dtype=torch.uint8, device=dev)
    big_q[pad:pad + M] = torch.from_numpy(q).to(dev)
    big_s[pad:pad + M] = torch.from_numpy(s).to(dev)
    big_out = torch.full(((M + 2 * pad) * N,), 0xAB, dtype=torch.uint8, device=dev)
    big_os = torch.full((srows + 2 * 4, N), float("nan"), dtype=torch.float32, device=dev)
    out_q = big_out[pad * N:(pad + M) * N].view(FP8)
    out_s = big_os[4:4 + srows]
    meta = [torch.tensor(v, dtype=torch.int32, device=dev) for v in (lens, offs, soffs)]
    omo.omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit(big_q[pad:pad + M], big_s[pad:pad + M], out_q, out_s, *meta, 300,
                                                    1e-10)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col_msplit(q, s, valid)
    np.testing.assert_array_equal(bits_u8(out_q), eo)
    np.testing.assert_array_equal(out_s.cpu().numpy().view(np.uint32), es.view(np.uint32))
    out_all = bits_u8(big_out)
    assert (out_all[:pad * N] == 0xAB).all() and (out_all[(pad + M) * N:] == 0xAB).all()
    os_all = big_os.cpu().numpy()
    assert np.isnan(os_all[:4]).all() and np.isnan(os_all[4 + srows:]).all()


@pytest.mark.parametrize("N", [256, 1056])
def test_row_to_fp8_col_msplit_short_max_len(oracle, dev, N):
    """The reference launches ceil(max_split_len / 128) row tiles per split
    (code/kernel/per_token_Mxfp4RowToBf16ToFp8Col_msplit.cu:256): with a
    max_split_len below a split's length, that split's rows past those tiles
    and their scale rows are left as they were."""
    splits, max_len = [300, 50, 260, 129], 200
    _say("msplit short max_split_len", splits, N, max_len)
    M = sum(splits)
    q, s = payload_from_normal(M, N, 7)
    got, got_s = _msplit_sentinel_run(dev, q, s, splits, N, max_len)
    eo, es = oracle.row_to_fp8_col_msplit(q, s, splits)
    eo, es = eo.copy(), es.view(np.uint32).copy()
    nan_bits = np.array([np.nan], dtype=np.float32).view(np.uint32)[0]
    tmax = (max_len + 127) // 128
    off, soff = 0, 0
    for m in splits:
        if m > tmax * 128:
            blk = eo[off * N:(off + m) * N].reshape(N, m)
            blk[:, tmax * 128:] = 0xAB
            es[soff + tmax:soff + (m + 127) // 128] = nan_bits
        off += m
        soff += (m + 127) // 128
    np.testing.assert_array_equal(got, eo)
    np.testing.assert_array_equal(got_s, es)


@pytest.mark.parametrize("eps,smax,mixed", [(1e3, 134, False), (1e5, 140, False), (1e3, 140, True)])
def test_row_to_fp8_col_msplit_large_eps(oracle, dev, eps, smax, mixed):
    """A column whose amax does not exceed eps gets multiplier 1 in the
    grouped rule (code/kernel/per_token_Mxfp4RowToBf16ToFp8Col_msplit.cu:23-43),
    so its values above 448 reach the clamp: scale bytes up to smax give
    column maxima up to 6 * 2^(smax - 127), above 448 and at most eps. In the
    mixed case the first half of the scale blocks stays below 135 (clamped
    columns) and the second half reaches 140 (columns with amax > eps)."""
    from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4RowToBf16ToFp8Col_msplit_wrapper
    rng = np.random.default_rng(int(eps))
    splits, N = [300, 129, 64], 512
    M = sum(splits)
    _say("msplit large eps", eps, splits, N)
    q = rng.integers(0, 256, size=(M, N // 2), dtype=np.uint8)
    s = rng.integers(120, smax + 1, size=(M, N // 32)).astype(np.uint8)
    if mixed:
        s[:, : N // 64] = rng.integers(120, 135, size=(M, N // 64)).astype(np.uint8)
    ys, ss = omo_per_token_mxfp4RowToBf16ToFp8Col_msplit_wrapper(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev),
                                                                 splits, eps)
    torch.cuda.synchronize()
    eo, es = oracle.row_to_fp8_col_msplit(q, s, splits, eps=eps)
    assert np.count_nonzero((eo & 0x7F) == 0x7E) > 0  # the clamp to +-448 is exercised
    np.testing.assert_array_equal(np.concatenate([bits_u8(y).reshape(-1) for y in ys]), eo)
    np.testing.assert_array_equal(torch.cat(ss).cpu().numpy().view(np.uint32), es.view(np.uint32))


# ------------------------------------------------------------- dual layout
@pytest.mark.parametrize("M,K,seed", [(32, 32, 1), (64, 7168, 2), (96, 1056, 3), (256, 256, 4)])
def test_dual_layout(oracle, dev, M, K, seed):
    _say("dual", M, K)
    from omo_python_api.mxfp4 import omo_per_token_group_quant_mxfp4_dual
    x = (torch.randn((M, K), generator=torch.Generator().manual_seed(seed)) * 2).to(torch.bfloat16)
    xb = bits_u16(x)
    xb[0, :32] = special_blocks()[32 * 6: 32 * 7]  # an inf block in row 0
    xd = from_u16(xb, dev)
    rq, rs, cq, cs = omo_per_token_group_quant_mxfp4_dual(xd)
    torch.cuda.synchronize()
    eq, es = oracle.quant_mxfp4(xb.reshape(-1))
    np.testing.assert_array_equal(bits_u8(rq).reshape(-1), eq)
    np.testing.assert_array_equal(bits_u8(rs).reshape(-1), es)
    eqt, est = oracle.quant_mxfp4(np.ascontiguousarray(xb.T).reshape(-1))
    np.testing.assert_array_equal(bits_u8(cq).reshape(-1), eqt)
    np.testing.assert_array_equal(bits_u8(cs).reshape(-1), est)


@pytest.mark.parametrize("M,K,seed", [(96, 1056, 5), (192, 7168, 6), (64, 32, 7), (576, 512, 8), (448, 768, 9),
                                      (1024, 256, 10), (320, 7168, 11)])
def test_dual_layout_every_byte_special_columns(oracle, dev, M, K, seed):
    """Special-value blocks placed down columns (inside the second 16-row half
    of a 32-row block, and across two blocks), outputs pre-filled with a
    sentinel so every byte must be written; shapes of several tile rows and
    columns, with and without a ragged 32-row last tile row."""
    import omo
    _say("dual every byte", M, K)
    x = (torch.randn((M, K), generator=torch.Generator().manual_seed(seed)) * 3).to(torch.bfloat16)
    xb = bits_u16(x)
    sb = special_blocks()
    nblk = sb.size // 32
    for i, c in enumerate(range(1, K, 7)):
        blk = sb[32 * (i % nblk): 32 * (i % nblk + 1)]
        if i % 3 == 0:
            xb[16:32, c] = blk[:16]  # half 1 of block 0 only
        elif M >= 64:
            xb[16:48, c] = blk  # straddles blocks 0 and 1
        else:
            xb[0:32, c] = blk
    xd = from_u16(xb, dev)
    fill = lambda *shape: torch.full(shape, 0xAB, dtype=torch.uint8, device=dev)  # noqa: E731
    rq, rs, cq, cs = fill(M, K // 2), fill(M, K // 32), fill(K, M // 2), fill(K, M // 32)
    omo.omo_quant_mxfp4_dual(xd, rq, rs, cq, cs, 1e-10)
    torch.cuda.synchronize()
    eq, es = oracle.quant_mxfp4(xb.reshape(-1))
    np.testing.assert_array_equal(bits_u8(rq).reshape(-1), eq)
    np.testing.assert_array_equal(bits_u8(rs).reshape(-1), es)
    eqt, est = oracle.quant_mxfp4(np.ascontiguousarray(xb.T).reshape(-1))
    np.testing.assert_array_equal(bits_u8(cq).reshape(-1), eqt)
    np.testing.assert_array_equal(bits_u8(cs).reshape(-1), est)


@pytest.mark.parametrize("shapes", [[(64, 256), (96, 1056), (0, 64), (32, 32), (256, 2048)] * 7,
                                    [(64, 256), (576, 768), (0, 256), (320, 512), (256, 2048)] * 7])
def test_dual_layout_grouped(oracle, dev, shapes):
    """One grouped launch over tensors of different shapes (more than one
    32-tensor launch, an empty tensor among them) == the oracle per tensor;
    the second set has only whole 64 x 256 tiles (the four-tile kernel)."""
    from omo_python_api.mxfp4 import omo_per_token_group_quant_mxfp4_dual_grouped
    _say("dual grouped", len(shapes), shapes[:5])
    g = torch.Generator().manual_seed(9)
    xs = [(torch.randn(sh, generator=g) * (1 + i)).to(torch.bfloat16) for i, sh in enumerate(shapes)]
    outs = omo_per_token_group_quant_mxfp4_dual_grouped([x.to(dev) for x in xs])
    torch.cuda.synchronize()
    for x, (rq, rs, cq, cs) in zip(xs, outs):
        if x.numel() == 0:
            continue
        xb = bits_u16(x)
        eq, es = oracle.quant_mxfp4(xb.reshape(-1))
        np.testing.assert_array_equal(bits_u8(rq).reshape(-1), eq)
        np.testing.assert_array_equal(bits_u8(rs).reshape(-1), es)
        eqt, est = oracle.quant_mxfp4(np.ascontiguousarray(xb.T).reshape(-1))
        np.testing.assert_array_equal(bits_u8(cq).reshape(-1), eqt)
        np.testing.assert_array_equal(bits_u8(cs).reshape(-1), est)


# ------------------------------------------------- expert-parallel payload rows
def _payload(codes, scales):
    """Megatron's torch.cat of codes [T, H/2] and scales [T, H/32] (numpy)."""
    T = codes.shape[0]
    return np.ascontiguousarray(np.concatenate([codes.reshape(T, -1), scales.reshape(T, -1)], axis=1))


# 4096 x 7168, 4090 x 7168 (a ragged last workgroup) and 4096 x 2048 take the
# two-phase payload kernel; the others the one-pass row kernel.
@pytest.mark.parametrize("T,H,seed", [(1, 128, 1), (300, 7168, 2), (64, 2048, 3), (5, 128, 0), (0, 7168, 5),
                                      (4096, 7168, 6), (4090, 7168, 7), (4096, 2048, 8), (4096, 2048, 0),
                                      (2048, 7168, 9)])
def test_payload_quant(oracle, dev, T, H, seed):
    """Quantize into payload rows == torch.cat of the unfused quantize outputs."""
    from omo_python_api.ep_payload import fp4_quantize_packed, join_payload
    from omo_python_api.mxfp4 import omo_per_token_group_quant_mxfp4
    _say("payload quant", T, H, seed)
    if seed == 0:  # the special-value blocks (inf, NaN, denormals, ...) padded to whole rows
        sb = special_blocks()
        xb = np.zeros(T * H, np.uint16)
        xb[: sb.size] = sb
        x = from_u16(xb, "cpu").view(T, H)
    else:
        x = (torch.randn((T, H), generator=torch.Generator().manual_seed(seed)) * 3).to(torch.bfloat16)
    xd = x.to(dev)
    p = fp4_quantize_packed(xd)
    q, s = omo_per_token_group_quant_mxfp4(xd)
    torch.cuda.synchronize()
    assert p.shape == (T, H // 2 + H // 32) and p.dtype == torch.uint8
    assert torch.equal(p, join_payload(q, s))
    if T:
        eq, es = oracle.quant_mxfp4(bits_u16(x).reshape(-1))
        np.testing.assert_array_equal(bits_u8(p), _payload(eq.reshape(T, -1), es.reshape(T, -1)))


@pytest.mark.parametrize("T,H,seed,spread", [(2, 128, 1, 16), (300, 7168, 2, 255), (64, 2048, 3, 8), (3, 256, 4, 3)])
def test_payload_dequant_and_requant(oracle, dev, T, H, seed, spread):
    """Dequant and FP8 requant of payload rows == the unfused kernels on the
    unpacked codes and scales (oracle), including m_splits."""
    from omo_python_api.ep_payload import packed_mxfp4ToBf16, packed_mxfp4ToFp8, split_payload
    _say("payload dequant/requant", T, H, seed, spread)
    q, s = scale_spread_payload(T, H // 2, seed, spread)
    p = torch.from_numpy(_payload(q, s)).to(dev)
    dq = packed_mxfp4ToBf16(p)
    splits = [T // 3, 0, T - T // 3]
    f8s, ss = packed_mxfp4ToFp8(p, splits)
    f8, sc = packed_mxfp4ToFp8(p)
    torch.cuda.synchronize()
    uq, us = split_payload(p)
    assert torch.equal(uq.cpu(), torch.from_numpy(q)) and torch.equal(us.cpu(), torch.from_numpy(s))
    np.testing.assert_array_equal(bits_u16(dq).reshape(-1), oracle.dequant_bf16(q, s))
    eo, es = oracle.mxfp4_to_fp8(q, s)
    np.testing.assert_array_equal(bits_u8(f8), eo)
    np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint32), es.view(np.uint32))
    assert [t.shape[0] for t in f8s] == splits and [t.shape[1] for t in ss] == splits
    np.testing.assert_array_equal(bits_u8(torch.cat(f8s)), eo)
    np.testing.assert_array_equal(torch.cat(ss, 1).cpu().numpy().view(np.uint32), es.view(np.uint32))


# ---------------------------------------------------------------- permutation
def test_permute_rows_byte_pieces(dev):
    """H = 96: 3-byte scale rows (and 51-byte payload rows) take the gather's
    byte-wise copy; numpy indexing as the reference, zero padding rows."""
    from omo_python_api.permutation import mxfp4_permute, payload_views
    T, H, E, k, pad = 37, 96, 5, 2, 3
    _say("permute byte pieces", T, H)
    rng = np.random.default_rng(9)
    q = rng.integers(0, 256, size=(T, H // 2), dtype=np.uint8)
    s = rng.integers(100, 150, size=(T, H // 32), dtype=np.uint8)
    rm = np.zeros((T, E), bool)
    for t in range(T):
        rm[t, rng.choice(E, k, replace=False)] = True
    e_idx, t_idx = np.nonzero(rm.T)
    n = t_idx.size
    exp_q = np.zeros((n + pad, H // 2), np.uint8)
    exp_s = np.zeros((n + pad, H // 32), np.uint8)
    exp_q[:n], exp_s[:n] = q[t_idx], s[t_idx]
    rmt = torch.from_numpy(rm).to(dev)
    cq, cs, _, _, _ = mxfp4_permute(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), rmt, None, n + pad)
    payload = torch.from_numpy(np.ascontiguousarray(np.concatenate([q, s], axis=1))).to(dev)
    cq2, cs2, _, _, _ = mxfp4_permute(*payload_views(payload), rmt, None, n + pad)
    torch.cuda.synchronize()
    for a, b in ((cq, exp_q), (cs, exp_s), (cq2, exp_q), (cs2, exp_s)):
        np.testing.assert_array_equal(bits_u8(a), b)


def test_permute_without_source_rows(oracle, dev):
    """Zero source rows (no token routed anywhere, an empty code tensor): every
    output row is a padding row, so the gather writes zero rows and the fused
    requant writes the requant of zero codes and zero scale bytes; neither
    reads the empty inputs."""
    omo = _omo()
    _say("permute with no source rows")
    H, N = 7168, 37
    codes = torch.empty((0, H // 2), dtype=torch.uint8, device=dev)
    scales = torch.empty((0, H // 32), dtype=torch.uint8, device=dev)
    src = torch.full((N,), -1, dtype=torch.int32, device=dev)
    oq = torch.full((N, H // 2), 0xAB, dtype=torch.uint8, device=dev)
    osc = torch.full((N, H // 32), 0xCD, dtype=torch.uint8, device=dev)
    omo.omo_mxfp4_permute_rows(codes, scales, src, oq, osc)
    o8 = torch.empty((N, H), dtype=FP8, device=dev)
    o8s = torch.empty((H // 128, N), dtype=torch.float32, device=dev)
    omo.omo_permute_Mxfp4ToFp8(codes, scales, src, o8, o8s)
    torch.cuda.synchronize()
    assert not bool(oq.any()) and not bool(osc.any())
    eo, es = oracle.mxfp4_to_fp8(np.zeros((N, H // 2), np.uint8), np.zeros((N, H // 32), np.uint8))
    np.testing.assert_array_equal(bits_u8(o8), eo)
    np.testing.assert_array_equal(o8s.cpu().numpy().view(np.uint32), es.view(np.uint32))


@pytest.mark.parametrize("T,H,E,k,pad,seed", [(300, 7168, 8, 2, 0, 1), (64, 256, 4, 1, 7, 2), (5, 128, 3, 3, 0, 3),
                                              (40, 1024, 16, 0, 3, 4)])
def test_permute_rows_and_fp8(oracle, dev, T, H, E, k, pad, seed):
    """Expert-major permutation of MXFP4 rows (numpy indexing as the
    reference) and the fused permutation + FP8 requant (oracle requant of the
    permuted rows, zero padding rows included); also from payload-row views."""
    from omo_python_api.permutation import mxfp4_permute, mxfp4_permute_to_fp8, payload_views
    _say("permute", T, H, E, k, pad, seed)
    rng = np.random.default_rng(seed)
    q, s = scale_spread_payload(T, H // 2, seed, 16)
    rm = np.zeros((T, E), bool)
    for t in range(T):
        rm[t, rng.choice(E, k, replace=False)] = True
    probs = rng.random((T, E)).astype(np.float32)
    e_idx, t_idx = np.nonzero(rm.T)  # expert-major, ascending tokens
    n = t_idx.size
    N = n + pad
    exp_q = np.zeros((N, H // 2), np.uint8)
    exp_s = np.zeros((N, H // 32), np.uint8)
    exp_q[:n], exp_s[:n] = q[t_idx], s[t_idx]
    exp_p = np.zeros(N, np.float32)
    exp_p[:n] = probs[t_idx, e_idx]
    qt, st = torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev)
    rmt = torch.from_numpy(rm).to(dev)
    cq, cs, pp, src, msp = mxfp4_permute(qt, st, rmt, torch.from_numpy(probs).to(dev), N)
    torch.cuda.synchronize()
    assert msp == np.bincount(e_idx, minlength=E).tolist()
    np.testing.assert_array_equal(src.cpu().numpy()[:n], t_idx)
    assert (src.cpu().numpy()[n:] == -1).all()
    np.testing.assert_array_equal(bits_u8(cq), exp_q)
    np.testing.assert_array_equal(bits_u8(cs), exp_s)
    np.testing.assert_array_equal(pp.cpu().numpy(), exp_p)
    eo, es = oracle.mxfp4_to_fp8(exp_q, exp_s)
    f8, f8s, _, _ = mxfp4_permute_to_fp8(qt, st, rmt, N, split=False)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits_u8(f8), eo)
    np.testing.assert_array_equal(f8s.cpu().numpy().view(np.uint32), es.view(np.uint32))
    # split the way omo_per_token_mxfp4ToFp8_wrapper does (padding rows as a trailing split)
    f8l, f8sl, _, _ = mxfp4_permute_to_fp8(qt, st, rmt, N)
    assert [t.shape[0] for t in f8l] == msp + ([pad] if pad else [])
    np.testing.assert_array_equal(bits_u8(torch.cat(f8l)), eo)
    # the same from payload rows [codes | scales], read in place through strided views
    payload = torch.from_numpy(np.ascontiguousarray(np.concatenate([q, s], axis=1))).to(dev)
    vq, vs = payload_views(payload)
    cq2, cs2, _, _, _ = mxfp4_permute(vq, vs, rmt, None, N)
    f82, f8s2, _, _ = mxfp4_permute_to_fp8(vq, vs, rmt, N, split=False)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits_u8(cq2), exp_q)
    np.testing.assert_array_equal(bits_u8(cs2), exp_s)
    np.testing.assert_array_equal(bits_u8(f82), eo)
    np.testing.assert_array_equal(f8s2.cpu().numpy().view(np.uint32), es.view(np.uint32))
