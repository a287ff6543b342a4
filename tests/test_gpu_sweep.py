"""Seeded randomized parity sweep: every entry point, bit for bit against the
oracle, on shapes drawn from the families the kernels choose paths by (ragged
and whole tiles, 128- and 256-column bands, one- and four-tile dual layout)
with randomized values (magnitudes 1e-30..1e30 with NaN, inf, zero, subnormal
and largest-finite patterns sprinkled in), scale bytes (uniform, narrow, or
spread within 128-element groups) and eps (1e-10, 0, -1, 1e-3, 3, 1e5 where
the entry point takes it). The seed is fixed, so a failure names a
reproducible case.
"""
import numpy as np
import pytest
import torch

from helpers import bits_u16, bits_u8, from_u16

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn
N_CASES = 484
SPECIALS = np.array([0x7FC0, 0xFFC0, 0x7F81, 0x7F80, 0xFF80, 0x0000, 0x8000, 0x0001, 0x807F, 0x7F7F, 0xFF7F, 0x0080],
                    np.uint16)
EPS = [1e-10, 0.0, -1.0, 1e-3, 3.0, 1e5]


def _eq(got, want, what):
    got, want = np.asarray(got), np.asarray(want)
    if not np.array_equal(got, want):
        idx = np.argwhere(got != want)[:5].tolist()
        raise AssertionError(f"{what}: first mismatches at {idx}")


def _scales_bits(t):
    return t.cpu().numpy().view(np.uint32)


class Sweep:
    def __init__(self, oracle, dev, seed):
        import omo
        self.o, self.dev, self.omo = oracle, dev, omo
        self.rng = np.random.default_rng(seed)

    # ---- inputs
    def bf16_values(self, n):
        r = self.rng
        x = np.clip((r.standard_normal(n) * 10.0 ** r.uniform(-30, 30)).astype(np.float32), -3e38, 3e38)
        b = (x.view(np.uint32) >> 16).astype(np.uint16)
        if r.random() < 0.5:
            k = r.random(n) < r.choice([1e-4, 1e-3, 1e-2])
            b[k] = r.choice(SPECIALS, k.sum())
        return b

    def codes_scales(self, M, Kb):
        """codes [M, Kb] and scales [M, Kb/16]."""
        r = self.rng
        q = r.integers(0, 256, (M, Kb), dtype=np.uint8)
        mode = int(r.integers(0, 3))
        if mode == 2 and Kb % 64:
            mode = 1
        if mode == 0:
            s = r.integers(0, 256, (M, Kb // 16), dtype=np.uint8)
        elif mode == 1:
            s = np.clip(int(r.integers(100, 150)) + r.integers(-8, 9, (M, Kb // 16)), 0, 255).astype(np.uint8)
        else:
            base = r.integers(0, 256, (M, Kb // 64, 1))
            s = np.clip(base + r.integers(-20, 1, (M, Kb // 64, 4)), 0, 255).astype(np.uint8).reshape(M, Kb // 16)
        return q, s

    def t(self, a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(self.dev)

    # ---- cases
    def quant(self):
        r, o, dev = self.rng, self.o, self.dev
        M, K = int(r.integers(1, 3000)), 32 * int(r.integers(1, 300))
        M = max(1, min(M, 4_000_000 // K))
        eps = float(r.choice([1e-10, 0.0, 1e-3, 3.0]))
        x = self.bf16_values(M * K).reshape(M, K)
        q = torch.empty((M, K // 2), dtype=torch.uint8, device=dev)
        s = torch.empty((M, K // 32), dtype=torch.uint8, device=dev)
        self.omo.omo_per_token_group_quant_fp4(from_u16(x, dev), q, s, 32, eps, -6.0, 6.0, False)
        y = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
        if (M * K) % 256 == 0:
            self.omo.omo_per_token_Mxfp4ToBf16_dequant(q, s, y, torch.empty((1, 1), device=dev), 32, 1e-10, -6.0, 6.0,
                                                       False)
        torch.cuda.synchronize()
        eq, es = o.quant_mxfp4(x.reshape(-1), eps=eps)
        _eq(bits_u8(q).reshape(-1), eq, "quantize codes")
        _eq(bits_u8(s).reshape(-1), es, "quantize scales")
        if (M * K) % 256 == 0:
            _eq(bits_u16(y).reshape(-1), o.dequant_bf16(eq, es), "dequant of the codes")
        return f"quantize {M}x{K} eps {eps}"

    def fp8_rows(self):
        r = self.rng
        M, Kb = int(r.integers(1, 600)), 64 * int(r.integers(1, 60))
        M += (M * Kb) % 128 != 0
        q, s = self.codes_scales(M, Kb)
        out = torch.empty((M, 2 * Kb), dtype=FP8, device=self.dev)
        outs = torch.empty((Kb // 64, M), dtype=torch.float32, device=self.dev)
        self.omo.omo_per_token_Mxfp4ToFp8(self.t(q), self.t(s), out, outs, 128, 1e-10, -6.0, 6.0, False)
        torch.cuda.synchronize()
        eo, es = self.o.mxfp4_to_fp8(q, s)
        _eq(bits_u8(out), eo, "FP8 rows")
        _eq(_scales_bits(outs), es.view(np.uint32), "FP8 row scales")
        return f"FP8 rows {M}x{2 * Kb}"

    def fp8_col(self):
        r = self.rng
        M, Kb = 128 * int(r.integers(1, 6)), 128 * int(r.integers(1, 12))
        eps = float(r.choice(EPS[:5]))
        q, s = self.codes_scales(M, Kb)
        out = torch.empty((2 * Kb, M), dtype=FP8, device=self.dev)
        outs = torch.empty((M // 128, 2 * Kb), dtype=torch.float32, device=self.dev)
        self.omo.omo_per_token_Mxfp4ToFp8_col(self.t(q), self.t(s), out, outs, 128, eps, -6.0, 6.0, False)
        torch.cuda.synchronize()
        eo, es = self.o.mxfp4_to_fp8_col(q, s, eps=eps)
        _eq(bits_u8(out), eo, "FP8 columns")
        _eq(_scales_bits(outs), es.view(np.uint32), "FP8 column scales")
        return f"FP8 columns {M}x{2 * Kb} eps {eps}"

    def row_to_col(self):
        r = self.rng
        if r.random() < 0.5:
            M, N = int(r.integers(1, 700)), 32 * int(r.integers(1, 50))
        else:
            M, N = int(r.integers(1, 1500)), 256 * int(r.integers(1, 12))
        eps = float(r.choice(EPS))
        q, s = self.codes_scales(M, N // 2)
        out = torch.empty((N, M), dtype=FP8, device=self.dev)
        outs = torch.empty(((M + 127) // 128, N), dtype=torch.float32, device=self.dev)
        self.omo.omo_per_token_Mxfp4RowToBf16ToFp8Col(self.t(q), self.t(s), out, outs, eps)
        torch.cuda.synchronize()
        eo, es = self.o.row_to_fp8_col(q, s, eps=eps)
        _eq(bits_u8(out), eo, "row->col")
        _eq(_scales_bits(outs), es.view(np.uint32), "row->col scales")
        return f"row->col {M}x{N} eps {eps}"

    def msplit(self):
        from omo_python_api.mxfp4_dequant import split_metadata
        r = self.rng
        u = r.random()
        if u < 0.3:  # many splits: two per lane on the flat grid, past 128 the 3-D grid
            splits = [int(v) for v in r.integers(0, 300, size=int(r.integers(60, 141)))]
            N = int(r.choice([128, 256])) * int(r.integers(1, 4))
        elif u < 0.65:
            splits, N = [int(v) for v in r.integers(0, 400, size=int(r.integers(1, 12)))], 128 * int(r.integers(1, 8))
        else:
            splits, N = [int(v) for v in r.integers(0, 700, size=int(r.integers(1, 10)))], 256 * int(r.integers(1, 8))
        eps = float(r.choice(EPS))
        R = sum(splits)
        if R == 0:
            return "per-split, no rows"
        q, s = self.codes_scales(R, N // 2)
        lens, offs, soffs, mx, _, srows = split_metadata(splits, self.dev)
        out = torch.empty(R * N, dtype=FP8, device=self.dev)
        outs = torch.empty((srows, N), dtype=torch.float32, device=self.dev)
        self.omo.omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit(self.t(q), self.t(s), out, outs, lens, offs, soffs, mx,
                                                            eps)
        torch.cuda.synchronize()
        eo, es = self.o.row_to_fp8_col_msplit(q, s, splits, eps=eps)
        _eq(bits_u8(out), eo, "per-split row->col")
        _eq(_scales_bits(outs), es.view(np.uint32), "per-split row->col scales")
        return f"per-split row->col {splits} N {N} eps {eps}"

    def dual(self):
        r = self.rng
        if r.random() < 0.5:
            M, K = 32 * int(r.integers(1, 40)), 32 * int(r.integers(1, 40))
        else:
            M, K = 64 * int(r.integers(1, 20)), 256 * int(r.integers(1, 6))
        eps = float(r.choice([1e-10, 0.0, 1e-3, 3.0]))
        x = self.bf16_values(M * K).reshape(M, K)
        outs = [torch.empty(sh, dtype=torch.uint8, device=self.dev)
                for sh in ((M, K // 2), (M, K // 32), (K, M // 2), (K, M // 32))]
        self.omo.omo_quant_mxfp4_dual(from_u16(x, self.dev), *outs, eps=eps)
        torch.cuda.synchronize()
        rq, rs = self.o.quant_mxfp4(x.reshape(-1), eps=eps)
        cq, cs = self.o.quant_mxfp4(np.ascontiguousarray(x.T).reshape(-1), eps=eps)
        for got, want, name in zip(outs, (rq, rs, cq, cs), ("row codes", "row scales", "column codes", "column scales")):
            _eq(bits_u8(got).reshape(-1), want, "dual layout " + name)
        return f"dual layout {M}x{K} eps {eps}"

    def packed(self):
        r = self.rng
        T, H = int(r.integers(1, 400)), 128 * int(r.integers(1, 60))
        x = self.bf16_values(T * H).reshape(T, H)
        pay = torch.empty((T, 17 * H // 32), dtype=torch.uint8, device=self.dev)
        self.omo.omo_quant_mxfp4_packed(from_u16(x, self.dev), pay)
        f8 = torch.empty((T, H), dtype=FP8, device=self.dev)
        f8s = torch.empty((H // 128, T), dtype=torch.float32, device=self.dev)
        self.omo.omo_packed_Mxfp4ToFp8(pay, f8, f8s)
        torch.cuda.synchronize()
        q, s = self.o.quant_mxfp4(x.reshape(-1))
        q, s = q.reshape(T, H // 2), s.reshape(T, H // 32)
        _eq(bits_u8(pay), np.concatenate([q, s], 1), "payload rows")
        eo, es = self.o.mxfp4_to_fp8(q, s)
        _eq(bits_u8(f8), eo, "payload FP8")
        _eq(_scales_bits(f8s), es.view(np.uint32), "payload FP8 scales")
        return f"payload rows {T}x{H}"

    def permute(self):
        r = self.rng
        T, H, n = int(r.integers(1, 500)), 128 * int(r.integers(1, 40)), int(r.integers(1, 2000))
        q, s = self.codes_scales(T, H // 2)
        src = r.integers(-3, T + 3, n).astype(np.int32)  # outside [0, T): zero rows
        qt, st, srt = self.t(q), self.t(s), self.t(src)
        gq = torch.empty((n, H // 2), dtype=torch.uint8, device=self.dev)
        gs = torch.empty((n, H // 32), dtype=torch.uint8, device=self.dev)
        self.omo.omo_mxfp4_permute_rows(qt, st, srt, gq, gs)
        f8 = torch.empty((n, H), dtype=FP8, device=self.dev)
        f8s = torch.empty((H // 128, n), dtype=torch.float32, device=self.dev)
        self.omo.omo_permute_Mxfp4ToFp8(qt, st, srt, f8, f8s)
        torch.cuda.synchronize()
        inside = (src >= 0) & (src < T)
        wq, ws = np.zeros((n, H // 2), np.uint8), np.zeros((n, H // 32), np.uint8)
        wq[inside], ws[inside] = q[src[inside]], s[src[inside]]
        _eq(bits_u8(gq), wq, "gathered codes")
        _eq(bits_u8(gs), ws, "gathered scales")
        eo, es = self.o.mxfp4_to_fp8(wq, ws)
        _eq(bits_u8(f8), eo, "gathered FP8")
        _eq(_scales_bits(f8s), es.view(np.uint32), "gathered FP8 scales")
        return f"permute {T}x{H} -> {n} rows"

    def dequant_raw(self):
        r = self.rng
        n = 128 * int(r.integers(1, 4000))
        q = r.integers(0, 256, n, dtype=np.uint8)
        if r.random() < 0.5:
            s = r.integers(0, 256, n // 16, dtype=np.uint8)
        else:
            s = np.clip(127 + r.integers(-30, 30, n // 16), 0, 255).astype(np.uint8)
        out = torch.empty(2 * n, dtype=torch.bfloat16, device=self.dev)
        self.omo.omo_per_token_Mxfp4ToBf16_dequant(self.t(q), self.t(s), out, torch.empty((1, 1), device=self.dev), 32,
                                                   1e-10, -6.0, 6.0, False)
        torch.cuda.synchronize()
        _eq(bits_u16(out), self.o.dequant_bf16(q, s), "dequant of random bytes")
        return f"dequant {n} code bytes"

    def dual_grouped(self):
        r = self.rng
        shapes = []
        for _ in range(int(r.integers(1, 7))):
            if r.random() < 0.5:
                shapes.append((32 * int(r.integers(0, 20)), 32 * int(r.integers(1, 20))))
            else:
                shapes.append((64 * int(r.integers(1, 10)), 256 * int(r.integers(1, 4))))
        xs = [self.bf16_values(M * K).reshape(M, K) for M, K in shapes]
        outs = [[torch.empty(sh, dtype=torch.uint8, device=self.dev)
                 for sh in ((M, K // 2), (M, K // 32), (K, M // 2), (K, M // 32))] for M, K in shapes]
        self.omo.omo_quant_mxfp4_dual_grouped([from_u16(x, self.dev) for x in xs], outs)
        torch.cuda.synchronize()
        for x, o in zip(xs, outs):
            rq, rs = self.o.quant_mxfp4(x.reshape(-1))
            cq, cs = self.o.quant_mxfp4(np.ascontiguousarray(x.T).reshape(-1))
            for got, want, name in zip(o, (rq, rs, cq, cs), ("row codes", "row scales", "column codes",
                                                             "column scales")):
                _eq(bits_u8(got).reshape(-1), want, "grouped dual layout " + name)
        return f"grouped dual layout {shapes}"

    def payload_dequant(self):
        r = self.rng
        T, H = int(r.integers(1, 400)), 256 * int(r.integers(1, 30))
        q, s = self.codes_scales(T, H // 2)
        pay = self.t(np.concatenate([q, s], 1))
        y = torch.empty((T, H), dtype=torch.bfloat16, device=self.dev)
        self.omo.omo_packed_Mxfp4ToBf16_dequant(pay, y)
        torch.cuda.synchronize()
        _eq(bits_u16(y).reshape(-1), self.o.dequant_bf16(q.reshape(-1), s.reshape(-1)), "payload dequant")
        return f"payload dequant {T}x{H}"


def test_randomized_sweep(oracle, dev):
    sw = Sweep(oracle, dev, seed=20261202)
    cases = [sw.quant, sw.dequant_raw, sw.fp8_rows, sw.fp8_col, sw.row_to_col, sw.msplit, sw.dual, sw.dual_grouped,
             sw.packed, sw.payload_dequant, sw.permute]
    for i in range(N_CASES):
        case = cases[i % len(cases)]
        try:
            desc = case()
        except AssertionError as e:
            raise AssertionError(f"sweep case {i} ({case.__name__}, seed 20261202): {e}") from None
        if i % 44 == 0:
            print("[case]", i, desc, flush=True)
