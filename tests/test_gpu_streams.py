"""Every entry point on the caller's stream and inside a captured HIP graph.

The omo binding hands the library torch's current stream, and every kernel
launches on it: work queued ahead of a call on a side stream has finished
before the call reads its inputs, while the default stream stays idle. No
entry point allocates, synchronises or clears memory with a memset, so a
sequence of calls can be captured once and replayed: each replay below, with
new inputs copied in eagerly and the outputs overwritten between replays, is
checked byte for byte against the oracle.
"""
import numpy as np
import pytest
import torch

from helpers import bits_u16, bits_u8

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn
M, K = 640, 1024           # whole 64 x 256 dual tiles, M % 128 == 0 for the transposed requant
M2, K2 = 96, 1056          # ragged dual tiles (the one-tile kernel)
SPLITS = [200, 0, 313, 127]  # per-split row->col over the M rows


def _say(*a):
    print("[case]", *a, flush=True)


def _x(rows, cols, seed):
    return torch.randn((rows, cols), generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)


class _Codec:
    """Static inputs and outputs of one pass over every entry point."""

    def __init__(self, dev):
        from omo_python_api.mxfp4_dequant import split_metadata
        u8, f32 = torch.uint8, torch.float32
        self.x = torch.zeros((M, K), dtype=torch.bfloat16, device=dev)
        self.x2 = torch.zeros((M2, K2), dtype=torch.bfloat16, device=dev)
        self.q = torch.empty((M, K // 2), dtype=u8, device=dev)
        self.s = torch.empty((M, K // 32), dtype=u8, device=dev)
        self.unused = torch.empty((1, 1), dtype=f32, device=dev)
        self.outs = {
            "y": torch.empty((M, K), dtype=torch.bfloat16, device=dev),
            "f8": torch.empty((M, K), dtype=FP8, device=dev), "f8s": torch.empty((K // 128, M), dtype=f32, device=dev),
            "c8": torch.empty((K, M), dtype=FP8, device=dev), "c8s": torch.empty((M // 128, K), dtype=f32, device=dev),
            "rc": torch.empty((K, M), dtype=FP8, device=dev), "rcs": torch.empty((M // 128, K), dtype=f32, device=dev),
            "ms": torch.empty((M * K,), dtype=FP8, device=dev),
            "mss": torch.empty((sum(-(-m // 128) for m in SPLITS), K), dtype=f32, device=dev),
            "dual": [torch.empty(sh, dtype=u8, device=dev) for sh in ((M, K // 2), (M, K // 32), (K, M // 2), (K, M // 32))],
            "dual2": [torch.empty(sh, dtype=u8, device=dev)
                      for sh in ((M2, K2 // 2), (M2, K2 // 32), (K2, M2 // 2), (K2, M2 // 32))],
            "pay": torch.empty((M, 17 * K // 32), dtype=u8, device=dev),
            "py": torch.empty((M, K), dtype=torch.bfloat16, device=dev),
            "p8": torch.empty((M, K), dtype=FP8, device=dev), "p8s": torch.empty((K // 128, M), dtype=f32, device=dev),
        }
        rng = np.random.default_rng(5)
        self.src = rng.integers(-1, M, size=900).astype(np.int32)  # -1: a zero row
        self.src_t = torch.from_numpy(self.src).to(dev)
        n = self.src.size
        self.outs.update({
            "gq": torch.empty((n, K // 2), dtype=u8, device=dev), "gs": torch.empty((n, K // 32), dtype=u8, device=dev),
            "g8": torch.empty((n, K), dtype=FP8, device=dev), "g8s": torch.empty((K // 128, n), dtype=f32, device=dev),
        })
        self.lens, self.offs, self.soffs, self.max_len, _, _ = split_metadata(SPLITS, dev)

    def run(self):
        import omo
        o = self.outs
        omo.omo_per_token_group_quant_fp4(self.x, self.q, self.s, 32, 1e-10, -6.0, 6.0, False)
        omo.omo_per_token_Mxfp4ToBf16_dequant(self.q, self.s, o["y"], self.unused, 32, 1e-10, -6.0, 6.0, False)
        omo.omo_per_token_Mxfp4ToFp8(self.q, self.s, o["f8"], o["f8s"], 128, 1e-10, -6.0, 6.0, False)
        omo.omo_per_token_Mxfp4ToFp8_col(self.q, self.s, o["c8"], o["c8s"], 128, 1e-10, -6.0, 6.0, False)
        omo.omo_per_token_Mxfp4RowToBf16ToFp8Col(self.q, self.s, o["rc"], o["rcs"], 1e-10)
        omo.omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit(self.q, self.s, o["ms"], o["mss"], self.lens, self.offs,
                                                       self.soffs, self.max_len, 1e-10)
        omo.omo_quant_mxfp4_dual(self.x, *o["dual"])
        omo.omo_quant_mxfp4_dual_grouped([self.x2], [o["dual2"]])
        omo.omo_quant_mxfp4_packed(self.x, o["pay"])
        omo.omo_packed_Mxfp4ToBf16_dequant(o["pay"], o["py"])
        omo.omo_packed_Mxfp4ToFp8(o["pay"], o["p8"], o["p8s"])
        omo.omo_mxfp4_permute_rows(self.q, self.s, self.src_t, o["gq"], o["gs"])
        omo.omo_permute_Mxfp4ToFp8(self.q, self.s, self.src_t, o["g8"], o["g8s"])

    def clobber(self):
        for t in (self.q, self.s):
            t.fill_(0xA5)
        for v in self.outs.values():
            for t in (v if isinstance(v, list) else [v]):
                t.view(torch.uint8).fill_(0x5A)

    def check(self, oracle, x, x2):
        o = self.outs
        xb = bits_u16(x)
        eq, es = oracle.quant_mxfp4(xb.reshape(-1))
        q2, s2 = eq.reshape(M, K // 2), es.reshape(M, K // 32)
        np.testing.assert_array_equal(bits_u8(self.q), q2)
        np.testing.assert_array_equal(bits_u8(self.s), s2)
        deq = oracle.dequant_bf16(eq, es)
        np.testing.assert_array_equal(bits_u16(o["y"]).reshape(-1), deq)
        eo, eos = oracle.mxfp4_to_fp8(q2, s2)
        np.testing.assert_array_equal(bits_u8(o["f8"]), eo)
        np.testing.assert_array_equal(o["f8s"].cpu().numpy().view(np.uint32), eos.view(np.uint32))
        co, cos = oracle.mxfp4_to_fp8_col(q2, s2)
        np.testing.assert_array_equal(bits_u8(o["c8"]), co)
        np.testing.assert_array_equal(o["c8s"].cpu().numpy().view(np.uint32), cos.view(np.uint32))
        ro, ros = oracle.row_to_fp8_col(q2, s2)
        np.testing.assert_array_equal(bits_u8(o["rc"]), ro)
        np.testing.assert_array_equal(o["rcs"].cpu().numpy().view(np.uint32), ros.view(np.uint32))
        mo, mos = oracle.row_to_fp8_col_msplit(q2, s2, SPLITS)
        np.testing.assert_array_equal(bits_u8(o["ms"]), mo)
        np.testing.assert_array_equal(o["mss"].cpu().numpy().view(np.uint32), mos.view(np.uint32))
        for xx, outs in ((x, o["dual"]), (x2, o["dual2"])):
            b = bits_u16(xx)
            rq, rs = oracle.quant_mxfp4(b.reshape(-1))
            cq, cs = oracle.quant_mxfp4(np.ascontiguousarray(b.T).reshape(-1))
            for got, exp in zip(outs, (rq, rs, cq, cs)):
                np.testing.assert_array_equal(bits_u8(got).reshape(-1), exp)
        np.testing.assert_array_equal(bits_u8(o["pay"]), np.concatenate([q2, s2], axis=1))
        np.testing.assert_array_equal(bits_u16(o["py"]).reshape(-1), deq)
        np.testing.assert_array_equal(bits_u8(o["p8"]), eo)
        np.testing.assert_array_equal(o["p8s"].cpu().numpy().view(np.uint32), eos.view(np.uint32))
        inside = self.src >= 0
        gq = np.zeros((self.src.size, K // 2), np.uint8)
        gs = np.zeros((self.src.size, K // 32), np.uint8)
        gq[inside], gs[inside] = q2[self.src[inside]], s2[self.src[inside]]
        np.testing.assert_array_equal(bits_u8(o["gq"]), gq)
        np.testing.assert_array_equal(bits_u8(o["gs"]), gs)
        go, gos = oracle.mxfp4_to_fp8(gq, gs)
        np.testing.assert_array_equal(bits_u8(o["g8"]), go)
        np.testing.assert_array_equal(o["g8s"].cpu().numpy().view(np.uint32), gos.view(np.uint32))


def test_entry_points_follow_the_current_stream(oracle, dev):
    """On a side stream held busy by a few milliseconds of matmuls, the inputs
    are copied in and every entry point called: a launch on any other stream
    would read the zeroed inputs before the copy lands."""
    _say("side stream", M, K)
    c = _Codec(dev)
    x, x2 = _x(M, K, 1), _x(M2, K2, 2)
    src, src2 = x.to(dev), x2.to(dev)
    a = torch.randn((4096, 4096), device=dev)
    b = torch.empty_like(a)
    c.clobber()
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(side):
        for _ in range(8):
            torch.mm(a, a, out=b)
        c.x.copy_(src)
        c.x2.copy_(src2)
        c.run()
    side.synchronize()
    c.check(oracle, x, x2)


def test_graph_capture_and_replay(oracle, dev):
    """One capture of every entry point, replayed three times with new inputs
    copied in (and outputs overwritten) eagerly between replays."""
    _say("graph capture", M, K)
    c = _Codec(dev)
    warm = torch.cuda.Stream(device=dev)
    warm.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(warm):
        c.run()
    torch.cuda.current_stream().wait_stream(warm)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        c.run()
    torch.cuda.synchronize()
    for i in range(3):
        _say("replay", i)
        x, x2 = _x(M, K, 10 + i), _x(M2, K2, 20 + i)
        c.x.copy_(x.to(dev))
        c.x2.copy_(x2.to(dev))
        c.clobber()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        c.check(oracle, x, x2)
    del g
