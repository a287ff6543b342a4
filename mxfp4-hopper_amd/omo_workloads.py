"""Seeded synthetic inputs for the benchmark configurations.

Each generator draws with a torch.Generator on the requested device, so the
same (seed, device type) gives the same bytes run to run. The shapes and
distributions are those of the benchmark configurations:
  cfg1  4096 x 4096 N(0,1) bf16 (quantize + dequantize round trip)
  cfg2  8192 x 7168 N(0,1), 0.1% of channels x100 before the bf16 cast
  cfg3  7168 x 18432 0.02*N(0,1), 1% of entries 0.02*Student-t(3)
  cfg4  4096 x 7168 MXFP4 payload quantized from N(0,1) bf16
  cfg5  MoE layer on one GPU: 16384 tokens, hidden 7168, 8 local experts of
        64, FFN 2048, top-8 routing
"""
from __future__ import annotations

import torch


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=torch.device(device))
    g.manual_seed(int(seed))
    return g


def normal_bf16(shape, seed: int, device="cpu", std: float = 1.0) -> torch.Tensor:
    g = _gen(seed, device)
    x = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    if std != 1.0:
        x.mul_(std)
    return x.to(torch.bfloat16)


CFG1_SHAPE = (4096, 4096)
CFG1_SEED = 4096


def cfg1_input(device="cpu") -> torch.Tensor:
    """cfg1: the seeded 4096 x 4096 N(0,1) bf16 tensor of the quantize +
    dequantize round trip."""
    return normal_bf16(CFG1_SHAPE, seed=CFG1_SEED, device=device)


def activations_with_outliers(M: int, K: int, seed: int, device="cpu", frac: float = 0.001,
                              gain: float = 100.0) -> torch.Tensor:
    """cfg2: N(0,1) [M, K] with round(frac*K) seeded channels scaled by gain
    before the bf16 cast."""
    g = _gen(seed, device)
    x = torch.randn((M, K), generator=g, device=device, dtype=torch.float32)
    n_out = max(1, round(frac * K))
    ch = torch.randperm(K, generator=g, device=device)[:n_out]
    x[:, ch] *= gain
    return x.to(torch.bfloat16)


def heavy_tail_weights(M: int, K: int, seed: int, device="cpu", std: float = 0.02,
                       frac: float = 0.01) -> torch.Tensor:
    """cfg3: std*N(0,1) with frac of the entries (seeded positions) replaced by
    std*t3, t3 = Z / sqrt(chi2_3 / 3)."""
    g = _gen(seed, device)
    w = torch.randn((M, K), generator=g, device=device, dtype=torch.float32)
    n = M * K
    k = int(frac * n)
    pos = torch.randint(0, n, (k,), generator=g, device=device)
    z = torch.randn((k,), generator=g, device=device)
    chi = torch.randn((k, 3), generator=g, device=device).pow(2).sum(1)
    t3 = z / torch.sqrt(chi / 3.0)
    # A position drawn more than once takes its last draw, as a sequential
    # assignment would; a device scatter with repeated indices keeps an
    # arbitrary one, so repeats are resolved here (stable sort, last of each run).
    order = torch.argsort(pos, stable=True)
    ps, ts = pos[order], t3[order]
    last = torch.ones_like(ps, dtype=torch.bool)
    last[:-1] = ps[:-1] != ps[1:]
    w = w.view(-1)
    w[ps[last]] = ts[last]
    return (w.view(M, K) * std).to(torch.bfloat16)


def moe_routing(tokens: int, n_experts: int, topk: int, local: range, seed: int):
    """Seeded top-k distinct expert choice per token; returns the number of
    (token, expert) pairs landing on each local expert."""
    g = _gen(seed, "cpu")
    scores = torch.rand((tokens, n_experts), generator=g)
    choice = scores.topk(topk, dim=1).indices
    counts = torch.bincount(choice.view(-1), minlength=n_experts)
    return [int(counts[e]) for e in local]


CFG5 = dict(tokens=16384, hidden=7168, ffn=2048, n_experts=64, local_experts=8, topk=8)


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)


def quant_bytes(numel: int) -> int:
    """Algorithmic HBM bytes of one BF16 -> MXFP4 quantize: 2N read, N/2 + N/32 written."""
    return 2 * numel + numel // 2 + numel // 32


def dequant_bytes(numel: int) -> int:
    """MXFP4 -> BF16: N/2 + N/32 read, 2N written."""
    return numel // 2 + numel // 32 + 2 * numel


def requant_fp8_bytes(numel: int) -> int:
    """MXFP4 -> FP8 with 1x128 fp32 scales: N/2 + N/32 read, N + 4N/128 written."""
    return numel // 2 + numel // 32 + numel + 4 * (numel // 128)


def dual_quant_bytes(numel: int) -> int:
    """Fused rowwise + columnwise quantize: 2N read, 2 x (N/2 + N/32) written."""
    return 2 * numel + 2 * (numel // 2 + numel // 32)


def row_to_col_fp8_bytes(M: int, N: int) -> int:
    """MXFP4 rowwise -> FP8 columnwise: MN/2 + MN/32 read, MN + 4*N*ceil(M/128) written."""
    return M * N // 2 + M * N // 32 + M * N + 4 * N * ceil_div(M, 128)


__all__ = [name for name in dir() if not name.startswith("_") and name != "annotations"]
