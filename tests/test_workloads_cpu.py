"""The seeded benchmark inputs (mxfp4-hopper_amd/omo_workloads.py) on the CPU:
the cfg3 weights resolve positions drawn twice to their last draw (the
result of assigning the draws one after another), the same bytes on every
call; the cfg2 activations scale whole channels; the MoE routing counts add
up to tokens x top-k."""
import torch

import omo_workloads as wl


def _heavy_tail_sequential(M, K, seed, std=0.02, frac=0.01):
    g = wl._gen(seed, "cpu")
    w = torch.randn((M, K), generator=g, dtype=torch.float32)
    n = M * K
    k = int(frac * n)
    pos = torch.randint(0, n, (k,), generator=g)
    z = torch.randn((k,), generator=g)
    chi = torch.randn((k, 3), generator=g).pow(2).sum(1)
    t3 = z / torch.sqrt(chi / 3.0)
    flat = w.view(-1).clone()
    for p, v in zip(pos.tolist(), t3.tolist()):
        flat[p] = v
    return (flat.view(M, K) * std).to(torch.bfloat16)


def test_heavy_tail_weights_last_draw_wins():
    M, K, seed = 300, 700, 3
    got = wl.heavy_tail_weights(M, K, seed=seed)
    g = wl._gen(seed, "cpu")
    torch.randn((M, K), generator=g)
    pos = torch.randint(0, M * K, (int(0.01 * M * K),), generator=g)
    assert pos.numel() > pos.unique().numel(), "the case must draw some position twice"
    assert torch.equal(got.view(torch.int16), _heavy_tail_sequential(M, K, seed).view(torch.int16))
    assert torch.equal(got.view(torch.int16), wl.heavy_tail_weights(M, K, seed=seed).view(torch.int16))


def test_activations_with_outliers_scales_whole_channels():
    M, K = 64, 7168
    x = wl.activations_with_outliers(M, K, seed=2026).float()
    big = (x.abs().amax(0) > 20).nonzero().view(-1)
    assert big.numel() == round(0.001 * K)


def test_moe_routing_counts():
    c5 = wl.CFG5
    counts = wl.moe_routing(c5["tokens"], c5["n_experts"], c5["topk"], range(c5["n_experts"]), seed=5)
    assert sum(counts) == c5["tokens"] * c5["topk"]
    assert wl.moe_routing(c5["tokens"], c5["n_experts"], c5["topk"], range(8), seed=5) == counts[:8]
