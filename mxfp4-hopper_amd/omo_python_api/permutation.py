"""MXFP4 token permutation for MoE experts.

TE's moe_permute (code/transformer_engine-2.8.diff:220-356) handles an
MXFP4Tensor input by permuting its code rows [T, H/2] and scale rows
[T, H/32] into expert-major order with TE's row permutation kernel, then
wrapping the result in a new MXFP4Tensor; the expert GEMMs then requantize
the permuted rows to FP8 per expert (omo_per_token_mxfp4ToFp8_wrapper with
m_splits). Here:

  * make_row_id_map builds the expert-major order from a routing map: the
    routed (token, expert) pairs sorted by expert, then by token, plus
    padding rows (-1) up to num_out_tokens;
  * mxfp4_permute gathers codes, scales (and probs) in that order;
  * mxfp4_permute_to_fp8 fuses the gather with the FP8 requant (one kernel,
    no permuted MXFP4 copy), equal to mxfp4_permute followed by the requant.

Inputs may be the two halves of expert-parallel payload rows (see
ep_payload.py): strided row views are read in place.
"""
from typing import List, Optional, Tuple

import torch

from omo import omo_mxfp4_permute_rows, omo_permute_Mxfp4ToFp8


def make_row_id_map(routing_map: torch.Tensor, num_out_tokens: Optional[int] = None
                    ) -> Tuple[torch.Tensor, List[int], torch.Tensor]:
    """routing_map [T, E] (bool or 0/1) -> (src_rows int32 [num_out_tokens],
    m_splits (routed tokens per expert), dest int32 [T, E]: the output row of
    each routed (token, expert) pair, -1 where not routed). Output rows are
    ordered by expert, then token; rows past the routed count are padding
    (src_rows = -1)."""
    rm = routing_map.bool()
    T, E = rm.shape
    e_idx, t_idx = torch.nonzero(rm.t(), as_tuple=True)  # expert-major, ascending tokens
    n = t_idx.numel()
    if num_out_tokens is None:
        num_out_tokens = n
    if num_out_tokens < n:
        raise ValueError(f"num_out_tokens={num_out_tokens} is smaller than the {n} routed tokens")
    src = torch.full((num_out_tokens,), -1, dtype=torch.int32, device=rm.device)
    src[:n] = t_idx.to(torch.int32)
    dest = torch.full((T, E), -1, dtype=torch.int32, device=rm.device)
    dest[t_idx, e_idx] = torch.arange(n, dtype=torch.int32, device=rm.device)
    m_splits = torch.bincount(e_idx, minlength=E).tolist()
    return src, m_splits, dest


def _splits_with_padding(m_splits: List[int], num_out: int) -> List[int]:
    pad = num_out - sum(m_splits)
    return list(m_splits) + ([pad] if pad else [])


def mxfp4_permute(codes: torch.Tensor, scales: torch.Tensor, routing_map: torch.Tensor,
                  probs: Optional[torch.Tensor] = None, num_out_tokens: Optional[int] = None):
    """Expert-major permutation of MXFP4 rows. Returns (codes [N, H/2],
    scales [N, H/32], permuted probs [N] or None, src_rows, m_splits); padding
    rows are zero (codes, scales and probs)."""
    src, m_splits, dest = make_row_id_map(routing_map, num_out_tokens)
    N = src.numel()
    out_q = torch.empty((N, codes.size(1)), dtype=torch.uint8, device=codes.device)
    out_s = torch.empty((N, scales.size(1)), dtype=torch.uint8, device=codes.device)
    if N > 0:
        omo_mxfp4_permute_rows(codes, scales, src.to(codes.device), out_q, out_s)
    p = None
    if probs is not None:
        p = torch.zeros((N,), dtype=probs.dtype, device=probs.device)
        routed = dest >= 0
        p[dest[routed].long()] = probs[routed]
    return out_q, out_s, p, src, m_splits


def mxfp4_permute_to_fp8(codes: torch.Tensor, scales: torch.Tensor, routing_map: torch.Tensor,
                         num_out_tokens: Optional[int] = None, split: bool = True):
    """Gather + FP8 E4M3 rowwise requant in one kernel (H % 128 == 0). Returns
    (fp8 [N, H], fp32 scales [H/128, N], src_rows, m_splits); with split=True
    the first two are split by m_splits (plus one trailing split of padding
    rows, if any) the way omo_per_token_mxfp4ToFp8_wrapper splits them."""
    src, m_splits, _ = make_row_id_map(routing_map, num_out_tokens)
    N, H = src.numel(), codes.size(1) * 2
    x_q = torch.empty((N, H), dtype=torch.float8_e4m3fn, device=codes.device)
    x_s = torch.empty((H // 128, N), dtype=torch.float32, device=codes.device)
    if N > 0:
        omo_permute_Mxfp4ToFp8(codes, scales, src.to(codes.device), x_q, x_s)
    if split:
        sp = _splits_with_padding(m_splits, N)
        return torch.split(x_q, sp, dim=0), torch.split(x_s, sp, dim=1), src, m_splits
    return x_q, x_s, src, m_splits


def payload_views(payload: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """The codes and scales halves of payload rows [T, 17H/32] as strided views
    (no copy), for the functions above."""
    width = payload.size(-1)
    if width % 17 != 0:
        raise ValueError(f"payload width {width} is not 17/32 of a hidden size")
    h2 = width // 17 * 16
    return payload[:, :h2], payload[:, h2:]
