"""Expert-parallel MXFP4 payload rows: [codes (H/2 bytes) | E8M0 scales (H/32 bytes)].

Megatron's FP4 dispatch (code/megatron-0.15.0rc7.diff:32-63, 91-124) sends each
token as one row of H/2 code bytes followed by its H/32 scale bytes, 17H/32
bytes in all. Its send side builds those rows by concatenating the quantize
outputs; its receive side cuts them apart again into two contiguous tensors
before the requant or dequant.

``join_payload`` / ``split_payload`` are that unfused composition, kept as the
comparison for the fused path and for callers that hold separate code and
scale tensors. The ``*_packed`` functions are the fused path: the quantize
kernel writes payload rows directly and the dequant / FP8 requant kernels read
them in place, so neither the concatenation nor the two split copies happen.
Their outputs are byte-identical to the unfused composition.
"""
from typing import List, Optional, Tuple

import torch

from omo import omo_packed_Mxfp4ToBf16_dequant, omo_packed_Mxfp4ToFp8, omo_quant_mxfp4_packed


def payload_width(hidden: int) -> int:
    """Bytes per payload row for hidden size H: H/2 + H/32 = 17H/32."""
    return hidden // 2 + hidden // 32


def hidden_of(packed: torch.Tensor) -> int:
    """Hidden size H of payload rows [T, 17H/32] (H a multiple of 32)."""
    if packed.dim() != 2:
        raise ValueError(f"payload must be 2-D [tokens, 17H/32], got {packed.dim()} dims")
    width = packed.size(1)
    if width == 0 or width % 17 != 0:
        raise ValueError(f"payload width {width} is not 17/32 of a hidden size")
    return width // 17 * 32


def join_payload(codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """Payload rows from separate rowwise codes [T, H/2] and scale bytes
    [T, H/32]: one concatenation along the row (the unfused send side)."""
    if codes.dim() != 2 or scales.dim() != 2:
        raise ValueError("codes and scales must both be 2-D [tokens, bytes]")
    if codes.size(0) != scales.size(0):
        raise ValueError(f"codes hold {codes.size(0)} tokens but scales hold {scales.size(0)}")
    if codes.size(1) != 16 * scales.size(1):
        raise ValueError(f"{codes.size(1)} code bytes per token need {codes.size(1) // 16} scale bytes, "
                         f"got {scales.size(1)}")
    return torch.cat((codes, scales), dim=1)


def split_payload(packed: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Contiguous codes [T, H/2] and scale bytes [T, H/32] cut out of payload
    rows (the unfused receive side: two copies)."""
    half = hidden_of(packed) // 2
    return packed[:, :half].contiguous(), packed[:, half:].contiguous()


def fp4_quantize_packed(x: torch.Tensor, eps: float = 1e-10) -> torch.Tensor:
    """Fused ``fp4_quantize`` (megatron-0.15.0rc7.diff:163-170): bf16 [T, H]
    (H % 128 == 0) -> payload [T, 17H/32] uint8, equal to
    join_payload(*omo_per_token_group_quant_mxfp4(x))."""
    assert x.dim() == 2, "`x` must be 2-D [tokens, hidden]"
    assert x.is_contiguous(), "`x` is not contiguous"
    T, H = x.shape
    out = torch.empty((T, payload_width(H)), device=x.device, dtype=torch.uint8)
    if T > 0:
        omo_quant_mxfp4_packed(x, out, eps)
    return out


def packed_mxfp4ToBf16(packed: torch.Tensor, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Payload [T, 17H/32] -> [T, H] in ``dtype``, equal to
    omo_per_token_mxfp4ToBf16_dequant_wrapper(*split_payload(packed), dtype)."""
    assert packed.is_contiguous(), "payload is not contiguous"
    T, H = packed.size(0), hidden_of(packed)
    out = torch.empty((T, H), device=packed.device, dtype=torch.bfloat16)
    if T > 0:
        omo_packed_Mxfp4ToBf16_dequant(packed, out)
    return out.to(dtype)


def packed_mxfp4ToFp8(packed: torch.Tensor, m_splits: Optional[List[int]] = None):
    """Payload [T, 17H/32] -> FP8 E4M3 [T, H] and fp32 scales [H/128, T], split
    by ``m_splits`` along tokens as omo_per_token_mxfp4ToFp8_wrapper does
    (code/kernel/api/mxfp4_dequant.py:172-181); without m_splits the whole
    tensors are returned."""
    assert packed.is_contiguous(), "payload is not contiguous"
    T, H = packed.size(0), hidden_of(packed)
    x_q = torch.empty((T, H), device=packed.device, dtype=torch.float8_e4m3fn)
    x_s = torch.empty((H // 128, T), device=packed.device, dtype=torch.float32)
    if T > 0:
        omo_packed_Mxfp4ToFp8(packed, x_q, x_s)
    if m_splits is None:
        return x_q, x_s
    return torch.split(x_q, m_splits, dim=0), torch.split(x_s, m_splits, dim=1)
