"""Expert-parallel MXFP4 payload rows: [codes (H/2 bytes) | E8M0 scales (H/32 bytes)].

Megatron's FP4 path (code/megatron-0.15.0rc7.diff:32-63, 163-170) quantizes the
tokens it sends through DeepEP, concatenates codes and scales along the last
dimension (``torch.cat``), and on the receiving side splits the payload again
with two ``.contiguous()`` copies before requantizing or dequantizing it.

``pack_rowwise_components`` / ``unpack_rowwise_components`` keep that
behaviour (same checks and errors) for callers that hold the pieces. The
``*_packed`` functions are the fused path: the quantize kernel writes payload
rows directly and the dequant / FP8 requant kernels read them in place, so the
concatenation and both split copies disappear. Their outputs are byte-identical
to the unfused composition.
"""
from typing import List, Optional, Tuple

import torch

from omo import omo_packed_Mxfp4ToBf16_dequant, omo_packed_Mxfp4ToFp8, omo_quant_mxfp4_packed

FP4_VALUES_PER_SCALE = 16  # code bytes per scale byte (megatron-0.15.0rc7.diff:17)


def pack_rowwise_components(rowwise_data: torch.Tensor, rowwise_scale: torch.Tensor) -> torch.Tensor:
    """_pack_rowwise_components (megatron-0.15.0rc7.diff:93-99)."""
    if rowwise_data.shape[:-1] != rowwise_scale.shape[:-1]:
        raise ValueError("rowwise_data and rowwise_scale_inv must match on all dims except the last.")
    return torch.cat((rowwise_data, rowwise_scale), dim=-1)


def unpack_rowwise_components(packed_tensor: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """_unpack_rowwise_components (megatron-0.15.0rc7.diff:101-122): the code
    width is last_dim * 16 / 17; both parts are returned as contiguous copies."""
    if packed_tensor.dim() < 1:
        raise ValueError("Packed FP4 tensor must have at least one dimension.")
    last_dim = packed_tensor.size(-1)
    numerator = last_dim * FP4_VALUES_PER_SCALE
    divisor = FP4_VALUES_PER_SCALE + 1
    if numerator % divisor != 0:
        raise ValueError(
            f"Cannot infer FP4 rowwise/scale split for last_dim={last_dim}. "
            "Dimension must be divisible by the 17/16 packing ratio.")
    rowwise_width = numerator // divisor
    scale_width = last_dim - rowwise_width
    if scale_width <= 0:
        raise ValueError("Packed FP4 tensor does not contain scale elements.")
    rowwise_data = packed_tensor.narrow(-1, 0, rowwise_width).contiguous()
    rowwise_scale = packed_tensor.narrow(-1, rowwise_width, scale_width).contiguous()
    return rowwise_data, rowwise_scale


def payload_width(hidden: int) -> int:
    """Bytes per payload row for hidden size H: H/2 + H/32 = 17H/32."""
    return hidden // 2 + hidden // 32


def _hidden_of(packed: torch.Tensor) -> int:
    width = packed.size(-1)
    if width % 17 != 0:
        raise ValueError(f"payload width {width} is not 17/32 of a hidden size")
    return width // 17 * 32


def fp4_quantize_packed(x: torch.Tensor, eps: float = 1e-10) -> torch.Tensor:
    """Fused ``fp4_quantize`` (megatron-0.15.0rc7.diff:163-170): bf16 [T, H]
    (H % 128 == 0) -> payload [T, 17H/32] uint8, equal to
    pack_rowwise_components(*omo_per_token_group_quant_mxfp4(x))."""
    assert x.dim() == 2, "`x` must be 2-D [tokens, hidden]"
    assert x.is_contiguous(), "`x` is not contiguous"
    T, H = x.shape
    out = torch.empty((T, payload_width(H)), device=x.device, dtype=torch.uint8)
    if T > 0:
        omo_quant_mxfp4_packed(x, out, eps)
    return out


def packed_mxfp4ToBf16(packed: torch.Tensor, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Payload [T, 17H/32] -> [T, H] in ``dtype``, equal to
    omo_per_token_mxfp4ToBf16_dequant_wrapper(*unpack_rowwise_components(packed), dtype)."""
    assert packed.dim() == 2, "payload must be 2-D [tokens, 17H/32]"
    assert packed.is_contiguous(), "payload is not contiguous"
    T, H = packed.size(0), _hidden_of(packed)
    out = torch.empty((T, H), device=packed.device, dtype=torch.bfloat16)
    if T > 0:
        omo_packed_Mxfp4ToBf16_dequant(packed, out)
    return out.to(dtype)


def packed_mxfp4ToFp8(packed: torch.Tensor, m_splits: Optional[List[int]] = None):
    """Payload [T, 17H/32] -> FP8 E4M3 [T, H] and fp32 scales [H/128, T], split
    by ``m_splits`` along tokens as omo_per_token_mxfp4ToFp8_wrapper does
    (code/kernel/api/mxfp4_dequant.py:172-181); without m_splits the whole
    tensors are returned."""
    assert packed.dim() == 2, "payload must be 2-D [tokens, 17H/32]"
    assert packed.is_contiguous(), "payload is not contiguous"
    T, H = packed.size(0), _hidden_of(packed)
    x_q = torch.empty((T, H), device=packed.device, dtype=torch.float8_e4m3fn)
    x_s = torch.empty((H // 128, T), device=packed.device, dtype=torch.float32)
    if T > 0:
        omo_packed_Mxfp4ToFp8(packed, x_q, x_s)
    if m_splits is None:
        return x_q, x_s
    return torch.split(x_q, m_splits, dim=0), torch.split(x_s, m_splits, dim=1)
