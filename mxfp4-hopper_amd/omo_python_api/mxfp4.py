"""BF16 -> MXFP4 quantize wrappers.

Mirrors code/kernel/api/mxfp4.py: same function names, defaults, output
allocation and return values. The wrappers allocate the outputs with
``torch.empty`` and call ``omo`` on the current stream.
"""
from typing import Optional

import torch

from omo import omo_per_token_group_quant_fp4, omo_quant_mxfp4_dual, omo_quant_mxfp4_dual_grouped

fp8_type_ = torch.float8_e4m3fn
uint8_type = torch.uint8
fp8_max = torch.finfo(fp8_type_).max
fp8_min = -fp8_max
mxfp4_max = 6.0
mxfp4_min = -mxfp4_max

FLOAT4_E2M1_MAX = 6.0
FLOAT8_E4M3_MAX = torch.finfo(torch.float8_e4m3fn).max


def align(x: int, y: int) -> int:
    """Round x up to a multiple of y (used by the ue8m0 scale layout; the
    reference calls an `align` it does not define, mxfp4.py:99-100)."""
    return (x + y - 1) // y * y


def omo_per_token_group_quant_4bit_warpper(
    x: torch.Tensor,
    group_size: int,
    dst_dtype: torch.dtype,
    eps: float = 1e-10,
    column_major_scales: bool = False,
    scale_tma_aligned: bool = False,
    scale_ue8m0: bool = False,
    fuse_silu_and_mul: bool = False,
    masked_m: Optional[torch.Tensor] = None,
    enable_v2: Optional[bool] = None,
):
    """Generic entry, forwards to omo_per_token_group_quant_fp4_warpper (mxfp4.py:17-44)."""
    return omo_per_token_group_quant_fp4_warpper(
        x=x,
        group_size=group_size,
        eps=eps,
        column_major_scales=column_major_scales,
        scale_tma_aligned=scale_tma_aligned,
        scale_ue8m0=scale_ue8m0,
        fuse_silu_and_mul=fuse_silu_and_mul,
        masked_m=masked_m,
        enable_v2=enable_v2,
    )


def omo_per_token_group_quant_fp4_warpper(
    x: torch.Tensor,
    group_size: int,
    eps: float = 1e-10,
    column_major_scales: bool = False,
    scale_tma_aligned: bool = False,
    scale_ue8m0: bool = False,
    fuse_silu_and_mul: bool = False,
    masked_m: Optional[torch.Tensor] = None,
    enable_v2: Optional[bool] = None,
):
    """mxfp4.py:45-81. Allocates the scale tensor from the *code* shape
    [M, K/2] as the reference does; the kernel fills its first numel/32 bytes
    in flat block order."""
    assert x.shape[-1] % group_size == 0, "the last dimension of `x` cannot be divisible by `group_size`"
    assert x.is_contiguous(), "`x` is not contiguous"
    out_shape = (*x.shape[:-1], x.shape[-1] // 2)
    x_q = torch.empty(out_shape, device=x.device, dtype=uint8_type)
    x_s = create_per_token_group_quant_fp8_output_scale(
        x_shape=out_shape,
        device=x.device,
        group_size=group_size,
        column_major_scales=column_major_scales,
        scale_tma_aligned=scale_tma_aligned,
        scale_ue8m0=scale_ue8m0,
    )
    if x.shape[0] > 0:
        omo_per_token_group_quant_fp4(x, x_q, x_s, group_size, eps, mxfp4_min, mxfp4_max, scale_ue8m0)
    return x_q, x_s


def create_per_token_group_quant_fp8_output_scale(
    x_shape,
    device,
    group_size,
    column_major_scales: bool,
    scale_tma_aligned: bool,
    scale_ue8m0: bool,
):
    """mxfp4.py:87-115: uint8 scales of shape (x_shape[0], x_shape[1]), or the
    transposed int32 ue8m0 layout (which the quantize kernel rejects)."""
    if scale_ue8m0:
        assert column_major_scales and scale_tma_aligned
        *x_batch, x_q_mn, x_q_k = x_shape
        x_s_mn, x_s_k = x_q_mn, x_q_k // 128
        aligned_mn = align(x_s_mn, 4)
        aligned_k = align(x_s_k, 4)
        return torch.empty((*x_batch, aligned_k // 4, aligned_mn), device=device,
                           dtype=torch.int).transpose(-1, -2)[..., :x_s_mn, :]
    scale_shape = (x_shape[0], x_shape[1])
    return torch.empty(scale_shape, device=device, dtype=torch.uint8)


def omo_per_token_group_quant_mxfp4(x: torch.Tensor):
    """The quantize entry used by TE (mxfp4.py:118-156; called at
    code/transformer_engine-2.8.diff:672-673). x [M, K] bf16, K % 32 == 0 ->
    (codes uint8 [M, K/2], scales uint8 E8M0 [M, K/32])."""
    group_size = 32
    eps = 1e-10
    scale_ue8m0 = False
    assert x.shape[-1] % group_size == 0, "the last dimension of `x` cannot be divisible by `group_size`"
    assert x.is_contiguous(), "`x` is not contiguous"
    out_shape = (*x.shape[:-1], x.shape[-1] // 2)
    scale_shape = (*x.shape[:-1], x.shape[-1] // 32)
    x_q = torch.empty(out_shape, device=x.device, dtype=uint8_type)
    x_s = create_per_token_group_quant_fp8_output_scale(
        x_shape=scale_shape,
        device=x.device,
        group_size=group_size,
        column_major_scales=False,
        scale_tma_aligned=True,
        scale_ue8m0=scale_ue8m0,
    )
    if x.shape[0] > 0:
        omo_per_token_group_quant_fp4(x, x_q, x_s, group_size, eps, mxfp4_min, mxfp4_max, scale_ue8m0)
    return x_q, x_s


def omo_per_token_group_quant_mxfp4_dual(x: torch.Tensor, eps: float = 1e-10):
    """Rowwise and columnwise MXFP4 of a 2-D [M, K] bf16 tensor in one pass:
    returns (row codes [M, K/2], row scales [M, K/32], col codes [K, M/2],
    col scales [K, M/32]); the column pair equals
    omo_per_token_group_quant_mxfp4(x.T.contiguous()), which is how TE builds
    the columnwise usage (code/transformer_engine-2.8.diff:1463-1466)."""
    assert x.dim() == 2, "`x` must be 2-D"
    M, K = x.shape
    assert M % 32 == 0 and K % 32 == 0, "both dimensions of `x` must be multiples of 32"
    assert x.is_contiguous(), "`x` is not contiguous"
    row_q = torch.empty((M, K // 2), device=x.device, dtype=uint8_type)
    row_s = torch.empty((M, K // 32), device=x.device, dtype=uint8_type)
    col_q = torch.empty((K, M // 2), device=x.device, dtype=uint8_type)
    col_s = torch.empty((K, M // 32), device=x.device, dtype=uint8_type)
    if M > 0 and K > 0:
        omo_quant_mxfp4_dual(x, row_q, row_s, col_q, col_s, eps)
    return row_q, row_s, col_q, col_s


def omo_per_token_group_quant_mxfp4_dual_grouped(xs, eps: float = 1e-10):
    """omo_per_token_group_quant_mxfp4_dual over a list of 2-D bf16 tensors
    (e.g. the gate/up/down weights of all local experts) in one launch; returns
    one (row codes, row scales, col codes, col scales) tuple per tensor."""
    outs = []
    for x in xs:
        assert x.dim() == 2, "every tensor must be 2-D"
        M, K = x.shape
        assert M % 32 == 0 and K % 32 == 0, "both dimensions must be multiples of 32"
        assert x.is_contiguous(), "tensors must be contiguous"
        outs.append((torch.empty((M, K // 2), device=x.device, dtype=uint8_type),
                     torch.empty((M, K // 32), device=x.device, dtype=uint8_type),
                     torch.empty((K, M // 2), device=x.device, dtype=uint8_type),
                     torch.empty((K, M // 32), device=x.device, dtype=uint8_type)))
    if xs:
        omo_quant_mxfp4_dual_grouped(list(xs), outs, eps)
    return outs
