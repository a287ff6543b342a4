"""MXFP4 -> BF16 dequant and MXFP4 -> FP8 requant wrappers.

Mirrors code/kernel/api/mxfp4_dequant.py (padding, output allocation, slicing
and splitting) and adds the two wrappers the TE integration imports but the
reference does not ship:
  * omo_per_token_mxfp4RowToBf16ToFp8Col_wrapper (code/transformer_engine-2.8.diff:198, 259-272)
  * omo_per_token_mxfp4RowToBf16ToFp8Col_msplit_wrapper (code/transformer_engine-2.8.diff:70, 159-176)
Their contracts are reconstructed from those call sites and from the host
checks of the bound functions; eps = 1e-10 as in every shipped wrapper.
"""
from typing import List

import torch
import torch.nn.functional as F

from omo import (
    omo_per_token_Mxfp4RowToBf16ToFp8Col,
    omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit,
    omo_per_token_Mxfp4ToBf16_dequant,
    omo_per_token_Mxfp4ToBf16ToFp8,
    omo_per_token_Mxfp4ToFp8,
    omo_per_token_Mxfp4ToFp8_col,
)

fp8_type_ = torch.float8_e4m3fn
uint8_type = torch.uint8
fp8_max = torch.finfo(fp8_type_).max
fp8_min = -fp8_max
mxfp4_max = 6.0
mxfp4_min = -mxfp4_max

FLOAT4_E2M1_MAX = 6.0
FLOAT8_E4M3_MAX = torch.finfo(torch.float8_e4m3fn).max


def pad_to_multiple(x, multiple=128):
    """Zero-pad the last dim to a multiple (mxfp4_dequant.py:15-29); returns
    (padded tensor, original last dim). No copy when already a multiple."""
    last_dim = x.shape[-1]
    pad_amount = (multiple - (last_dim % multiple)) % multiple
    x_padded = F.pad(x, (0, pad_amount)) if pad_amount > 0 else x
    return x_padded, last_dim


def unpad_from_multiple(x_padded, original_size):
    """mxfp4_dequant.py:31-33."""
    return x_padded[..., :original_size]


def omo_per_token_mxfp4ToBf16_dequant_wrapper(x: torch.Tensor, x_in_s: torch.Tensor, dtype):
    """codes [M, K/2] + scales [M, K/32] -> x_q.to(dtype) of shape [M, K]
    (mxfp4_dequant.py:39-74; called at code/transformer_engine-2.8.diff:392)."""
    group_size = 32
    eps = 1e-10
    scale_ue8m0 = False
    assert x.shape[-1] % group_size == 0, "the last dimension of `x` cannot be divisible by `group_size`"
    assert x.is_contiguous(), "`x` is not contiguous"
    out_shape = (*x.shape[:-1], x.shape[-1] * 2)
    scale_shape = (*x.shape[:-1], x.shape[-1] * 2 // 128)
    x_q = torch.empty(out_shape, device=x.device, dtype=torch.bfloat16)
    x_s = torch.empty(scale_shape, device=x.device, dtype=torch.float)
    if x.shape[0] > 0:
        omo_per_token_Mxfp4ToBf16_dequant(x, x_in_s, x_q, x_s, group_size, eps, mxfp4_min, mxfp4_max, scale_ue8m0)
    return x_q.to(dtype)


def omo_per_token_mxfp4ToBf16ToFp8_wrapper(x: torch.Tensor, x_in_s: torch.Tensor):
    """mxfp4_dequant.py:79-121: codes padded to 16 bytes, fp8 [M, 2Kp] sliced to
    [M, 2K], scales [2Kp/128, M] (TE layout)."""
    group_size = 128
    eps = 1e-10
    scale_ue8m0 = False
    x_padded, original_w = pad_to_multiple(x, multiple=16)
    assert x.is_contiguous(), "`x` is not contiguous"
    out_shape = (*x_padded.shape[:-1], x_padded.shape[-1] * 2)
    scale_shape = ((x_padded.shape[-1] * 2 // 128), *x_padded.shape[:-1])
    x_q = torch.empty(out_shape, device=x.device, dtype=fp8_type_)
    x_s = torch.empty(scale_shape, device=x.device, dtype=torch.float)
    if x.shape[0] > 0:
        omo_per_token_Mxfp4ToBf16ToFp8(x_padded, x_in_s, x_q, x_s, group_size, eps, mxfp4_min, mxfp4_max, scale_ue8m0)
    x_q = x_q[:, :original_w * 2]
    return x_q, x_s


def omo_per_token_mxfp4ToFp8_wrapper(x: torch.Tensor, x_in_s: torch.Tensor, m_splits: List[int] = None):
    """mxfp4_dequant.py:122-187 (called at code/transformer_engine-2.8.diff:163):
    codes padded to 64 bytes and scales to 4 columns, fp8 [M, 2Kp] + fp32
    [2Kp/128, M], sliced, then split by m_splits along rows (fp8, dim 0) and
    columns (scales, dim 1)."""
    group_size = 128
    eps = 1e-10
    scale_ue8m0 = False
    assert x.is_contiguous(), "`x` is not contiguous"
    x_padded, original_w = pad_to_multiple(x, multiple=64)
    x_in_s_pad, original_w_scale = pad_to_multiple(x_in_s, multiple=4)
    out_shape = (*x_padded.shape[:-1], x_padded.shape[-1] * 2)
    scale_shape = ((x_padded.shape[-1] * 2 // 128), *x_padded.shape[:-1])
    x_q = torch.empty(out_shape, device=x.device, dtype=fp8_type_)
    x_s = torch.empty(scale_shape, device=x.device, dtype=torch.float)
    if x.shape[0] > 0:
        omo_per_token_Mxfp4ToFp8(x_padded, x_in_s_pad, x_q, x_s, group_size, eps, mxfp4_min, mxfp4_max, scale_ue8m0)
    x_q = x_q[:, :original_w * 2]
    # the reference slices the scale rows with the MX scale width
    # (mxfp4_dequant.py:172), which keeps every row
    x_s = x_s[:original_w_scale, :]
    x_q_split = torch.split(x_q, m_splits, dim=0)
    x_s_split = torch.split(x_s, m_splits, dim=1)
    return x_q_split, x_s_split


def omo_per_token_mxfp4ToFp8_col_wrapper(x: torch.Tensor, x_in_s: torch.Tensor):
    """mxfp4_dequant.py:189-237: codes padded to 16 bytes -> fp8 transposed
    [2Kp, M] (sliced on the last dim as the reference does) + fp32
    [M/128, 2Kp]."""
    group_size = 128
    eps = 1e-10
    scale_ue8m0 = False
    x_padded, original_w = pad_to_multiple(x, multiple=16)
    assert x.is_contiguous(), "`x` is not contiguous"
    out_shape = (x_padded.shape[-1] * 2, *x_padded.shape[:-1])
    scale_shape = ((x_padded.shape[0] // 128), x_padded.shape[-1] * 2)
    x_q = torch.empty(out_shape, device=x.device, dtype=fp8_type_)
    x_s = torch.empty(scale_shape, device=x.device, dtype=torch.float)
    if x.shape[0] > 0:
        omo_per_token_Mxfp4ToFp8_col(x_padded, x_in_s, x_q, x_s, group_size, eps, mxfp4_min, mxfp4_max, scale_ue8m0)
    x_q = x_q[..., :original_w * 2]
    return x_q, x_s


def omo_per_token_mxfp4RowToBf16ToFp8Col_wrapper(data: torch.Tensor, scale: torch.Tensor, eps: float = 1e-10):
    """Reconstructed wrapper of omo_per_token_Mxfp4RowToBf16ToFp8Col for TE's
    dense wgrad (code/transformer_engine-2.8.diff:259-272): codes [M, N/2] +
    scales [M, N/32] -> (fp8 columnwise data [N, M], fp32 columnwise
    scale_inv [ceil(M/128), N]) in TE's GEMM_READY layout."""
    assert data.dim() == 2 and data.is_contiguous(), "`data` must be a contiguous 2-D tensor"
    M, half = data.shape
    N = half * 2
    out_q = torch.empty((N, M), device=data.device, dtype=fp8_type_)
    out_s = torch.empty(((M + 127) // 128, N), device=data.device, dtype=torch.float)
    if M > 0 and N > 0:
        omo_per_token_Mxfp4RowToBf16ToFp8Col(data, scale.contiguous(), out_q, out_s, eps)
    return out_q, out_s


def split_metadata(m_splits: List[int], device) -> tuple:
    """int32 device tensors (lengths, row offsets, scale-row offsets) and the
    longest split, as the msplit kernel expects them
    (code/kernel/per_token_Mxfp4RowToBf16ToFp8Col_msplit.cu:74-80, 256)."""
    lens = [int(m) for m in m_splits]
    if any(m < 0 for m in lens):
        raise ValueError(f"m_splits must be non-negative, got {lens}")
    offs, soffs, o, so = [], [], 0, 0
    for m in lens:
        offs.append(o)
        soffs.append(so)
        o += m
        so += (m + 127) // 128
    meta = torch.tensor([lens, offs, soffs], dtype=torch.int32).to(device, non_blocking=False)
    return meta[0], meta[1], meta[2], (max(lens) if lens else 0), o, so


def omo_per_token_mxfp4RowToBf16ToFp8Col_msplit_wrapper(data: torch.Tensor, scale: torch.Tensor,
                                                        m_splits: List[int], eps: float = 1e-10):
    """Reconstructed wrapper of omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit for
    TE's grouped wgrad (code/transformer_engine-2.8.diff:159-176): codes
    [sum(m), N/2] + scales -> (list of fp8 [N, m_i], list of fp32
    [ceil(m_i/128), N]), one per expert split, each a view of one buffer."""
    assert data.dim() == 2 and data.is_contiguous(), "`data` must be a contiguous 2-D tensor"
    total_m, half = data.shape
    N = half * 2
    lens, offs, soffs, max_len, rows, srows = split_metadata(m_splits, data.device)
    if rows != total_m:
        raise ValueError(f"sum(m_splits)={rows} does not match data rows {total_m}")
    out_q = torch.empty(total_m * N, device=data.device, dtype=fp8_type_)
    out_s = torch.empty((srows, N), device=data.device, dtype=torch.float)
    if len(m_splits) > 0 and N > 0 and total_m > 0:
        omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit(data, scale.contiguous(), out_q, out_s, lens, offs, soffs, max_len,
                                                    eps)
    y_data, y_scale, o = [], [], 0
    for m in m_splits:
        m = int(m)
        y_data.append(out_q[o * N:(o + m) * N].view(N, m))
        o += m
    y_scale = list(torch.split(out_s, [(int(m) + 127) // 128 for m in m_splits], dim=0))
    return y_data, y_scale
