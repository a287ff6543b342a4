"""``omo``: drop-in for the reference's pybind module of the same name.

The reference binds seven functions (code/kernel/ops.cu:27-41) plus imports an
eighth from its Python API (code/kernel/api/mxfp4_dequant.py:1). This module
exposes the same names, keyword names and argument order. Each function
runs the reference host checks (``CHECK_INPUT`` = on the GPU and contiguous,
``CHECK_EQ`` on sizes; failures raise ``RuntimeError``), then calls the
gfx950 HIP library through its C ABI (include/omo_mxfp4.h) on the current
HIP stream of the input's device. Outputs are preallocated by the caller and
written in place; nothing is returned, as in the reference.

Deliberate differences from the reference host code, each where the
reference would launch a kernel on memory it does not own or silently do
nothing:
  * wrong tensor dtypes raise ``RuntimeError`` (the reference's dispatch
    macro skips the launch);
  * ``scale_ue8m0=True`` and column-major scale tensors raise
    ``NotImplementedError`` (the reference routes them to a kernel launched
    with a thread count it does not support, per_token_quant_mxfp4.cu:287,418);
  * undersized outputs, shapes the reference kernels cannot index (see the
    C ABI), and NaN / non-finite constants raise ``RuntimeError``.
"""
from __future__ import annotations

import torch

from ._abi import check as _check
from ._abi import lib as _lib

__all__ = [
    "omo_per_token_group_quant_fp4",
    "omo_per_token_Mxfp4ToBf16_dequant",
    "omo_per_token_Mxfp4ToBf16ToFp8",
    "omo_per_token_group_quant_fp4_fused_ToFp8",
    "omo_per_token_Mxfp4RowToBf16ToFp8Col",
    "omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit",
    "omo_per_token_Mxfp4ToFp8_col",
    "omo_per_token_Mxfp4ToFp8",
    "omo_quant_mxfp4_dual",
    "omo_quant_mxfp4_dual_grouped",
    "omo_quant_mxfp4_packed",
    "omo_packed_Mxfp4ToBf16_dequant",
    "omo_packed_Mxfp4ToFp8",
    "omo_mxfp4_permute_rows",
    "omo_permute_Mxfp4ToFp8",
]

_FP8 = torch.float8_e4m3fn


def _check_input(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _check_eq(a, b, what: str) -> None:
    if a != b:
        raise RuntimeError(f"Expected {what} ({a} vs. {b})")


def _check_dtype(t: torch.Tensor, dtype: torch.dtype, name: str) -> None:
    if t.dtype != dtype:
        raise RuntimeError(f"{name} must have dtype {dtype}, got {t.dtype}")


def _same_device(ref: torch.Tensor, *others) -> None:
    for o in others:
        if o.device != ref.device:
            raise RuntimeError(f"all tensors must be on {ref.device}, got {o.device}")


def _nbytes(t: torch.Tensor) -> int:
    return t.numel() * t.element_size()


# torch's raw current-stream getter (a few tens of ns) where this torch build
# has it; the public torch.cuda.current_stream(...).cuda_stream builds a Stream
# object per call (about 2 us, a quarter of this binding's host time).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


class _on_device:
    """Make ``t``'s device current for the launch (the library launches on
    the current HIP device) and yield its current stream handle."""

    def __init__(self, t: torch.Tensor):
        self.dev = t.device

    def __enter__(self):
        idx = self.dev.index if self.dev.index is not None else torch.cuda.current_device()
        self.prev = torch.cuda.current_device()
        self.switched = idx != self.prev
        if self.switched:
            torch.cuda.set_device(idx)
        if _raw_stream is not None:
            return _raw_stream(idx)
        return torch.cuda.current_stream(idx).cuda_stream

    def __exit__(self, *exc):
        if self.switched:
            torch.cuda.set_device(self.prev)
        return False


def omo_per_token_group_quant_fp4(input, output_q, output_s, group_size, eps, fp4_min, fp4_max, scale_ue8m0):
    """BF16 -> MXFP4 quantize, 1x32 blocks over the flat tensor.
    Reference: omo::omo_per_token_group_quant_fp4, code/kernel/per_token_quant_mxfp4.cu:387-487."""
    _check_input(input, "input")
    _check_input(output_q, "output_q")
    if group_size <= 0:
        raise RuntimeError(f"group_size must be positive, got {group_size}")
    _check_eq(input.numel() % group_size, 0, "input.numel() % group_size == 0")
    _check_eq(output_s.dim(), 2, "output_s.dim() == 2")
    _same_device(input, output_q, output_s)
    if output_s.stride(0) < output_s.stride(1):
        raise NotImplementedError("column-major scale tensors are not supported")
    if not output_s.is_contiguous():
        raise RuntimeError("output_s must be contiguous")
    _check_dtype(input, torch.bfloat16, "input")
    _check_dtype(output_q, torch.uint8, "output_q")
    with _on_device(input) as stream:
        _check(_lib.omo_hip_per_token_group_quant_fp4(
            input.data_ptr(), input.numel(), output_q.data_ptr(), _nbytes(output_q), output_s.data_ptr(),
            _nbytes(output_s), int(group_size), float(eps), float(fp4_min), float(fp4_max), int(bool(scale_ue8m0)),
            stream))


def omo_per_token_Mxfp4ToBf16_dequant(input, input_s, output_q, output_s, group_size, eps, fp4_min, fp4_max,
                                      scale_ue8m0):
    """MXFP4 -> BF16 dequant over the flat code tensor.
    Reference: omo::omo_per_token_Mxfp4ToBf16_dequant, code/kernel/per_token_Mxfp4ToBf16_dequant.cu:164-238."""
    _check_input(input, "input")
    _check_input(output_q, "output_q")
    _check_eq(input.numel() % 128, 0, "input.numel() % group_size == 0")
    _check_eq(output_s.dim(), 2, "output_s.dim() == 2")
    _same_device(input, input_s, output_q)
    _check_input(input_s, "input_s")
    _check_dtype(input, torch.uint8, "input")
    _check_dtype(input_s, torch.uint8, "input_s")
    _check_dtype(output_q, torch.bfloat16, "output_q")
    with _on_device(input) as stream:
        _check(_lib.omo_hip_per_token_Mxfp4ToBf16_dequant(
            input.data_ptr(), input.numel(), input_s.data_ptr(), input_s.numel(), output_q.data_ptr(),
            output_q.numel(), output_s.data_ptr(), _nbytes(output_s), int(group_size), float(eps), float(fp4_min),
            float(fp4_max), int(bool(scale_ue8m0)), stream))


def _requant_args(name, input, input_s, output_q, output_s):
    _check_input(input, "input")
    _check_input(output_q, "output_q")
    _check_eq(input.numel() % 128, 0, "input.numel() % group_size == 0")
    _check_eq(output_s.dim(), 2, "output_s.dim() == 2")
    if input.dim() != 2:
        raise RuntimeError(f"{name}: input must be 2-D [M, K/2]")
    _same_device(input, input_s, output_q, output_s)
    _check_input(input_s, "input_s")
    _check_input(output_s, "output_s")
    _check_dtype(input, torch.uint8, "input")
    _check_dtype(input_s, torch.uint8, "input_s")
    _check_dtype(output_q, _FP8, "output_q")
    _check_dtype(output_s, torch.float32, "output_s")


def _requant_rowwise(fn, name, input, input_s, output_q, output_s, group_size, eps, fp4_min, fp4_max, scale_ue8m0):
    _requant_args(name, input, input_s, output_q, output_s)
    with _on_device(input) as stream:
        _check(fn(input.data_ptr(), input.size(0), input.size(1), input_s.data_ptr(), input_s.numel(),
                  output_q.data_ptr(), output_q.numel(), output_s.data_ptr(), output_s.numel(), int(group_size),
                  float(eps), float(fp4_min), float(fp4_max), int(bool(scale_ue8m0)), stream))


def omo_per_token_Mxfp4ToFp8(input, input_s, output_q, output_s, group_size, eps, fp4_min, fp4_max, scale_ue8m0):
    """MXFP4 -> FP8 E4M3 rowwise with 1x128 power-of-two scales, stored [K/64, M].
    Reference: omo::omo_per_token_Mxfp4ToFp8, code/kernel/per_token_Mxfp4ToFp8.cu:238-309."""
    _requant_rowwise(_lib.omo_hip_per_token_Mxfp4ToFp8, "omo_per_token_Mxfp4ToFp8", input, input_s, output_q,
                     output_s, group_size, eps, fp4_min, fp4_max, scale_ue8m0)


def omo_per_token_Mxfp4ToBf16ToFp8(input, input_s, output_q, output_s, group_size, eps, fp4_min, fp4_max,
                                   scale_ue8m0):
    """Bound by the reference (code/kernel/ops.cu:32-33) without a shipped source;
    same signature and call site shape as omo_per_token_Mxfp4ToFp8, computed by it."""
    _requant_rowwise(_lib.omo_hip_per_token_Mxfp4ToBf16ToFp8, "omo_per_token_Mxfp4ToBf16ToFp8", input, input_s,
                     output_q, output_s, group_size, eps, fp4_min, fp4_max, scale_ue8m0)


def omo_per_token_Mxfp4ToFp8_col(input, input_s, output_q, output_s, group_size, eps, fp4_min, fp4_max, scale_ue8m0):
    """MXFP4 rowwise -> FP8 transposed [K, M] with 128-row power-of-two scales (sign dropped).
    Reference: omo::omo_per_token_Mxfp4ToFp8_col, code/kernel/per_token_Mxfp4ToFp8_col.cu:305-384."""
    _requant_args("omo_per_token_Mxfp4ToFp8_col", input, input_s, output_q, output_s)
    with _on_device(input) as stream:
        _check(_lib.omo_hip_per_token_Mxfp4ToFp8_col(
            input.data_ptr(), input.size(0), input.size(1), input_s.data_ptr(), input_s.numel(), output_q.data_ptr(),
            output_q.numel(), output_s.data_ptr(), output_s.numel(), int(group_size), float(eps), float(fp4_min),
            float(fp4_max), int(bool(scale_ue8m0)), stream))


def omo_per_token_Mxfp4RowToBf16ToFp8Col(input, input_s, output_q, output_s, eps):
    """MXFP4 rowwise -> FP8 columnwise [N, M] + scale_inv [ceil(M/128), N] (amax/448).
    Reference: omo::omo_per_token_Mxfp4RowToBf16ToFp8Col, code/kernel/per_token_Mxfp4RowToBf16ToFp8Col.cu:204-246."""
    _check_input(input, "input")
    _check_input(output_q, "output_q")
    _check_eq(input.dim(), 2, "input.dim() == 2")
    _check_eq(output_q.dim(), 2, "output_q.dim() == 2")
    _same_device(input, input_s, output_q, output_s)
    _check_input(input_s, "input_s")
    _check_input(output_s, "output_s")
    _check_dtype(input, torch.uint8, "input")
    _check_dtype(input_s, torch.uint8, "input_s")
    _check_dtype(output_q, _FP8, "output_q")
    _check_dtype(output_s, torch.float32, "output_s")
    if input_s.dim() != 2 or output_s.dim() != 2:
        raise RuntimeError("input_s and output_s must be 2-D")
    with _on_device(input) as stream:
        _check(_lib.omo_hip_per_token_Mxfp4RowToBf16ToFp8Col(
            input.data_ptr(), input.size(0), input.size(1), input_s.data_ptr(), input_s.size(0), input_s.size(1),
            output_q.data_ptr(), output_q.size(0), output_q.size(1), output_s.data_ptr(), output_s.size(0),
            output_s.size(1), float(eps), stream))


def omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit(input, input_s, output_q, output_s, m_splits, split_offsets,
                                                scale_offsets, max_split_len, eps):
    """Per-split (MoE expert) MXFP4 rowwise -> FP8 columnwise with power-of-two scales.
    ``m_splits``, ``split_offsets``, ``scale_offsets`` are int32 device tensors.
    Reference: omo::omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit,
    code/kernel/per_token_Mxfp4RowToBf16ToFp8Col_msplit.cu:232-283."""
    for t, n in ((input, "input"), (output_q, "output_q"), (m_splits, "m_splits"), (split_offsets, "split_offsets"),
                 (scale_offsets, "scale_offsets")):
        _check_input(t, n)
    _same_device(input, input_s, output_q, output_s, m_splits, split_offsets, scale_offsets)
    _check_input(input_s, "input_s")
    _check_input(output_s, "output_s")
    if input.dim() != 2:
        raise RuntimeError("input must be 2-D [total_M, N/2]")
    _check_dtype(input, torch.uint8, "input")
    _check_dtype(input_s, torch.uint8, "input_s")
    _check_dtype(output_q, _FP8, "output_q")
    _check_dtype(output_s, torch.float32, "output_s")
    for t, n in ((m_splits, "m_splits"), (split_offsets, "split_offsets"), (scale_offsets, "scale_offsets")):
        _check_dtype(t, torch.int32, n)
        if t.numel() != m_splits.numel():
            raise RuntimeError(f"{n} must have one entry per split")
    with _on_device(input) as stream:
        _check(_lib.omo_hip_per_token_Mxfp4RowToBf16ToFp8Col_msplit(
            input.data_ptr(), input.size(0), input.size(1), input_s.data_ptr(), input_s.numel(), output_q.data_ptr(),
            output_q.numel(), output_s.data_ptr(), output_s.numel(), m_splits.data_ptr(), split_offsets.data_ptr(),
            scale_offsets.data_ptr(), m_splits.numel(), int(max_split_len), float(eps), stream))


def omo_per_token_group_quant_fp4_fused_ToFp8(input, output_q, output_s, output_bf16_q, output_bf16_s, group_size,
                                              eps, fp4_min, fp4_max, scale_ue8m0):
    """Bound by the reference (code/kernel/ops.cu:34-35) but shipped without a
    source or any caller, so its semantics are unknown; it is not implemented."""
    raise NotImplementedError(
        "omo_per_token_group_quant_fp4_fused_ToFp8: the reference ships no implementation of this binding")


def omo_quant_mxfp4_dual(input, row_q, row_s, col_q, col_s, eps=1e-10):
    """Fused rowwise + columnwise BF16 -> MXFP4 quantize of a 2-D [M, K] tensor.
    col_q/col_s equal omo_per_token_group_quant_fp4 applied to input.T.contiguous(),
    the columnwise path of TE's _QuantizeFunc (code/transformer_engine-2.8.diff:1463-1466)."""
    for t, n in ((input, "input"), (row_q, "row_q"), (row_s, "row_s"), (col_q, "col_q"), (col_s, "col_s")):
        _check_input(t, n)
    _same_device(input, row_q, row_s, col_q, col_s)
    if input.dim() != 2:
        raise RuntimeError("input must be 2-D")
    _check_dtype(input, torch.bfloat16, "input")
    for t, n in ((row_q, "row_q"), (row_s, "row_s"), (col_q, "col_q"), (col_s, "col_s")):
        _check_dtype(t, torch.uint8, n)
    with _on_device(input) as stream:
        _check(_lib.omo_hip_quant_mxfp4_dual(
            input.data_ptr(), input.size(0), input.size(1), row_q.data_ptr(), row_q.numel(), row_s.data_ptr(),
            row_s.numel(), col_q.data_ptr(), col_q.numel(), col_s.data_ptr(), col_s.numel(), float(eps), stream))


def omo_quant_mxfp4_dual_grouped(inputs, outputs, eps=1e-10):
    """omo_quant_mxfp4_dual over a list of 2-D bf16 tensors in one launch (per
    32 tensors). outputs[i] = (row_q, row_s, col_q, col_s) of inputs[i]."""
    from ._abi import DualItem
    if len(inputs) != len(outputs):
        raise RuntimeError("inputs and outputs differ in length")
    items = (DualItem * max(1, len(inputs)))()
    for i, (x, outs) in enumerate(zip(inputs, outputs)):
        row_q, row_s, col_q, col_s = outs
        for t, n in ((x, "input"), (row_q, "row_q"), (row_s, "row_s"), (col_q, "col_q"), (col_s, "col_s")):
            _check_input(t, n)
        _same_device(inputs[0], x, row_q, row_s, col_q, col_s)
        if x.dim() != 2:
            raise RuntimeError(f"input {i} must be 2-D")
        _check_dtype(x, torch.bfloat16, "input")
        for t, n in ((row_q, "row_q"), (row_s, "row_s"), (col_q, "col_q"), (col_s, "col_s")):
            _check_dtype(t, torch.uint8, n)
        items[i] = DualItem(x.data_ptr(), x.size(0), x.size(1), row_q.data_ptr(), row_q.numel(), row_s.data_ptr(),
                            row_s.numel(), col_q.data_ptr(), col_q.numel(), col_s.data_ptr(), col_s.numel())
    if not inputs:
        return
    with _on_device(inputs[0]) as stream:
        _check(_lib.omo_hip_quant_mxfp4_dual_grouped(items, len(inputs), float(eps), stream))

# ---------------------------------------------------------------- payload rows
# The expert-parallel payload row [codes (H/2 B) | E8M0 scales (H/32 B)] that
# Megatron builds with torch.cat before the DeepEP dispatch and splits with
# two .contiguous() copies after it (code/megatron-0.15.0rc7.diff:32-63,
# 163-170). These entry points write and read it in place.
def _payload_cols(packed: torch.Tensor) -> int:
    width = packed.size(-1)
    if width % 17 != 0:
        raise RuntimeError(f"payload width {width} is not 17/16 of a code width")
    return width // 17 * 32


def omo_quant_mxfp4_packed(input, output, eps=1e-10):
    """BF16 [T, H] -> payload rows [T, 17H/32] uint8, byte-identical to
    torch.cat(quantize codes, quantize scales, dim=-1). H % 128 == 0."""
    _check_input(input, "input")
    _check_input(output, "output")
    _same_device(input, output)
    if input.dim() != 2:
        raise RuntimeError("input must be 2-D")
    _check_dtype(input, torch.bfloat16, "input")
    _check_dtype(output, torch.uint8, "output")
    with _on_device(input) as stream:
        _check(_lib.omo_hip_quant_mxfp4_packed(input.data_ptr(), input.size(0), input.size(1), output.data_ptr(),
                                               output.numel(), float(eps), stream))


def omo_packed_Mxfp4ToBf16_dequant(input, output):
    """Payload rows [T, 17H/32] -> bf16 [T, H]."""
    _check_input(input, "input")
    _check_input(output, "output")
    _same_device(input, output)
    if input.dim() != 2:
        raise RuntimeError("input must be 2-D")
    _check_dtype(input, torch.uint8, "input")
    _check_dtype(output, torch.bfloat16, "output")
    cols = _payload_cols(input)
    with _on_device(input) as stream:
        _check(_lib.omo_hip_packed_Mxfp4ToBf16_dequant(input.data_ptr(), input.size(0), cols, output.data_ptr(),
                                                       output.numel(), stream))


def omo_packed_Mxfp4ToFp8(input, output_q, output_s):
    """Payload rows [T, 17H/32] -> fp8 [T, H] + fp32 [H/128, T], the outputs of
    omo_per_token_Mxfp4ToFp8 on the unpacked codes and scales."""
    for t, n in ((input, "input"), (output_q, "output_q"), (output_s, "output_s")):
        _check_input(t, n)
    _same_device(input, output_q, output_s)
    if input.dim() != 2:
        raise RuntimeError("input must be 2-D")
    _check_dtype(input, torch.uint8, "input")
    _check_dtype(output_q, _FP8, "output_q")
    _check_dtype(output_s, torch.float32, "output_s")
    cols = _payload_cols(input)
    with _on_device(input) as stream:
        _check(_lib.omo_hip_packed_Mxfp4ToFp8(input.data_ptr(), input.size(0), cols, output_q.data_ptr(),
                                              output_q.numel(), output_s.data_ptr(), output_s.numel(), stream))


# ----------------------------------------------------------------- permutation
# Row gathers of MXFP4 tensors (the data movement of TE's moe_permute for
# MXFP4 inputs, code/transformer_engine-2.8.diff:256-261, 338-354). codes
# [T, H/2] and scales [T, H/32] may be row-strided views (last-dim stride 1),
# e.g. the two halves of payload rows.
def _rows_view(t: torch.Tensor, name: str):
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if t.dim() != 2 or (t.size(1) > 1 and t.stride(1) != 1):
        raise RuntimeError(f"{name} must be 2-D with unit stride along the last dimension")
    _check_dtype(t, torch.uint8, name)
    rows = t.size(0)
    stride = t.stride(0) if rows > 1 else t.size(1)
    span = 0 if rows == 0 else (rows - 1) * stride + t.size(1)
    return t.data_ptr(), span, stride


def _permute_args(codes, scales, src_rows):
    if codes.size(0) != scales.size(0):
        raise RuntimeError("codes and scales must have the same number of rows")
    cols = codes.size(1) * 2
    if scales.size(1) != cols // 32:
        raise RuntimeError("scales must have H/32 columns for codes of H/2 columns")
    _check_input(src_rows, "src_rows")
    _check_dtype(src_rows, torch.int32, "src_rows")
    _same_device(codes, scales, src_rows)
    cp, cb, cs = _rows_view(codes, "codes")
    sp, sb, ss = _rows_view(scales, "scales")
    return (cp, cb, cs, sp, sb, ss, codes.size(0), cols, src_rows.data_ptr(), src_rows.numel())


def omo_mxfp4_permute_rows(codes, scales, src_rows, out_codes, out_scales):
    """out_codes[r] = codes[src_rows[r]], out_scales[r] = scales[src_rows[r]]
    (zero rows for indices outside [0, T))."""
    args = _permute_args(codes, scales, src_rows)
    for t, n in ((out_codes, "out_codes"), (out_scales, "out_scales")):
        _check_input(t, n)
        _check_dtype(t, torch.uint8, n)
    _same_device(codes, out_codes, out_scales)
    with _on_device(codes) as stream:
        _check(_lib.omo_hip_mxfp4_permute_rows(*args, out_codes.data_ptr(), out_codes.numel(),
                                               out_scales.data_ptr(), out_scales.numel(), stream))


def omo_permute_Mxfp4ToFp8(codes, scales, src_rows, output_q, output_s):
    """omo_per_token_Mxfp4ToFp8 of the gathered rows in one kernel: output_q
    [N, H] fp8, output_s [H/128, N] fp32, N = src_rows.numel()."""
    args = _permute_args(codes, scales, src_rows)
    _check_input(output_q, "output_q")
    _check_input(output_s, "output_s")
    _check_dtype(output_q, _FP8, "output_q")
    _check_dtype(output_s, torch.float32, "output_s")
    _same_device(codes, output_q, output_s)
    with _on_device(codes) as stream:
        _check(_lib.omo_hip_permute_Mxfp4ToFp8(*args, output_q.data_ptr(), output_q.numel(), output_s.data_ptr(),
                                               output_s.numel(), stream))
