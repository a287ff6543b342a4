"""TE-facing MXFP4 tensor and quantizer on the HIP codec.

Restates the behaviour of the classes the TE integration adds:
  * MXFP4TensorBase, _FromMXFP4Func
    (code/transformer_engine-2.8.diff:346-637, tensor/_internal/mxfp4_tensor_base.py)
  * MXFP4Quantizer, MXFP4Tensor, _ViewFunc, _ReshapeFunc, _QuantizeFunc
    (code/transformer_engine-2.8.diff:638-1480, tensor/mxfp4_tensor.py)
TE itself is not a dependency: the small part of TE's ``Quantizer`` /
``QuantizedTensor`` base classes these classes rely on (usage flags,
``__call__``, ``make_like``, the dequantize-and-run default of
``__torch_dispatch__``) is restated here as ``Quantizer`` and
``QuantizedTensor``, and the module's classes derive from those.
``build_mxfp4_classes`` defines the same family on any bases, and
``bind_to_te()`` builds it on TE's own ``Quantizer`` / ``QuantizedTensor`` /
``QuantizedTensorBase`` (imported from an installed transformer_engine, or
passed in), so that TE's ``isinstance`` checks recognise the tensors.

Differences from the reference, each where it would fail or go stale:
  * rowwise + columnwise quantize of a 2-D tensor is one launch of the fused
    dual-layout kernel; the reference quantizes ``tensor.T.contiguous()`` in a
    second pass (diff:1463-1466). The outputs are identical byte for byte.
  * ``update_quantized`` (``quantize_``, ``.data =``) refreshes the
    columnwise pair too when the destination holds one; the reference only
    rewrites the rowwise pair (diff:721-740), leaving stale columnwise data.
  * ``__reduce_ex__`` passes every argument ``_make_in_reduce_ex`` takes (the
    reference passes 8 of 10, diff:1115-1160, so pickling raised).
  * ``zero_`` zeroes the codes and sets the scale bytes to 1 in place; the
    reference builds a new tensor with those values inside
    ``__torch_dispatch__`` (diff:1070-1098), which the in-place call discards,
    so the tensor kept its values.
"""
from __future__ import annotations

import copy
import math
import warnings
from collections.abc import Iterable
from types import SimpleNamespace
from typing import Any, Dict, Optional, Tuple, Union

import torch
from torch.utils._pytree import tree_map

from .mxfp4 import omo_per_token_group_quant_mxfp4, omo_per_token_group_quant_mxfp4_dual
from .mxfp4_dequant import omo_per_token_mxfp4ToBf16_dequant_wrapper

aten = torch.ops.aten

MXFP4_BLOCK_SCALING_SIZE = 32  # constants.py addition, diff:28-30

# TE passes its own ``tex.DType`` enum member here; this name stands in for
# ``tex.DType.kFloat8E4M3`` when TE is not installed. The value is carried,
# never interpreted.
DEFAULT_FP8_DTYPE = "kFloat8E4M3"


def _round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


def _canonical_shape(shape, cur_shape) -> list:
    """Shape argument of view/reshape: a tuple, a single iterable or an int,
    with at most one -1 inferred (diff:508-523)."""
    if not isinstance(shape, Iterable):
        shape = [shape]
    elif len(shape) == 1 and isinstance(shape[0], Iterable):
        shape = shape[0]
    shape = list(shape)
    if -1 in shape:
        inferred = -math.prod(cur_shape) // math.prod(shape)
        shape[shape.index(-1)] = inferred
    return shape


def _reshaped_data(tensor, shape, cur_shape, op: str):
    """Rowwise codes reshaped to shape[:-1] + [shape[-1]/2], columnwise codes
    to [shape[-1], prod(shape[:-1])/2]; the inner dimension cannot change
    (diff:524-575, 1251-1276)."""
    if shape[-1] != cur_shape[-1]:
        raise RuntimeError("MXFP4Tensor does not support reshaping inner dimension "
                           f"(attempted to reshape dims={tuple(cur_shape)} to {tuple(shape)})")
    row = col = None
    if tensor._rowwise_data is not None:
        if shape[-1] % 2 != 0:
            raise ValueError(f"Cannot represent row-wise data for MXFP4 tensor with shape={shape} as byte array.")
        row = getattr(tensor._rowwise_data, op)(list(shape[:-1]) + [shape[-1] // 2])
    if tensor._columnwise_data is not None:
        inner, outer = shape[-1], math.prod(shape[:-1])
        if outer % 2 != 0:
            raise ValueError(f"Cannot represent column-wise data for MXFP4 tensor with shape={shape} as byte array.")
        col = getattr(tensor._columnwise_data, op)((inner, outer // 2))
    return row, col


# --------------------------------------------------------------------------- base classes
class Quantizer:
    """The part of TE's quantizer base the MXFP4 quantizer uses: usage flags,
    ``internal``, ``set_usage``, ``copy`` and ``__call__`` -> ``quantize``."""

    def __init__(self, *, rowwise: bool = True, columnwise: bool = True) -> None:
        self.rowwise_usage = rowwise
        self.columnwise_usage = columnwise
        self.internal = False

    def set_usage(self, *, rowwise: Optional[bool] = None, columnwise: Optional[bool] = None) -> None:
        if rowwise is not None:
            self.rowwise_usage = rowwise
        if columnwise is not None:
            self.columnwise_usage = columnwise

    def copy(self) -> "Quantizer":
        return copy.copy(self)

    def __call__(self, tensor: torch.Tensor):
        return self.quantize(tensor)


class QuantizedTensor(torch.Tensor):
    """Wrapper tensor with a nominal shape and dtype and no storage of its own.

    Ops this class does not handle take the dequantized value; ops that write
    to a quantized operand compute on the dequantized value and quantize the
    result back into it."""

    def __new__(cls, shape, dtype, *, requires_grad: bool = False, device: Optional[torch.device] = None):
        return torch.Tensor._make_wrapper_subclass(cls, shape, dtype=dtype, layout=torch.strided,
                                                   requires_grad=requires_grad,
                                                   device=torch.cuda.current_device() if device is None else device)

    @classmethod
    def make_like(cls, tensor, *, shape=None, dtype=None, requires_grad: bool = False, data=None):
        kwargs = tensor.get_metadata()
        if data is not None:
            kwargs["data"] = data
        return cls(shape=tensor.shape if shape is None else shape, dtype=tensor.dtype if dtype is None else dtype,
                   requires_grad=requires_grad, device=tensor.device, **kwargs)

    @classmethod
    def __torch_dispatch__(cls, func, types, args, kwargs=None):
        kwargs = kwargs or {}
        if func == aten.detach.default:
            return args[0].detach()
        if func == aten.copy_.default:
            dst, src = args[0], args[1]
            if isinstance(dst, QuantizedTensor):
                dst.quantize_(src)
            else:
                dst.copy_(src.dequantize() if isinstance(src, QuantizedTensor) else src)
            return dst
        if func == aten.view.default:
            raise NotImplementedError(f"{cls.__name__} class does not support tensor views")

        def unwrap(a):
            return a.dequantize(dtype=a.dtype) if isinstance(a, QuantizedTensor) else a

        new_args, new_kwargs = tree_map(unwrap, args), tree_map(unwrap, kwargs)
        if func._schema.is_mutable:
            func(*new_args, **new_kwargs)
            schema_args = func._schema.arguments
            pairs = list(zip(args, new_args, schema_args))
            pairs += [(kwargs[a.name], new_kwargs[a.name], a) for a in schema_args if a.name in kwargs]
            for old, new, sa in pairs:
                info = getattr(sa, "alias_info", None)
                if isinstance(old, QuantizedTensor) and info is not None and info.is_write:
                    old.quantize_(new)
            return args[0]
        return func(*new_args, **new_kwargs)

    __torch_function__ = torch._C._disabled_torch_function_impl


# --------------------------------------------------------------------------- quantizer
def _quantize_pairs(tensor: torch.Tensor, rowwise: bool, columnwise: bool):
    """(row codes, row scales, col codes, col scales); pairs not asked for are
    None. Both pairs of a 2-D tensor come from one dual-layout launch."""
    if columnwise and tensor.dim() == 2:
        rq, rs, cq, cs = omo_per_token_group_quant_mxfp4_dual(tensor)
        return (rq, rs, cq, cs) if rowwise else (None, None, cq, cs)
    rq = rs = cq = cs = None
    if rowwise:
        rq, rs = omo_per_token_group_quant_mxfp4(tensor)
    if columnwise:
        cq, cs = omo_per_token_group_quant_mxfp4(tensor.T.contiguous())
    return rq, rs, cq, cs


# --------------------------------------------------------------------------- the MXFP4 classes
def build_mxfp4_classes(Quantizer=Quantizer, QuantizedTensor=QuantizedTensor, QuantizedTensorBase=object,
                        name_prefix: str = ""):
    """Defines MXFP4TensorBase, MXFP4Quantizer and MXFP4Tensor (and their
    autograd functions) on the given base classes, the way the TE patch
    derives them from TE's own ``QuantizedTensorBase``, ``QuantizedTensor``
    and ``Quantizer`` (code/transformer_engine-2.8.diff:409, 667, 908).

    The defaults are the bases restated in this module; the module's
    ``MXFP4TensorBase`` / ``MXFP4Quantizer`` / ``MXFP4Tensor`` are built from
    them. Passing TE's classes gives a family that TE's ``isinstance``
    dispatch, ``prepare_for_saving`` and GEMM paths recognise (``bind_to_te``).
    The classes are registered in this module as ``name_prefix + name`` so
    that pickling finds them. Returns a namespace of the new classes."""

    class _FromMXFP4Func(torch.autograd.Function):
        """MXFP4 -> ``dtype`` through the rowwise dequant kernel (diff:379-406);
        the gradient passes through unchanged."""

        @staticmethod
        def forward(_ctx, tensor: "MXFP4TensorBase", dtype: torch.dtype) -> torch.Tensor:
            if tensor._rowwise_data is not None:
                return omo_per_token_mxfp4ToBf16_dequant_wrapper(tensor._rowwise_data, tensor._rowwise_scale_inv,
                                                                 dtype=dtype)
            if tensor._columnwise_data is not None:
                raise NotImplementedError("Dequantizing column-wise MXFP4 data is not implemented yet!")
            raise ValueError("Attempted to dequantize MXFP4 tensor with no data")

        @staticmethod
        def backward(_ctx, grad: torch.Tensor):
            return grad, None


    class MXFP4TensorBase(QuantizedTensorBase):
        """Holder of the rowwise pair (codes [M, K/2], E8M0 scales [M, K/32]) and
        the columnwise pair (codes [K, M/2], scales [K, M/32]) of one tensor
        (diff:409-637). Either pair may be absent."""

        _rowwise_data: Optional[torch.Tensor]
        _columnwise_data: Optional[torch.Tensor]
        _quantizer: Optional[Quantizer]
        _rowwise_scale_inv: Optional[torch.Tensor]
        _columnwise_scale_inv: Optional[torch.Tensor]
        _fp8_dtype: Any
        _is_2D_scaled: bool

        def __new__(cls, rowwise_data, rowwise_scale_inv, columnwise_data, columnwise_scale_inv, fp8_dtype, quantizer,
                    *args, **kwargs):
            instance = super().__new__(cls, *args, **kwargs)
            instance._rowwise_data = rowwise_data
            instance._columnwise_data = columnwise_data
            instance._fp8_dtype = fp8_dtype
            instance._quantizer = quantizer.copy() if quantizer is not None else None
            instance._rowwise_scale_inv = rowwise_scale_inv
            instance._columnwise_scale_inv = columnwise_scale_inv
            instance._is_2D_scaled = False
            return instance

        def clear(self):
            """Release the memory of all four tensors (they become empty)."""
            for t in (self._rowwise_data, self._columnwise_data, self._rowwise_scale_inv, self._columnwise_scale_inv):
                if t is not None:
                    t.data = torch.empty(0, dtype=t.dtype, device=t.device)

        def get_metadata(self) -> Dict[str, Any]:
            return {
                "rowwise_data": self._rowwise_data,
                "rowwise_scale_inv": self._rowwise_scale_inv,
                "columnwise_data": self._columnwise_data,
                "columnwise_scale_inv": self._columnwise_scale_inv,
                "fp8_dtype": self._fp8_dtype,
                "quantizer": self._quantizer,
            }

        def prepare_for_saving(self):
            """Hand the four tensors to autograd's saved-tensor list and drop them
            here (diff:474-486)."""
            tensors = [self._rowwise_data, self._columnwise_data, self._rowwise_scale_inv, self._columnwise_scale_inv]
            self._rowwise_data = self._columnwise_data = None
            self._rowwise_scale_inv = self._columnwise_scale_inv = None
            return tensors, self

        def restore_from_saved(self, tensors):
            self._rowwise_data, self._columnwise_data = tensors[0], tensors[1]
            self._rowwise_scale_inv, self._columnwise_scale_inv = tensors[2], tensors[3]
            return tensors[4:]

        def get_data_tensors(self):
            return self._rowwise_data, self._columnwise_data

        def dequantize(self, *, dtype: torch.dtype = torch.float32) -> torch.Tensor:
            return _FromMXFP4Func.forward(None, self, dtype)

        def size(self, dim: Optional[int] = None) -> Union[torch.Size, int]:
            """Logical shape: rowwise codes [..., K/2] -> [..., K]; columnwise-only
            codes [K, ..., M/2] -> [..., M, K] (diff:506-524)."""
            if self._rowwise_data is not None:
                b = list(self._rowwise_data.size())
                shape = b[:-1] + [b[-1] * 2]
            elif self._columnwise_data is not None:
                warnings.warn("Attempting to get shape of MXFP4 tensor with only column-wise data.")
                b = list(self._columnwise_data.size())
                shape = b[1:-1] + [b[-1] * 2, b[0]]
            else:
                raise RuntimeError("Attempted to get shape of MXFP4 tensor with no data")
            return torch.Size(shape) if dim is None else shape[dim]

        def view(self, shape: torch.Size):
            cur_shape = self.size()
            if shape is None or shape == cur_shape:
                return self
            shape = _canonical_shape(shape, cur_shape)
            row, col = _reshaped_data(self, shape, cur_shape, "view")
            return MXFP4TensorBase(rowwise_data=row, rowwise_scale_inv=self._rowwise_scale_inv, columnwise_data=col,
                                   columnwise_scale_inv=self._columnwise_scale_inv, quantizer=self._quantizer,
                                   fp8_dtype=self._fp8_dtype)

        def __repr__(self):
            return f"MXFP4TensorBase(rowwise_scaled_data={self.dequantize()},rowwise_scale_inv={self._rowwise_scale_inv},)"

        def update_usage(self, rowwise_usage: Optional[bool] = None, columnwise_usage: Optional[bool] = None):
            """Drop a usage, or check that a requested one is present; a missing
            usage is never recreated (diff:593-637)."""
            if rowwise_usage is None:
                rowwise_usage = self._rowwise_data is not None
            if columnwise_usage is None:
                columnwise_usage = self._columnwise_data is not None
            if rowwise_usage:
                if self._rowwise_data is None:
                    raise RuntimeError("Requested row-wise usage, but MXFP4Tensor is missing row-scaled MXFP4 data")
                if self._rowwise_scale_inv is None:
                    raise RuntimeError("Requested row-wise usage, but MXFP4Tensor is missing row-scaled scale-inverses")
            else:
                self._rowwise_data = None
                self._rowwise_scale_inv = None
            if columnwise_usage:
                if self._columnwise_data is None:
                    raise RuntimeError(
                        "Requested column-wise usage, but MXFP4Tensor is missing column-scaled MXFP4 data")
                if self._columnwise_scale_inv is None:
                    raise RuntimeError(
                        "Requested column-wise usage, but MXFP4Tensor is missing column-scaled scale-inverses")
            else:
                self._columnwise_data = None
                self._columnwise_scale_inv = None


    class MXFP4Quantizer(Quantizer):
        """Builds MXFP4 tensors: 1x32 blocks along the last dimension (rowwise)
        and along the flattened leading dimensions (columnwise), E8M0 scales,
        eps 1e-10 (diff:676-906). The RHT, 2-D, stochastic-rounding and
        amax-reduction options are stored and, as in the reference, not applied."""

        def __init__(self, fp8_dtype=DEFAULT_FP8_DTYPE, rowwise: bool = True, columnwise: bool = True,
                     with_amax_reduction: bool = False, amax_reduction_group=None, with_rht: bool = False,
                     with_post_rht_amax: bool = False, with_2d_quantization: bool = False,
                     stochastic_rounding: bool = False, with_random_sign_mask: bool = True) -> None:
            super().__init__(rowwise=rowwise, columnwise=columnwise)
            self.dtype = fp8_dtype
            self.with_rht = with_rht
            self.with_post_rht_amax = with_post_rht_amax
            self.with_amax_reduction = with_amax_reduction
            self.amax_reduction_group = amax_reduction_group
            self.with_2d_quantization = with_2d_quantization
            self.stochastic_rounding = stochastic_rounding
            self.with_random_sign_mask = with_random_sign_mask

        def update_quantized(self, src: torch.Tensor, dst: "MXFP4Tensor", *, noop_flag=None) -> "MXFP4Tensor":
            assert isinstance(dst, MXFP4Tensor), f"Cannot store quantized MXFP4 in {type(dst)} type."
            if src.device != dst.device:
                src = src.to(device=dst.device)
            if not src.is_contiguous():
                src = src.contiguous()
            rq, rs, cq, cs = _quantize_pairs(src, True, dst._columnwise_data is not None)
            dst._rowwise_data, dst._rowwise_scale_inv = rq, rs
            if cq is not None:
                dst._columnwise_data, dst._columnwise_scale_inv = cq, cs
            return dst

        def is_quantizable(self, inp: torch.Tensor) -> bool:
            if inp.ndim < 2:
                return False
            if inp.shape[-1] % MXFP4_BLOCK_SCALING_SIZE != 0:
                return False
            return math.prod(inp.shape[:-1]) % MXFP4_BLOCK_SCALING_SIZE == 0

        def get_scale_shape(self, shape: Iterable[int], columnwise: bool) -> Tuple[int, int]:
            """Padded scale shape of ``make_empty``: rowwise (M up to 128,
            ceil(K/32) up to 4), columnwise (K up to 128, ceil(M/32) up to 4)
            with M the product of the leading dimensions (diff:752-787)."""
            M, K = math.prod(shape[:-1]), shape[-1]
            if columnwise:
                return (_round_up(K, 128), _round_up(math.ceil(M / MXFP4_BLOCK_SCALING_SIZE), 4))
            return (_round_up(M, 128), _round_up(math.ceil(K / MXFP4_BLOCK_SCALING_SIZE), 4))

        @staticmethod
        def get_columnwise_shape(shape: Iterable[int]) -> Tuple[int, ...]:
            """(d1, ..., dn) -> (dn, d1, ..., dn-1); () -> ()."""
            shape = tuple(shape)
            return () if len(shape) == 0 else (shape[-1],) + shape[:-1]

        @staticmethod
        def convert_shape_for_fp4(shape: Iterable[int]) -> Tuple[int, ...]:
            shape = list(shape)
            shape[-1] = shape[-1] // 2
            return tuple(shape)

        def make_empty(self, shape: Iterable[int], *, dtype: torch.dtype = torch.float32,
                       device: Optional[torch.device] = None, requires_grad: bool = False) -> "MXFP4Tensor":
            """Uninitialised tensor with the reference's buffer shapes (codes
            unpadded, scales padded as in ``get_scale_shape``; diff:821-881)."""
            if device is None:
                device = torch.device("cuda")
            assert shape[-1] % MXFP4_BLOCK_SCALING_SIZE == 0, (
                f"Incorrect shape {shape} for MXFP4. Tensor dims must be divisible by {MXFP4_BLOCK_SCALING_SIZE}")
            flat_first_dim = math.prod(shape[:-1])
            data = scale_inv = col = col_scale_inv = None
            if self.rowwise_usage:
                data = torch.empty(self.convert_shape_for_fp4(shape), dtype=torch.uint8, device=device)
                scale_inv = torch.empty(self.get_scale_shape(shape, columnwise=False), dtype=torch.uint8, device=device)
            if self.columnwise_usage:
                col = torch.empty(self.convert_shape_for_fp4(self.get_columnwise_shape((flat_first_dim, shape[-1]))),
                                  dtype=torch.uint8, device=device)
                col_scale_inv = torch.empty(self.get_scale_shape(shape, columnwise=True), dtype=torch.uint8,
                                            device=device)
            return MXFP4Tensor(shape=shape, dtype=dtype, rowwise_data=data, rowwise_scale_inv=scale_inv,
                               columnwise_data=col, columnwise_scale_inv=col_scale_inv, fp8_dtype=self.dtype,
                               quantizer=self, requires_grad=requires_grad, device=device)

        def quantize(self, tensor: torch.Tensor, *, out=None, dtype: Optional[torch.dtype] = None):
            if out is not None:
                return self.update_quantized(tensor, out)
            if (not self.internal) and torch.is_grad_enabled():
                return _QuantizeFunc.apply(tensor, self)
            return _QuantizeFunc.forward(None, tensor, self)

        def calibrate(self, tensor: torch.Tensor) -> None:
            pass

        def _get_compatible_recipe(self):
            return None


    # --------------------------------------------------------------------------- tensor
    class MXFP4Tensor(MXFP4TensorBase, QuantizedTensor):
        """A tensor that presents its nominal shape and dtype and holds MXFP4
        data (diff:908-1215)."""

        def __new__(cls, *args, rowwise_data, rowwise_scale_inv, columnwise_data, columnwise_scale_inv, fp8_dtype,
                    quantizer, **kwargs):
            return super().__new__(cls, rowwise_data, rowwise_scale_inv, columnwise_data, columnwise_scale_inv,
                                   fp8_dtype, quantizer, *args, **kwargs)

        def __repr__(self, *, tensor_contents=None):
            return f"MXFP4Tensor, data={self.dequantize(dtype=self.dtype)})"

        def dequantize(self, *, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
            if dtype is None:
                dtype = self.dtype
            if torch.is_grad_enabled():
                return _FromMXFP4Func.apply(self, dtype)
            return _FromMXFP4Func.forward(None, self, dtype)

        def _get_quantizer(self) -> Quantizer:
            return self._quantizer if self._quantizer is not None else MXFP4Quantizer()

        def quantize_(self, tensor: torch.Tensor, *, noop_flag=None) -> "MXFP4Tensor":
            if isinstance(tensor, QuantizedTensor):
                return self.quantize_(tensor.dequantize())
            self._get_quantizer().update_quantized(tensor, self, noop_flag=noop_flag)
            return self

        def detach(self) -> "MXFP4Tensor":
            return MXFP4Tensor.make_like(self)

        def clone(self) -> "MXFP4Tensor":
            assert self._rowwise_data is not None
            meta = self.get_metadata()
            meta["rowwise_data"] = self._rowwise_data.detach().clone()
            if self._columnwise_data is not None:
                meta["columnwise_data"] = self._columnwise_data.detach().clone()
            return MXFP4Tensor(shape=self.shape, dtype=self.dtype, requires_grad=self.requires_grad, **meta)

        def view(self, *shape) -> "MXFP4Tensor":
            return _ViewFunc.apply(self, shape)

        def reshape(self, *shape) -> "MXFP4Tensor":
            return _ReshapeFunc.apply(self, shape)

        def contiguous(self, memory_format: torch.memory_format = torch.contiguous_format) -> "MXFP4Tensor":
            if self._rowwise_data is not None and self._rowwise_data.is_contiguous(memory_format=memory_format):
                return self
            if self._columnwise_data is not None and self._columnwise_data.is_contiguous(memory_format=memory_format):
                return self
            raise ValueError("MXFP4Tensor does not support different memory formats!")

        @classmethod
        def __torch_dispatch__(cls, func, types, args, kwargs=None):
            if func == aten.view.default:
                tensor, shape = args[0], args[1]
                if len(args) != 2:
                    raise RuntimeError(f"Unexpected args for view op (expected 2 args, got {len(args)})")
                return tensor.detach() if shape == tensor.size() else tensor.view(shape)
            if func == aten.zero_.default:
                # codes 0 and scale bytes 1, the values the reference picks (diff:1075-1078)
                tensor = args[0]
                for d, s in ((tensor._rowwise_data, tensor._rowwise_scale_inv),
                             (tensor._columnwise_data, tensor._columnwise_scale_inv)):
                    if d is not None:
                        d.zero_()
                        s.fill_(1)
                return tensor
            if func == aten.empty_like.default:
                tensor = args[0]
                row = rs = col = cs = None
                if tensor._rowwise_data is not None:
                    row, rs = torch.empty_like(tensor._rowwise_data), torch.empty_like(tensor._rowwise_scale_inv)
                if tensor._columnwise_data is not None:
                    col, cs = torch.empty_like(tensor._columnwise_data), torch.empty_like(tensor._columnwise_scale_inv)
                return MXFP4Tensor(shape=tensor.shape, dtype=tensor.dtype, fp8_dtype=tensor._fp8_dtype, rowwise_data=row,
                                   rowwise_scale_inv=rs, columnwise_data=col, columnwise_scale_inv=cs,
                                   quantizer=tensor._quantizer, requires_grad=tensor.requires_grad,
                                   device=tensor.device)
            return super().__torch_dispatch__(func, types, args, kwargs)

        @classmethod
        def _make_in_reduce_ex(cls, shape, rowwise_data, rowwise_scale_inv, columnwise_data, columnwise_scale_inv,
                               amax_rowwise, amax_columnwise, fp8_dtype, dtype, quantizer) -> "MXFP4Tensor":
            """Rebuild for unpickling; MXFP4 keeps no amax, so both amax slots
            arrive as None."""
            device = next((t.device for t in (rowwise_data, columnwise_data) if t is not None), None)
            return MXFP4Tensor(shape=shape, dtype=dtype, fp8_dtype=fp8_dtype, rowwise_data=rowwise_data,
                               rowwise_scale_inv=rowwise_scale_inv, columnwise_data=columnwise_data,
                               columnwise_scale_inv=columnwise_scale_inv, quantizer=quantizer, requires_grad=False,
                               device=device)

        def __reduce_ex__(self, protocol: int) -> tuple:
            return (MXFP4Tensor._make_in_reduce_ex,
                    (self.shape, self._rowwise_data, self._rowwise_scale_inv, self._columnwise_data,
                     self._columnwise_scale_inv, None, None, self._fp8_dtype, self.dtype, self._quantizer))

        def _get_data(self) -> "MXFP4Tensor":
            return super().data

        @torch.no_grad()
        def _set_data(self, tensor: torch.Tensor) -> None:
            """``.data = t``: take t's MXFP4 buffers when t is an MXFP4Tensor,
            else quantize t into this tensor (diff:1167-1215)."""
            new_device = tensor.device if tensor.is_cuda else self.device
            if tensor.device != new_device:
                tensor = tensor.to(device=new_device)
            if isinstance(tensor, MXFP4Tensor):
                if (self.size() != tensor.size() or self.stride() != tensor.stride()
                        or self.storage_offset() != tensor.storage_offset() or self.dtype != tensor.dtype
                        or self.layout != tensor.layout or self.device != new_device):
                    dummy = torch.Tensor._make_wrapper_subclass(MXFP4Tensor, tensor.size(), strides=tensor.stride(),
                                                                storage_offset=tensor.storage_offset(),
                                                                dtype=tensor.dtype, layout=tensor.layout,
                                                                requires_grad=tensor.requires_grad, device=new_device)
                    super(MXFP4Tensor, type(self)).data.__set__(self, dummy)
                self._rowwise_data = tensor._rowwise_data
                self._columnwise_data = tensor._columnwise_data
                self._quantizer = tensor._quantizer
                self._rowwise_scale_inv = tensor._rowwise_scale_inv
                self._columnwise_scale_inv = tensor._columnwise_scale_inv
                return
            assert self._quantizer is not None, "Can't quantize without a quantizer"
            self._quantizer.update_quantized(tensor, self)
            if self.requires_grad != tensor.requires_grad:
                self.requires_grad_(requires_grad=tensor.requires_grad)

        data = property(_get_data, _set_data)


    class _ViewFunc(torch.autograd.Function):
        """View of an MXFP4Tensor (inner dimension fixed); backward views the
        gradient back (diff:1219-1333)."""

        @staticmethod
        def forward(ctx, tensor: MXFP4Tensor, shape=None) -> MXFP4Tensor:
            cur_shape = tensor.shape
            if ctx is not None:
                ctx.shape = cur_shape
            if shape is None:
                return tensor
            shape = _canonical_shape(shape, cur_shape)
            row, col = _reshaped_data(tensor, shape, cur_shape, "view")
            return MXFP4Tensor(shape, tensor.dtype, rowwise_data=row, rowwise_scale_inv=tensor._rowwise_scale_inv,
                               columnwise_data=col, columnwise_scale_inv=tensor._columnwise_scale_inv,
                               quantizer=tensor._quantizer, fp8_dtype=tensor._fp8_dtype,
                               requires_grad=tensor.requires_grad, device=tensor.device)

        @staticmethod
        def backward(ctx, grad):
            return _reshape_grad(ctx.shape, grad, "view"), None


    class _ReshapeFunc(torch.autograd.Function):
        """Reshape of an MXFP4Tensor; like the view but through ``reshape`` on
        the code tensors (diff:1335-1446)."""

        @staticmethod
        def forward(ctx, tensor: MXFP4Tensor, shape=None) -> MXFP4Tensor:
            ctx.shape = tensor.shape
            if shape is None:
                return tensor
            shape = _canonical_shape(shape, ctx.shape)
            row, col = _reshaped_data(tensor, shape, ctx.shape, "reshape")
            return MXFP4Tensor(shape, tensor.dtype, rowwise_data=row, rowwise_scale_inv=tensor._rowwise_scale_inv,
                               columnwise_data=col, columnwise_scale_inv=tensor._columnwise_scale_inv,
                               quantizer=tensor._quantizer, fp8_dtype=tensor._fp8_dtype,
                               requires_grad=tensor.requires_grad, device=tensor.device)

        @staticmethod
        def backward(ctx, grad):
            return _reshape_grad(ctx.shape, grad, "reshape"), None


    def _reshape_grad(shape, grad, op: str):
        if isinstance(grad, MXFP4Tensor):
            row, col = _reshaped_data(grad, list(shape), list(shape), op)
            return MXFP4Tensor(shape, grad.dtype, rowwise_data=row, rowwise_scale_inv=grad._rowwise_scale_inv,
                               columnwise_data=col, columnwise_scale_inv=grad._columnwise_scale_inv,
                               quantizer=grad._quantizer, fp8_dtype=grad._fp8_dtype, requires_grad=grad.requires_grad,
                               device=grad.device)
        return grad.view(shape)


    class _QuantizeFunc(torch.autograd.Function):
        """High precision -> MXFP4Tensor; the gradient passes through unchanged
        (diff:1448-1480)."""

        @staticmethod
        def forward(_ctx, tensor: torch.Tensor, quantizer: MXFP4Quantizer) -> MXFP4Tensor:
            rq, rs, cq, cs = _quantize_pairs(tensor, quantizer.rowwise_usage, quantizer.columnwise_usage)
            dst = MXFP4Tensor(shape=tensor.shape, dtype=tensor.dtype, rowwise_data=rq, rowwise_scale_inv=rs,
                              columnwise_data=cq, columnwise_scale_inv=cs, fp8_dtype=quantizer.dtype,
                              quantizer=quantizer, requires_grad=tensor.requires_grad, device=tensor.device)
            dst._is_2D_scaled = quantizer.with_2d_quantization
            return dst

        @staticmethod
        def backward(_ctx, grad: torch.Tensor):
            return grad, None

    for c in (MXFP4TensorBase, MXFP4Quantizer, MXFP4Tensor):
        c.__name__ = c.__qualname__ = name_prefix + c.__name__
        c.__module__ = __name__
        globals()[c.__name__] = c
    return SimpleNamespace(MXFP4TensorBase=MXFP4TensorBase, MXFP4Quantizer=MXFP4Quantizer,
                           MXFP4Tensor=MXFP4Tensor, _FromMXFP4Func=_FromMXFP4Func, _ViewFunc=_ViewFunc,
                           _ReshapeFunc=_ReshapeFunc, _QuantizeFunc=_QuantizeFunc)


_default = build_mxfp4_classes()
MXFP4TensorBase = _default.MXFP4TensorBase
MXFP4Quantizer = _default.MXFP4Quantizer
MXFP4Tensor = _default.MXFP4Tensor
_FromMXFP4Func = _default._FromMXFP4Func
_ViewFunc = _default._ViewFunc
_ReshapeFunc = _default._ReshapeFunc
_QuantizeFunc = _default._QuantizeFunc


def bind_to_te(te_quantizer=None, te_quantized_tensor=None, te_quantized_tensor_base=None):
    """The MXFP4 classes derived from TE's own base classes, built once per
    set of bases and registered here as ``TEMXFP4TensorBase`` /
    ``TEMXFP4Quantizer`` / ``TEMXFP4Tensor``. With no arguments the bases are
    imported from an installed transformer_engine (``Quantizer`` and
    ``QuantizedTensor`` from ``transformer_engine.pytorch.tensor.quantized_tensor``,
    ``QuantizedTensorBase`` from the same module where it exists); an
    ImportError means TE is not installed and the restated classes above are
    the ones to use.

    One set of bases per process: the registered names are what pickles
    record, so a second binding on other bases would make the first family's
    instances unpicklable; it raises RuntimeError instead. Loading a pickled
    TE-bound tensor in a new process needs bind_to_te() to have run first."""
    if te_quantizer is None or te_quantized_tensor is None:
        from transformer_engine.pytorch.tensor import quantized_tensor as _te_qt  # noqa: F401
        te_quantizer = te_quantizer or _te_qt.Quantizer
        te_quantized_tensor = te_quantized_tensor or _te_qt.QuantizedTensor
        if te_quantized_tensor_base is None:
            te_quantized_tensor_base = getattr(_te_qt, "QuantizedTensorBase", None)
    key = (te_quantizer, te_quantized_tensor, te_quantized_tensor_base)
    if key not in _TE_BOUND:
        if _TE_BOUND:
            raise RuntimeError("bind_to_te: the TE-bound MXFP4 classes already exist on other base classes; "
                               "their registered names (TEMXFP4Tensor, ...) can name only one family per process")
        _TE_BOUND[key] = build_mxfp4_classes(te_quantizer, te_quantized_tensor, te_quantized_tensor_base or object,
                                             name_prefix="TE")
    return _TE_BOUND[key]


_TE_BOUND: Dict[tuple, SimpleNamespace] = {}
