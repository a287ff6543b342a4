"""TE-facing MXFP4 tensor and quantizer (omo_python_api.mxfp4_tensor).

CPU tests cover the host logic the reference defines in
code/transformer_engine-2.8.diff:346-1480 (buffer shapes, views, usage
updates, dispatch of empty_like / zero_ / detach, pickling); they hold uint8
buffers on the CPU and launch nothing. GPU tests check that the quantizer's
buffers equal the reference composition (rowwise quantize of x, rowwise
quantize of x.T.contiguous(), diff:1460-1466) byte for byte, and against the
oracle on a small case, and exercise dequantize, autograd, quantize_ and the
dequantize-and-run default of __torch_dispatch__.
"""
import io
import pickle

import numpy as np
import pytest
import torch

from helpers import bits_u16, bits_u8


def _mx():
    from omo_python_api import mxfp4_tensor
    return mxfp4_tensor


# ------------------------------------------------------------------ CPU: host logic
def test_quantizer_shapes():
    mx = _mx()
    q = mx.MXFP4Quantizer()
    assert q.rowwise_usage and q.columnwise_usage and not q.internal
    # rowwise (M up to 128, ceil(K/32) up to 4); columnwise (K up to 128, ceil(M/32) up to 4)
    assert q.get_scale_shape((300, 96), columnwise=False) == (384, 4)
    assert q.get_scale_shape((300, 96), columnwise=True) == (128, 12)
    assert q.get_scale_shape((2, 3, 64), columnwise=False) == (128, 4)
    assert q.get_scale_shape((4096, 7168), columnwise=True) == (7168, 128)
    assert mx.MXFP4Quantizer.get_columnwise_shape((2, 3, 4)) == (4, 2, 3)
    assert mx.MXFP4Quantizer.get_columnwise_shape(()) == ()
    assert mx.MXFP4Quantizer.convert_shape_for_fp4((5, 64)) == (5, 32)
    assert q.is_quantizable(torch.empty(64, 32))
    assert not q.is_quantizable(torch.empty(64))
    assert not q.is_quantizable(torch.empty(64, 48))
    assert not q.is_quantizable(torch.empty(40, 32))
    q.set_usage(columnwise=False)
    assert q.rowwise_usage and not q.columnwise_usage
    c = q.copy()
    c.set_usage(rowwise=False)
    assert q.rowwise_usage and not c.rowwise_usage


def test_make_empty_buffers():
    mx = _mx()
    t = mx.MXFP4Quantizer().make_empty((4, 64, 96), dtype=torch.bfloat16, device="cpu")
    assert isinstance(t, mx.MXFP4Tensor) and t.shape == (4, 64, 96) and t.dtype == torch.bfloat16
    assert t._rowwise_data.shape == (4, 64, 48) and t._rowwise_scale_inv.shape == (256, 4)
    assert t._columnwise_data.shape == (96, 128) and t._columnwise_scale_inv.shape == (128, 8)
    r = mx.MXFP4Quantizer(rowwise=True, columnwise=False).make_empty((64, 32), device="cpu")
    assert r._columnwise_data is None and r._columnwise_scale_inv is None and r.dtype == torch.float32
    with pytest.raises(AssertionError):
        mx.MXFP4Quantizer().make_empty((64, 48), device="cpu")


def _cpu_tensor(M=256, K=64, columnwise=True):
    mx = _mx()
    g = torch.Generator().manual_seed(M * 7 + K)
    row = torch.randint(0, 256, (M, K // 2), dtype=torch.uint8, generator=g)
    rs = torch.randint(0, 256, (M, K // 32), dtype=torch.uint8, generator=g)
    col = torch.randint(0, 256, (K, M // 2), dtype=torch.uint8, generator=g) if columnwise else None
    cs = torch.randint(0, 256, (K, M // 32), dtype=torch.uint8, generator=g) if columnwise else None
    return mx.MXFP4Tensor(shape=(M, K), dtype=torch.bfloat16, rowwise_data=row, rowwise_scale_inv=rs,
                          columnwise_data=col, columnwise_scale_inv=cs, fp8_dtype=mx.DEFAULT_FP8_DTYPE,
                          quantizer=mx.MXFP4Quantizer(), device="cpu")


def test_view_and_reshape():
    mx = _mx()
    t = _cpu_tensor()
    v = t.view(4, 64, 64)
    assert isinstance(v, mx.MXFP4Tensor) and v.shape == (4, 64, 64)
    assert v._rowwise_data.shape == (4, 64, 32) and v._columnwise_data.shape == (64, 128)
    assert v._rowwise_data.data_ptr() == t._rowwise_data.data_ptr()
    assert t.view(-1, 8, 64).shape == (32, 8, 64)
    assert t.reshape((2, -1, 64)).shape == (2, 128, 64)
    assert t.view(torch.Size([256, 64])).shape == (256, 64)
    with pytest.raises(RuntimeError, match="inner dimension"):
        t.view(128, 128)
    # the base class views its buffers the same way and returns itself for its own shape
    b = mx.MXFP4TensorBase(t._rowwise_data, t._rowwise_scale_inv, t._columnwise_data, t._columnwise_scale_inv,
                           mx.DEFAULT_FP8_DTYPE, None)
    assert b.size() == (256, 64) and b.size(0) == 256 and b.view((256, 64)) is b
    assert b.view((8, 32, 64))._rowwise_data.shape == (8, 32, 32)
    with pytest.warns(UserWarning):
        c = mx.MXFP4TensorBase(None, None, t._columnwise_data, t._columnwise_scale_inv, mx.DEFAULT_FP8_DTYPE, None)
        assert c.size() == (256, 64)
    with pytest.raises(RuntimeError, match="no data"):
        mx.MXFP4TensorBase(None, None, None, None, mx.DEFAULT_FP8_DTYPE, None).size()


def test_view_backward_restores_shape():
    t = _cpu_tensor()
    t.requires_grad_(True)
    g = torch.ones(4, 64, 64)
    for op in ("view", "reshape"):
        (back,) = torch.autograd.grad(getattr(t, op)(4, 64, 64), t, g)
        assert back.shape == (256, 64)


def test_update_usage_and_saving():
    t = _cpu_tensor()
    with pytest.raises(RuntimeError, match="column-wise"):
        _cpu_tensor(columnwise=False).update_usage(columnwise_usage=True)
    t.update_usage(rowwise_usage=True, columnwise_usage=False)
    assert t._columnwise_data is None and t._columnwise_scale_inv is None and t._rowwise_data is not None
    t = _cpu_tensor()
    saved, obj = t.prepare_for_saving()
    assert obj is t and t._rowwise_data is None and len(saved) == 4
    assert t.restore_from_saved(saved + ["rest"]) == ["rest"]
    assert t._rowwise_data is saved[0] and t._columnwise_scale_inv is saved[3]
    row, col = t.get_data_tensors()
    assert row is saved[0] and col is saved[1]
    meta = t.get_metadata()
    assert set(meta) == {"rowwise_data", "rowwise_scale_inv", "columnwise_data", "columnwise_scale_inv",
                         "fp8_dtype", "quantizer"}
    t.clear()
    assert t._rowwise_data.numel() == 0 and t._columnwise_scale_inv.numel() == 0


def test_dispatch_without_kernels():
    mx = _mx()
    t = _cpu_tensor()
    e = torch.empty_like(t)
    assert isinstance(e, mx.MXFP4Tensor) and e._rowwise_data.shape == t._rowwise_data.shape
    assert e._rowwise_data.data_ptr() != t._rowwise_data.data_ptr()
    d = t.detach()
    assert isinstance(d, mx.MXFP4Tensor) and d._rowwise_data is t._rowwise_data and d.shape == t.shape
    z = t.zero_()
    assert z is t
    assert int(t._rowwise_data.count_nonzero()) == 0 and int(t._columnwise_data.count_nonzero()) == 0
    assert bool((t._rowwise_scale_inv == 1).all()) and bool((t._columnwise_scale_inv == 1).all())
    assert t.contiguous() is t


def test_pickle_round_trip():
    mx = _mx()
    t = _cpu_tensor()
    for s in (pickle.loads(pickle.dumps(t)), _torch_save_load(t)):
        assert isinstance(s, mx.MXFP4Tensor) and s.shape == t.shape and s.dtype == t.dtype
        assert torch.equal(s._rowwise_data, t._rowwise_data)
        assert torch.equal(s._columnwise_scale_inv, t._columnwise_scale_inv)
        assert s._fp8_dtype == t._fp8_dtype and s._quantizer.columnwise_usage


class _StandInTE:
    """Stand-ins for TE's Quantizer / QuantizedTensor / QuantizedTensorBase:
    the constructor signatures TE's bases have, and a generic
    __torch_dispatch__ that records which ops reach it."""

    class Quantizer:
        def __init__(self, *, rowwise: bool = True, columnwise: bool = True):
            self.rowwise_usage, self.columnwise_usage, self.internal = rowwise, columnwise, False

        def copy(self):
            import copy
            return copy.copy(self)

        def __call__(self, tensor):
            return self.quantize(tensor)

    class QuantizedTensorBase:
        def get_usages(self):
            return {"rowwise": self._rowwise_data is not None, "columnwise": self._columnwise_data is not None}

    class QuantizedTensor(torch.Tensor):
        seen = []
        result = torch.full((1,), 7.0)

        def __new__(cls, shape, dtype, *, requires_grad=False, device=None):
            return torch.Tensor._make_wrapper_subclass(cls, shape, dtype=dtype, requires_grad=requires_grad,
                                                       device=device)

        @classmethod
        def make_like(cls, tensor, *, shape=None, dtype=None, requires_grad=False, data=None):
            return cls(shape=tensor.shape if shape is None else shape, dtype=tensor.dtype if dtype is None else dtype,
                       requires_grad=requires_grad, device=tensor.device, **tensor.get_metadata())

        @classmethod
        def __torch_dispatch__(cls, func, types, args, kwargs=None):
            cls.seen.append(func)
            return cls.result

        __torch_function__ = torch._C._disabled_torch_function_impl


def test_bind_to_te_bases():
    """The class family rebuilt on TE-like bases: isinstance against each
    base, the MXFP4 ops handled before the base's generic __torch_dispatch__,
    every other op routed to it, and pickling of the bound class."""
    mx = _mx()
    te = _StandInTE
    ns = mx.bind_to_te(te.Quantizer, te.QuantizedTensor, te.QuantizedTensorBase)
    assert mx.bind_to_te(te.Quantizer, te.QuantizedTensor, te.QuantizedTensorBase) is ns
    q = ns.MXFP4Quantizer(rowwise=True, columnwise=True)
    assert isinstance(q, te.Quantizer) and not isinstance(q, mx.Quantizer)
    t = q.make_empty((256, 64), dtype=torch.bfloat16, device="cpu")
    assert type(t) is ns.MXFP4Tensor and type(t).__name__ == "TEMXFP4Tensor"
    assert isinstance(t, te.QuantizedTensor) and isinstance(t, te.QuantizedTensorBase)
    assert isinstance(t, ns.MXFP4TensorBase) and not isinstance(t, mx.MXFP4Tensor)
    assert t.get_usages() == {"rowwise": True, "columnwise": True}
    assert t._rowwise_data.shape == (256, 32) and t._columnwise_data.shape == (64, 128)
    e = torch.empty_like(t)                                # handled by MXFP4Tensor
    assert type(e) is ns.MXFP4Tensor and e._columnwise_scale_inv.shape == t._columnwise_scale_inv.shape
    assert t.zero_() is t and int(t._rowwise_data.count_nonzero()) == 0
    assert type(t.detach()) is ns.MXFP4Tensor
    te.QuantizedTensor.seen.clear()
    assert torch.ops.aten.add.Tensor(t, t) is te.QuantizedTensor.result  # anything else goes to the base
    assert te.QuantizedTensor.seen == [torch.ops.aten.add.Tensor]
    tensors, obj = t.prepare_for_saving()
    assert obj is t and len(tensors) == 4 and t._rowwise_data is None
    t.restore_from_saved(tensors + ["rest"])
    s = pickle.loads(pickle.dumps(t))
    assert type(s) is ns.MXFP4Tensor and torch.equal(s._rowwise_data, t._rowwise_data)
    # the module's default family is untouched
    assert not isinstance(mx.MXFP4Quantizer(), te.Quantizer)


def test_bind_to_te_refuses_other_bases():
    """A second binding on different bases would re-register TEMXFP4Tensor and
    break pickling of the first family's instances: it raises, and the first
    family still round-trips through pickle."""
    mx = _mx()
    te = _StandInTE
    ns = mx.bind_to_te(te.Quantizer, te.QuantizedTensor, te.QuantizedTensorBase)

    class OtherQuantizer(te.Quantizer):
        pass

    with pytest.raises(RuntimeError, match="already exist"):
        mx.bind_to_te(OtherQuantizer, te.QuantizedTensor, te.QuantizedTensorBase)
    assert mx.bind_to_te(te.Quantizer, te.QuantizedTensor, te.QuantizedTensorBase) is ns
    t = ns.MXFP4Quantizer(rowwise=True, columnwise=False).make_empty((64, 32), dtype=torch.bfloat16, device="cpu")
    s = pickle.loads(pickle.dumps(t))
    assert type(s) is ns.MXFP4Tensor and torch.equal(s._rowwise_data, t._rowwise_data)


def test_bind_to_te_without_te():
    """With no bases given the TE package is imported; it is absent here."""
    mx = _mx()
    try:
        import transformer_engine  # noqa: F401
        pytest.skip("transformer_engine is installed")
    except ImportError:
        pass
    with pytest.raises(ImportError):
        mx.bind_to_te()


def _torch_save_load(t):
    buf = io.BytesIO()
    torch.save(t, buf)
    buf.seek(0)
    return torch.load(buf, weights_only=False)  # written by this test a line above


# ------------------------------------------------------------------ GPU: HIP path
def _x(M, K, seed, dev):
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(M, K, generator=g) * torch.exp2(torch.randint(-6, 7, (M, K), generator=g).float())
    return x.to(torch.bfloat16).to(dev)


@pytest.mark.gpu
@pytest.mark.parametrize("M,K", [(64, 96), (256, 1024), (4096, 7168)])
def test_quantize_both_usages_equals_reference_composition(dev, M, K):
    from omo_python_api.mxfp4 import omo_per_token_group_quant_mxfp4
    mx = _mx()
    x = _x(M, K, M + K, dev)
    t = mx.MXFP4Quantizer()(x)
    assert isinstance(t, mx.MXFP4Tensor) and t.shape == (M, K) and t.dtype == torch.bfloat16
    rq, rs = omo_per_token_group_quant_mxfp4(x)
    cq, cs = omo_per_token_group_quant_mxfp4(x.T.contiguous())
    torch.cuda.synchronize()
    for got, exp in ((t._rowwise_data, rq), (t._rowwise_scale_inv, rs), (t._columnwise_data, cq),
                     (t._columnwise_scale_inv, cs)):
        assert got.shape == exp.shape
        assert torch.equal(got, exp)


@pytest.mark.gpu
def test_quantize_against_oracle(dev, oracle):
    mx = _mx()
    x = _x(96, 192, 11, dev)  # the dequant wrapper needs K % 64 == 0 (mxfp4_dequant.py:51-53)
    t = mx.MXFP4Quantizer()(x)
    xb = bits_u16(x)
    q, s = oracle.quant_mxfp4(xb.reshape(-1))
    qt, st = oracle.quant_mxfp4(np.ascontiguousarray(xb.T).reshape(-1))
    np.testing.assert_array_equal(bits_u8(t._rowwise_data).reshape(-1), q)
    np.testing.assert_array_equal(bits_u8(t._rowwise_scale_inv).reshape(-1), s)
    np.testing.assert_array_equal(bits_u8(t._columnwise_data).reshape(-1), qt)
    np.testing.assert_array_equal(bits_u8(t._columnwise_scale_inv).reshape(-1), st)
    # dequantize (rowwise kernel) against the oracle's dequant of the same codes
    np.testing.assert_array_equal(bits_u16(t.dequantize()).reshape(-1), oracle.dequant_bf16(q, s))


@pytest.mark.gpu
def test_single_usage_and_errors(dev):
    from omo_python_api.mxfp4 import omo_per_token_group_quant_mxfp4
    mx = _mx()
    x = _x(128, 256, 5, dev)
    r = mx.MXFP4Quantizer(rowwise=True, columnwise=False)(x)
    assert r._columnwise_data is None and torch.equal(r._rowwise_data, omo_per_token_group_quant_mxfp4(x)[0])
    c = mx.MXFP4Quantizer(rowwise=False, columnwise=True)(x)
    assert c._rowwise_data is None
    assert torch.equal(c._columnwise_data, omo_per_token_group_quant_mxfp4(x.T.contiguous())[0])
    with pytest.raises(NotImplementedError, match="column-wise"):
        c.dequantize()
    # rowwise-only quantize of rows that are not a multiple of 32 is fine; columnwise needs them
    y = _x(40, 64, 6, dev)
    assert mx.MXFP4Quantizer(rowwise=True, columnwise=False)(y)._rowwise_data.shape == (40, 32)
    with pytest.raises(AssertionError):
        mx.MXFP4Quantizer()(y)


@pytest.mark.gpu
def test_autograd_and_dispatch(dev):
    from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4ToBf16_dequant_wrapper
    mx = _mx()
    x = _x(64, 128, 7, dev).requires_grad_(True)
    t = mx.MXFP4Quantizer(rowwise=True, columnwise=False)(x)
    assert t.requires_grad and t.grad_fn is not None
    y = t.dequantize()
    assert y.dtype == torch.bfloat16
    expect = omo_per_token_mxfp4ToBf16_dequant_wrapper(t._rowwise_data, t._rowwise_scale_inv, dtype=torch.bfloat16)
    assert torch.equal(y, expect)
    (y.float() * 3.0).sum().backward()
    assert torch.equal(x.grad, torch.full_like(x, 3.0))
    with torch.no_grad():
        assert torch.equal(t + 1.0, expect + 1.0)  # default dispatch: dequantize, then run
        assert torch.equal(torch.matmul(t.float(), torch.ones(128, 2, device=dev)),
                           torch.matmul(expect.float(), torch.ones(128, 2, device=dev)))
        assert torch.equal(t.dequantize(dtype=torch.float32), expect.float())


@pytest.mark.gpu
def test_quantize_into_existing_refreshes_both_usages(dev):
    from omo_python_api.mxfp4 import omo_per_token_group_quant_mxfp4
    mx = _mx()
    q = mx.MXFP4Quantizer()
    x1, x2, x3 = _x(128, 256, 1, dev), _x(128, 256, 2, dev), _x(128, 256, 3, dev)
    t = q(x1)
    t.quantize_(x2)
    assert torch.equal(t._rowwise_data, omo_per_token_group_quant_mxfp4(x2)[0])
    assert torch.equal(t._columnwise_data, omo_per_token_group_quant_mxfp4(x2.T.contiguous())[0])
    assert torch.equal(t._columnwise_scale_inv, omo_per_token_group_quant_mxfp4(x2.T.contiguous())[1])
    t.copy_(x3)  # aten.copy_ quantizes into the tensor
    assert torch.equal(t._rowwise_data, omo_per_token_group_quant_mxfp4(x3)[0])
    t.data = x1  # .data = high precision quantizes too
    assert torch.equal(t._columnwise_data, omo_per_token_group_quant_mxfp4(x1.T.contiguous())[0])
    out = q.make_empty((128, 256), dtype=torch.bfloat16, device=dev)
    assert q.quantize(x2, out=out) is out and torch.equal(out._rowwise_data, omo_per_token_group_quant_mxfp4(x2)[0])
    with torch.no_grad():
        before = t.dequantize()
        t.mul_(2.0)  # in-place op: dequantize, multiply, quantize back
    assert torch.equal(t._rowwise_data, omo_per_token_group_quant_mxfp4(before * 2.0)[0])
    assert torch.equal(t._columnwise_data, omo_per_token_group_quant_mxfp4((before * 2.0).T.contiguous())[0])
    c = t.clone()
    assert c._rowwise_data.data_ptr() != t._rowwise_data.data_ptr() and torch.equal(c._rowwise_data, t._rowwise_data)
    s = pickle.loads(pickle.dumps(t))
    assert s.device == t.device and torch.equal(s._columnwise_data, t._columnwise_data)
