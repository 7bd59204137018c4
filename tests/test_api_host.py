"""Precondition behaviour of the Python API, checked without a GPU.

The reference raises AssertionError for violated preconditions
(headwise.py:332-336, lowrank.py:328-337); the drop-in keeps that.
"""

import pytest
import torch

import headwise
import lowrank


def test_import_paths_match_reference():
    assert callable(headwise.headwise_dynamic_convolution)
    assert callable(lowrank.lowrank_dynamic_convolution)
    assert issubclass(headwise._HeadwiseDynamicConvolutionFn, torch.autograd.Function)
    assert issubclass(lowrank._LowrankDynamicConvolutionFn, torch.autograd.Function)


def test_headwise_requires_device_tensor():
    x = torch.randn(1, 4, 8)
    w = torch.randn(1, 4, 8, 2)
    with pytest.raises(AssertionError):
        headwise.headwise_dynamic_convolution(x, w)


def test_lowrank_requires_device_tensor():
    x = torch.randn(1, 4, 8)
    z = torch.randn(1, 4, 4)
    U = torch.randn(4, 16)
    with pytest.raises(AssertionError):
        lowrank.lowrank_dynamic_convolution(x, z, U)


def test_signatures():
    import inspect

    s = inspect.signature(headwise.headwise_dynamic_convolution)
    assert list(s.parameters) == ["x", "weight", "static_w", "residual"]
    assert s.parameters["static_w"].default is None and s.parameters["residual"].default is False
    s = inspect.signature(lowrank.lowrank_dynamic_convolution)
    assert list(s.parameters) == ["x", "z", "U", "static_w", "residual"]


def test_device_guard_passes_through_on_cpu():
    """The autograd Functions' device guard (dynconv._capi.on_tensor_device): with no CUDA tensor
    among the arguments it only forwards the call, arguments and result unchanged."""
    from dynconv import _capi

    seen = []

    @_capi.on_tensor_device
    def fn(ctx, *args):
        seen.append((ctx, args))
        return "result"

    t = torch.zeros(3)
    assert fn("ctx", None, t, 4) == "result"
    assert seen == [("ctx", (None, t, 4))]
    assert fn.__name__ == "fn"


def test_module_proj_in_keeps_the_layer_semantics():
    """The modules call the library's proj_in kernels only where that is indistinguishable from
    calling self.proj_in (README.md:67, 75): a plain bias-free nn.Linear without hooks, autocast off.
    A forward hook on the layer, or a subclass in its place, makes them call the layer itself."""
    from torch import nn

    from dynconv.modules import _module_proj_in, _plain_linear

    layer = nn.Linear(16, 6, bias=False)
    assert _plain_linear(layer)
    pre_z = torch.randn(2, 5, 16)
    calls = []
    h = layer.register_forward_hook(lambda mod, inp, out: calls.append(out.shape))
    assert not _plain_linear(layer)
    zs = _module_proj_in(layer, pre_z, 2, 3)
    h.remove()
    assert calls == [torch.Size([2, 5, 6])]
    ref = pre_z @ layer.weight.t()
    assert all(z.is_contiguous() for z in zs)
    torch.testing.assert_close(torch.cat(zs, -1), ref)

    class Scaled(nn.Linear):  # e.g. an adapter: its forward is not F.linear
        def forward(self, inp):
            return 2 * super().forward(inp)

    sub = Scaled(16, 6, bias=False)
    assert not _plain_linear(sub)
    (z,) = _module_proj_in(sub, pre_z, 1, 6)
    torch.testing.assert_close(z, 2 * (pre_z @ sub.weight.t()))
    assert not _plain_linear(nn.Linear(16, 6, bias=True))
