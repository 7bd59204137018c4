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
