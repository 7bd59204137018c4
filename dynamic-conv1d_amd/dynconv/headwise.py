"""Headwise dynamic short convolution on MI355X (drop-in for the reference's headwise.py).

Same public function, signature, preconditions and autograd semantics as
headwise.py:218-337; the Triton launches are replaced by calls into
libdynconv.so (dc_headwise_fwd / dc_headwise_bwd).
"""

import torch

from . import _capi


class _HeadwiseDynamicConvolutionFn(torch.autograd.Function):
    """Autograd glue; mirrors headwise.py:218-309."""

    @staticmethod
    @_capi.on_tensor_device
    def forward(ctx, x, weight, static_w, residual):
        B, T, D = x.shape
        H = weight.shape[2]
        W = weight.shape[-1]
        assert D % H == 0, f"D={D} must be divisible by H={H}"
        y = torch.empty_like(x)
        lib = _capi.load()
        status = lib.dc_headwise_fwd(
            _capi.ptr(x), _capi.ptr(weight), _capi.ptr(static_w), _capi.ptr(y),
            B, T, D, H, W, _capi.dtype_code(x.dtype), int(bool(residual)), _capi.stream_of(x),
        )
        _capi.check(status, "headwise forward")
        ctx.save_for_backward(x, weight, static_w)
        ctx.residual = bool(residual)
        return y

    @staticmethod
    @_capi.on_tensor_device
    def backward(ctx, dy):
        dy = dy.contiguous()
        x, weight, static_w = ctx.saved_tensors
        B, T, D = x.shape
        H = weight.shape[2]
        W = weight.shape[-1]
        has_static = static_w is not None
        dtype = _capi.dtype_code(x.dtype)
        if dy.dtype != x.dtype:
            dy = dy.to(x.dtype)
        dx = torch.empty_like(x)
        dweight = torch.empty_like(weight)
        dstatic_w = torch.empty_like(static_w) if has_static else None
        lib = _capi.load()
        ws_bytes = lib.dc_headwise_bwd_ws_bytes(B, T, D, H, W, dtype, int(has_static))
        _capi.check(int(ws_bytes) if ws_bytes < 0 else 0, "headwise backward workspace query")
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes > 0 else None
        status = lib.dc_headwise_bwd(
            _capi.ptr(x), _capi.ptr(weight), _capi.ptr(static_w), _capi.ptr(dy),
            _capi.ptr(dx), _capi.ptr(dweight), _capi.ptr(dstatic_w), _capi.ptr(ws), ws_bytes,
            B, T, D, H, W, dtype, int(ctx.residual), _capi.stream_of(x),
        )
        _capi.check(status, "headwise backward")
        return dx, dweight, dstatic_w, None


def headwise_dynamic_convolution(
    x: torch.Tensor,
    weight: torch.Tensor,
    static_w: torch.Tensor | None = None,
    residual: bool = False,
) -> torch.Tensor:
    """Headwise dynamic causal short convolution, with optional fused (per-channel) static short convolution.

    Args:
        x:          [B, T, D] input activations.
        weight:     [B, T, H, W] per-token (dynamic) convolution weights. D must be divisible by H.
                    Each head spans D // H consecutive channels.
        static_w:   [W, D] optional per-channel static filter added to the dynamic weight at every (b, t).
        residual:   add x to the output.

    Returns:
        y: [B, T, D] with y[b, t, d] = sum_w (weight[b, t, d // head_size, w] + static_w[w, d]) * x[b, t-w, d]
        (+ x[b, t, d] if residual).

    Preconditions as headwise.py:332-336, plus (checked here, assumed by the
    reference) a 4-D weight; a non-contiguous weight is copied.

    weight and static_w may have dtypes other than x's (float32, bfloat16 or
    float16), as in the reference, whose kernels load both in fp32
    (headwise.py:63, 78, 180, 187) and return dweight in weight's dtype and
    dstatic_w in static_w's (headwise.py:268, 305).  Such calls run the
    kernels in float32 on float32 copies (every 16-bit value is exact in
    float32) and round y and each gradient once to its tensor's dtype, as the
    reference stores its fp32 results; one dtype throughout takes no copies.
    """
    assert x.is_cuda and x.is_contiguous()
    if static_w is not None:
        assert static_w.is_cuda and static_w.is_contiguous()
        assert static_w.shape == (weight.shape[-1], x.shape[-1])
        assert static_w.dtype in _FLOATS, "static_w must be float32, bfloat16 or float16"
    assert weight.dim() == 4 and weight.shape[:2] == x.shape[:2], "weight must be [B, T, H, W]"
    assert weight.dtype in _FLOATS, "weight must be float32, bfloat16 or float16"
    assert weight.is_cuda
    if weight.dtype == x.dtype and (static_w is None or static_w.dtype == x.dtype):
        return _HeadwiseDynamicConvolutionFn.apply(x, weight.contiguous(), static_w, residual)
    # mixed dtypes: float32 operands; autograd rounds each gradient back to its input's dtype
    f32 = torch.float32
    sw = None if static_w is None else static_w.to(f32)
    y = _HeadwiseDynamicConvolutionFn.apply(x.to(f32), weight.to(f32).contiguous(), sw, residual)
    return y.to(x.dtype)


_FLOATS = (torch.float32, torch.bfloat16, torch.float16)
