"""Lowrank dynamic short convolution on MI355X (drop-in for the reference's lowrank.py).

Same public function, signature, preconditions and autograd semantics as
lowrank.py:214-338.  The per-token weights z @ U (and the static filter as
the extra rank with z == 1, lowrank.py:223-225) are formed inside the HIP
kernels; neither the padded z nor the concatenated U is materialised.
"""

import torch

from . import _capi


class _LowrankDynamicConvolutionFn(torch.autograd.Function):
    """Autograd glue; mirrors lowrank.py:214-299."""

    @staticmethod
    def forward(ctx, x, z, U, static_w, residual):
        B, T, D = x.shape
        R = z.shape[-1]
        W = U.shape[-1] // D
        y = torch.empty_like(x)
        lib = _capi.load()
        status = lib.dc_lowrank_fwd(
            _capi.ptr(x), _capi.ptr(z), _capi.ptr(U), _capi.ptr(static_w), _capi.ptr(y),
            B, T, D, R, W, _capi.dtype_code(x.dtype), int(bool(residual)), _capi.stream_of(x),
        )
        _capi.check(status, "lowrank forward")
        ctx.save_for_backward(x, z, U, static_w)
        ctx.residual = bool(residual)
        return y

    @staticmethod
    def backward(ctx, dy):
        dy = dy.contiguous()
        x, z, U, static_w = ctx.saved_tensors
        B, T, D = x.shape
        R = z.shape[-1]
        W = U.shape[-1] // D
        has_static = static_w is not None
        dtype = _capi.dtype_code(x.dtype)
        if dy.dtype != x.dtype:
            dy = dy.to(x.dtype)
        dx = torch.empty_like(x)
        dz = torch.empty_like(z)
        dU = torch.empty_like(U)
        dstatic_w = torch.empty_like(static_w) if has_static else None
        lib = _capi.load()
        ws_bytes = lib.dc_lowrank_bwd_ws_bytes(B, T, D, R, W, dtype, int(has_static))
        _capi.check(int(ws_bytes) if ws_bytes < 0 else 0, "lowrank backward workspace query")
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes > 0 else None
        status = lib.dc_lowrank_bwd(
            _capi.ptr(x), _capi.ptr(z), _capi.ptr(U), _capi.ptr(static_w), _capi.ptr(dy),
            _capi.ptr(dx), _capi.ptr(dz), _capi.ptr(dU), _capi.ptr(dstatic_w), _capi.ptr(ws), ws_bytes,
            B, T, D, R, W, dtype, int(ctx.residual), _capi.stream_of(x),
        )
        _capi.check(status, "lowrank backward")
        return dx, dz, dU, dstatic_w, None


def lowrank_dynamic_convolution(
    x: torch.Tensor,
    z: torch.Tensor,
    U: torch.Tensor,
    static_w: torch.Tensor | None = None,
    residual: bool = False,
) -> torch.Tensor:
    """Lowrank dynamic short convolution, with optional fused (per-channel) static short convolution.

    The dynamic convolution weights z @ U are produced on chip from the low-rank inputs.

    Args:
        x:          [B, T, D] input activations.
        z:          [B, T, R] hidden states after the first projection of the low-rank factorization.
        U:          [R, W*D] second projection of the low-rank factorization, viewed as (R, W, D).
        static_w:   [W, D] optional per-channel static filter added to the dynamic weight at every (b, t).
                    It is fused as one extra rank, so a rank-R dynamic + static convolution costs about
                    as much as a rank-(R+1) dynamic convolution.
        residual:   add x to the output.

    Returns:
        y: [B, T, D] with y[b, t, d] = sum_w (sum_r z[b, t, r] * U[r, w*D + d] + static_w[w, d]) * x[b, t-w, d]
        (+ x[b, t, d] if residual).

    Preconditions as lowrank.py:328-337, plus (checked here, assumed by the
    reference) one shared dtype for x, z and U and W*D columns in U.
    """
    assert x.is_cuda and x.is_contiguous()
    assert z.is_cuda and z.is_contiguous()
    assert U.is_cuda and U.is_contiguous()
    R = z.shape[-1]
    R_kernel = R + 1 if static_w is not None else R  # static_w is fused into dynamic convolution using one rank
    assert R_kernel & (R_kernel - 1) == 0, "rank R must be a power of 2. If static_w is set R+1 must be a power of 2."
    if static_w is not None:
        assert static_w.is_cuda and static_w.is_contiguous()
        assert static_w.dtype == z.dtype == U.dtype
        assert static_w.shape == (U.shape[-1] // x.shape[-1], x.shape[-1])
    assert x.dim() == 3 and z.dim() == 3 and z.shape[:2] == x.shape[:2], "z must be [B, T, R]"
    assert U.dim() == 2 and U.shape[0] == R and U.shape[1] % x.shape[-1] == 0, "U must be [R, W*D]"
    assert x.dtype == z.dtype == U.dtype, "x, z and U must share one dtype"
    return _LowrankDynamicConvolutionFn.apply(x, z, U, static_w, residual)
