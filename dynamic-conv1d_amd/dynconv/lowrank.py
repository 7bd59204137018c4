"""Lowrank dynamic short convolution on MI355X (drop-in for the reference's lowrank.py).

Same public function, signature, preconditions and autograd semantics as
lowrank.py:214-338.  The per-token weights z @ U (and the static filter as
the extra rank with z == 1, lowrank.py:223-225) are formed inside the HIP
kernels; the concatenated U is never materialised.  Where the backward's
matrix-core kernel reads z through a padded copy (static column included:
with static_w, or an odd rank), the forward writes that copy as a by-product
and keeps it for the backward (dc_lowrank_zeff_bytes), instead of the backward
building it in a launch of its own.
"""

import torch

from . import _capi


def _zeff_buffers(lib, n, B, T, D, R, W, dtype, has_static, device):
    """(n buffers for the forward's padded z copy, their size), or (None, 0) when the backward reads z itself."""
    nb = lib.dc_lowrank_zeff_bytes(B, T, D, R, W, dtype, int(has_static))
    _capi.check(int(nb) if nb < 0 else 0, "lowrank z_eff size query")
    if nb <= 0:
        return None, 0
    return [torch.empty(nb, dtype=torch.uint8, device=device) for _ in range(n)], nb


class _LowrankDynamicConvolutionFn(torch.autograd.Function):
    """Autograd glue; mirrors lowrank.py:214-299."""

    @staticmethod
    @_capi.on_tensor_device
    def forward(ctx, x, z, U, static_w, residual):
        B, T, D = x.shape
        R = z.shape[-1]
        W = U.shape[-1] // D
        y = torch.empty_like(x)
        lib = _capi.load()
        dtype = _capi.dtype_code(x.dtype)
        # the padded z copy only serves a backward: none when no input needs a gradient (inference)
        zeffs, nzeff = (_zeff_buffers(lib, 1, B, T, D, R, W, dtype, static_w is not None, x.device)
                        if any(ctx.needs_input_grad) else (None, 0))
        zeff = zeffs[0] if zeffs else None
        status = lib.dc_lowrank_fwd(
            _capi.ptr(x), _capi.ptr(z), _capi.ptr(U), _capi.ptr(static_w), _capi.ptr(y), _capi.ptr(zeff), nzeff,
            B, T, D, R, W, dtype, int(bool(residual)), _capi.stream_of(x),
        )
        _capi.check(status, "lowrank forward")
        ctx.save_for_backward(x, z, U, static_w)
        ctx.zeff = zeff  # internal buffer, a function of z: kept on ctx like the reference's padded z
        ctx.nzeff = nzeff
        ctx.residual = bool(residual)
        return y

    @staticmethod
    @_capi.on_tensor_device
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
            _capi.ptr(x), _capi.ptr(z), _capi.ptr(U), _capi.ptr(static_w), _capi.ptr(ctx.zeff), ctx.nzeff,
            _capi.ptr(dy),
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


class _GroupedLowrankDynamicConvolutionFn(torch.autograd.Function):
    """G lowrank convolutions of one shape in one launch per direction.

    x is [B, T, G*D] (a fused projection, read in place: rows may be further
    apart than G*D); group g convolves its columns g*D .. g*D+D-1.  The
    backward writes the gradient of x as one [B, T, G*D] tensor, so the
    README's .contiguous() copies (README.md:76-78) and the concatenation of
    dq, dk, dv do not happen.
    """

    @staticmethod
    @_capi.on_tensor_device
    def forward(ctx, x, residual, G, has_static, hd, *params):
        zs, Us = params[:G], params[G:2 * G]
        sws = params[2 * G:3 * G] if has_static else None
        B, T, C = x.shape
        D = C // G
        R = zs[0].shape[-1]
        W = Us[0].shape[-1] // D
        shape = (B, T, D) if hd == 0 else (B, D // hd, T, hd)
        ys = [torch.empty(shape, dtype=x.dtype, device=x.device) for _ in range(G)]
        lib = _capi.load()
        dtype = _capi.dtype_code(x.dtype)
        zeffs, nzeff = (_zeff_buffers(lib, G, B, T, D, R, W, dtype, has_static, x.device)
                        if any(ctx.needs_input_grad) else (None, 0))
        status = lib.dc_lowrank_fwd_grouped(
            G, _capi.ptr(x), x.stride(1), _capi.ptr_array(zs), _capi.ptr_array(Us), _capi.ptr_array(sws),
            _capi.ptr_array(ys), _capi.ptr_array(zeffs), nzeff, hd, B, T, D, R, W, dtype, int(bool(residual)),
            _capi.stream_of(x),
        )
        _capi.check(status, "grouped lowrank forward")
        ctx.save_for_backward(x, *params)
        ctx.zeffs, ctx.nzeff = zeffs, nzeff
        ctx.G, ctx.has_static, ctx.residual, ctx.hd = G, has_static, bool(residual), hd
        return tuple(ys)

    @staticmethod
    @_capi.on_tensor_device
    def backward(ctx, *dys):
        x, *params = ctx.saved_tensors
        G, has_static = ctx.G, ctx.has_static
        zs, Us = params[:G], params[G:2 * G]
        sws = params[2 * G:3 * G] if has_static else None
        B, T, C = x.shape
        D = C // G
        R = zs[0].shape[-1]
        W = Us[0].shape[-1] // D
        dtype = _capi.dtype_code(x.dtype)
        hd = ctx.hd
        # an output that did not reach the loss has no gradient: it contributes zeros
        shape = (B, T, D) if hd == 0 else (B, D // hd, T, hd)
        dys = [torch.zeros(shape, dtype=x.dtype, device=x.device) if d is None else d.to(x.dtype).contiguous()
               for d in dys]
        dx = torch.empty(B, T, C, dtype=x.dtype, device=x.device)
        dzs = [torch.empty_like(z) for z in zs]
        dUs = [torch.empty_like(U) for U in Us]
        dsws = [torch.empty_like(s) for s in sws] if has_static else None
        lib = _capi.load()
        ws_bytes = lib.dc_lowrank_bwd_grouped_ws_bytes(G, B, T, D, R, W, dtype, int(has_static))
        _capi.check(int(ws_bytes) if ws_bytes < 0 else 0, "grouped lowrank backward workspace query")
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes > 0 else None
        status = lib.dc_lowrank_bwd_grouped(
            G, _capi.ptr(x), x.stride(1), _capi.ptr_array(zs), _capi.ptr_array(Us), _capi.ptr_array(sws),
            _capi.ptr_array(ctx.zeffs), ctx.nzeff, _capi.ptr_array(dys), hd, _capi.ptr(dx), C, _capi.ptr_array(dzs),
            _capi.ptr_array(dUs),
            _capi.ptr_array(dsws), _capi.ptr(ws), ws_bytes, B, T, D, R, W, dtype, int(ctx.residual),
            _capi.stream_of(x),
        )
        _capi.check(status, "grouped lowrank backward")
        return (dx, None, None, None, None, *dzs, *dUs, *(dsws or []))


def lowrank_dynamic_convolution_grouped(
    x: torch.Tensor,
    z,
    U,
    static_w=None,
    residual: bool = False,
    head_dim=None,
):
    """G lowrank dynamic short convolutions of one shape, e.g. on the q, k and v of an attention layer.

    Equivalent to
        [lowrank_dynamic_convolution(x[..., g*D:(g+1)*D].contiguous(), z[g], U[g], static_w[g], residual)
         for g in range(G)]
    (README.md:57-110), computed by one launch per direction with x read in place.  With head_dim
    set, each output is written head-major, as
        y.view(B, T, D // head_dim, head_dim).transpose(1, 2).contiguous()
    (README.md:106-110): the layout attention reads, produced by the kernel's own stores.

    Args:
        x:          [B, T, G*D] activations, e.g. the fused q|k|v projection.  Channels must be
                    contiguous (stride 1); rows may be further apart (a column slice of a wider tensor).
        z:          G tensors [B, T, R], contiguous.
        U:          G tensors [R, W*D], contiguous.
        static_w:   None, or G tensors [W, D] fused as one extra rank each.
        residual:   add each group's input to its output.
        head_dim:   None for [B, T, D] outputs, or a head dim hd (D % hd == 0) for contiguous
                    [B, D // hd, T, hd] outputs.  hd a multiple of 64 keeps the fast kernels of
                    every dtype (bitwise the values of the [B, T, D] layout); other head dims
                    take slower kernels in some cases.

    Returns:
        a tuple of G tensors [B, T, D] (or [B, D // head_dim, T, head_dim]).

    Per group, the preconditions of lowrank_dynamic_convolution (lowrank.py:328-337); G <= 4.
    """
    z, U = list(z), list(U)
    G = len(z)
    assert 1 <= G <= 4, "between 1 and 4 groups"
    assert len(U) == G, "one U per group"
    has_static = static_w is not None
    if has_static:
        static_w = list(static_w)
        assert len(static_w) == G, "one static_w per group"
    assert x.is_cuda and x.dim() == 3 and x.shape[-1] % G == 0, "x must be [B, T, G*D]"
    if x.stride(2) != 1 or x.stride(0) != x.shape[1] * x.stride(1):
        x = x.contiguous()
    B, T, C = x.shape
    D = C // G
    R = z[0].shape[-1]
    R_kernel = R + 1 if has_static else R
    assert R_kernel & (R_kernel - 1) == 0, "rank R must be a power of 2. If static_w is set R+1 must be a power of 2."
    for g in range(G):
        assert z[g].is_cuda and z[g].is_contiguous()
        assert U[g].is_cuda and U[g].is_contiguous()
        assert z[g].dim() == 3 and tuple(z[g].shape) == (B, T, R), "every z must be [B, T, R]"
        assert U[g].dim() == 2 and U[g].shape[0] == R and U[g].shape[1] % D == 0, "U must be [R, W*D]"
        assert U[g].shape == U[0].shape, "every U must have one shape"
        assert x.dtype == z[g].dtype == U[g].dtype, "x, z and U must share one dtype"
        if has_static:
            s = static_w[g]
            assert s.is_cuda and s.is_contiguous()
            assert s.dtype == z[g].dtype == U[g].dtype
            assert s.shape == (U[g].shape[-1] // D, D)
    hd = 0 if head_dim is None else int(head_dim)
    assert hd == 0 or (0 < hd <= D and D % hd == 0), "head_dim must divide D"
    params = z + U + (static_w if has_static else [])
    return _GroupedLowrankDynamicConvolutionFn.apply(x, residual, G, has_static, hd, *params)
