"""nn.Modules around the lowrank operator (README.md:55-110).

LowRankDynamicShortConvolution is the README's module (README.md:57-83): a
rank-R dynamic filter z = proj_in(pre_z) with U = proj_out, plus the static
filter proj_out_bias fused as rank R+1.

GroupedLowRankDynamicShortConvolution holds G such modules (the q, k and v
convolutions of README.md:86-110) and runs them as one grouped operator: one
proj_in GEMM for all groups, and one launch per direction that reads the fused
[B, T, G*D] projection in place instead of three .contiguous() slices.

The proj_in GEMM (README.md:67, 75) runs on libdynconv.so's own matrix-core
kernels (dc_proj_in_fwd / dc_proj_in_bwd): skinny products bound by streaming
pre_z, which the library GEMM runs at about a quarter of HBM bandwidth in the
backward.  Shapes those kernels do not take (fp32, G*R > 128, d_model % 8 != 0,
non-contiguous pre_z) use torch's GEMM (F.linear).  A proj_in that is not a
plain bias-free nn.Linear (a subclass or wrapper in its place), one with hooks,
and calls under autocast run the layer itself, as the reference module does.
"""

import math

import torch
import torch.nn.functional as F
from torch import nn

from . import _capi
from .lowrank import lowrank_dynamic_convolution, lowrank_dynamic_convolution_grouped


class _ProjInFn(torch.autograd.Function):
    """z_g = (pre_z @ W_in^T)[..., g*R:(g+1)*R] for g < G, as G contiguous tensors, and its backward."""

    @staticmethod
    @_capi.on_tensor_device
    def forward(ctx, pre_z, w_in, G, R):
        B, T, K = pre_z.shape
        M = B * T
        zs = [torch.empty(B, T, R, dtype=pre_z.dtype, device=pre_z.device) for _ in range(G)]
        lib = _capi.load()
        status = lib.dc_proj_in_fwd(_capi.ptr(pre_z), _capi.ptr(w_in), _capi.ptr_array(zs), G, M, K, R,
                                    _capi.dtype_code(pre_z.dtype), _capi.stream_of(pre_z))
        _capi.check(status, "proj_in forward")
        ctx.save_for_backward(pre_z, w_in)
        ctx.G, ctx.R = G, R
        return tuple(zs)

    @staticmethod
    @_capi.on_tensor_device
    def backward(ctx, *dzs):
        pre_z, w_in = ctx.saved_tensors
        G, R = ctx.G, ctx.R
        B, T, K = pre_z.shape
        M = B * T
        dzs = [torch.zeros(B, T, R, dtype=pre_z.dtype, device=pre_z.device) if d is None
               else d.to(pre_z.dtype).contiguous() for d in dzs]
        dpre = torch.empty_like(pre_z)
        dw = torch.empty_like(w_in)
        lib = _capi.load()
        dtype = _capi.dtype_code(pre_z.dtype)
        nws = lib.dc_proj_in_bwd_ws_bytes(G, M, K, R, dtype)
        _capi.check(int(nws) if nws < 0 else 0, "proj_in backward workspace query")
        ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=pre_z.device)
        status = lib.dc_proj_in_bwd(_capi.ptr(pre_z), _capi.ptr(w_in), _capi.ptr_array(dzs), _capi.ptr(dpre),
                                    _capi.ptr(dw), _capi.ptr(ws), nws, G, M, K, R, dtype, _capi.stream_of(pre_z))
        _capi.check(status, "proj_in backward")
        return dpre, dw, None, None


def _proj_in_native(pre_z, w_in, G, R) -> bool:
    """Whether the library's proj_in kernels take this call (else torch's GEMM)."""
    return (pre_z.is_cuda and pre_z.dim() == 3 and pre_z.dtype in (torch.bfloat16, torch.float16)
            and w_in.dtype == pre_z.dtype and pre_z.is_contiguous() and w_in.is_contiguous()
            and G * R <= 128 and pre_z.shape[-1] % 8 == 0
            and pre_z.data_ptr() % 16 == 0 and w_in.data_ptr() % 16 == 0)


def _plain_linear(m: nn.Module) -> bool:
    """Whether m is exactly an nn.Linear whose call is just F.linear(input, weight): no
    subclass or wrapper in its place (adapters, quantised layers) and no hooks on it or
    installed globally, so that calling the library kernel instead changes nothing a
    caller could observe."""
    return (type(m) is nn.Linear and m.bias is None and not m._forward_hooks and not m._forward_pre_hooks
            and not m._backward_hooks and not getattr(m, "_backward_pre_hooks", None)
            and not nn.modules.module._global_forward_hooks
            and not nn.modules.module._global_forward_pre_hooks
            and not nn.modules.module._global_backward_hooks)


def _module_proj_in(layer: nn.Module, pre_z: torch.Tensor, G: int, R: int):
    """The modules' z: the library's proj_in kernels when calling them is indistinguishable
    from calling `layer` (a plain bias-free nn.Linear, no hooks, autocast off), else the
    layer itself, as the reference module does (README.md:67, 75)."""
    if _plain_linear(layer) and not torch.is_autocast_enabled(pre_z.device.type):
        return proj_in(pre_z, layer.weight, G, R)
    z = layer(pre_z)
    return tuple(z[..., g * R:(g + 1) * R].contiguous() for g in range(G))


def proj_in(pre_z: torch.Tensor, w_in: torch.Tensor, G: int, R: int):
    """The modules' proj_in GEMM for G groups: a tuple of G contiguous [B, T, R] tensors,
    group g being pre_z @ w_in[g*R:(g+1)*R].T (README.md:67, 75)."""
    if _proj_in_native(pre_z, w_in, G, R):
        return _ProjInFn.apply(pre_z, w_in, G, R)
    z = F.linear(pre_z, w_in)
    return tuple(z[..., g * R:(g + 1) * R].contiguous() for g in range(G))


def _check_rank(R: int) -> None:
    # fused bias term is an additional rank (README.md:64-65)
    if ((R + 1) & R) != 0:
        raise ValueError("R+1 must be a power of two")


class LowRankDynamicShortConvolution(nn.Module):
    """Low-rank dynamic short convolution with bias term, as README.md:57-83."""

    def __init__(self, d_model: int, R: int, W: int):
        super().__init__()
        _check_rank(R)
        self.d_model, self.R, self.W = d_model, R, W
        self.proj_in = nn.Linear(d_model, R, bias=False)
        self.proj_out = nn.Parameter(torch.zeros(R, W * d_model))
        self.proj_out_bias = nn.Parameter(torch.empty(W, d_model))
        nn.init.uniform_(self.proj_out_bias, -1.0 / math.sqrt(W), +1.0 / math.sqrt(W))

    def forward(self, x: torch.Tensor, pre_z: torch.Tensor) -> torch.Tensor:
        (z,) = _module_proj_in(self.proj_in, pre_z, 1, self.R)
        return lowrank_dynamic_convolution(
            x=x.contiguous(),
            z=z.contiguous(),
            U=self.proj_out,
            static_w=self.proj_out_bias,
            residual=True,
        )


class GroupedLowRankDynamicShortConvolution(nn.Module):
    """G LowRankDynamicShortConvolution modules of one shape run as one grouped operator.

    forward(x, pre_z) takes x = [B, T, G*d_model] (e.g. c_attn(x_norm), the fused
    q|k|v projection of README.md:99-104) and returns G tensors [B, T, d_model],
    group g being what a LowRankDynamicShortConvolution with parameters
    (proj_in.weight[g*R:(g+1)*R], proj_out[g], proj_out_bias[g]) returns for
    x[..., g*d_model:(g+1)*d_model].  With head_dim set the outputs come as
    [B, d_model // head_dim, T, head_dim] (README.md:106-110's
    .view(B, T, H, head_dim).transpose(1, 2), written directly).
    """

    def __init__(self, d_model: int, R: int, W: int, groups: int = 3, head_dim=None):
        super().__init__()
        _check_rank(R)
        if not 1 <= groups <= 4:
            raise ValueError("groups must be between 1 and 4")
        if head_dim is not None and (head_dim <= 0 or d_model % head_dim != 0):
            raise ValueError("head_dim must divide d_model")
        self.d_model, self.R, self.W, self.groups, self.head_dim = d_model, R, W, groups, head_dim
        self.proj_in = nn.Linear(d_model, groups * R, bias=False)
        self.proj_out = nn.Parameter(torch.zeros(groups, R, W * d_model))
        self.proj_out_bias = nn.Parameter(torch.empty(groups, W, d_model))
        nn.init.uniform_(self.proj_out_bias, -1.0 / math.sqrt(W), +1.0 / math.sqrt(W))

    def forward(self, x: torch.Tensor, pre_z: torch.Tensor):
        G, R = self.groups, self.R
        zs = list(_module_proj_in(self.proj_in, pre_z, G, R))  # one GEMM for every group
        Us = [self.proj_out[g] for g in range(G)]
        sws = [self.proj_out_bias[g] for g in range(G)]
        return lowrank_dynamic_convolution_grouped(x, zs, Us, static_w=sws, residual=True, head_dim=self.head_dim)
