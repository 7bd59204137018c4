"""nn.Modules around the lowrank operator (README.md:55-110).

LowRankDynamicShortConvolution is the README's module (README.md:57-83): a
rank-R dynamic filter z = proj_in(pre_z) with U = proj_out, plus the static
filter proj_out_bias fused as rank R+1.

GroupedLowRankDynamicShortConvolution holds G such modules (the q, k and v
convolutions of README.md:86-110) and runs them as one grouped operator: one
proj_in GEMM for all groups, and one launch per direction that reads the fused
[B, T, G*D] projection in place instead of three .contiguous() slices.
"""

import math

import torch
from torch import nn

from .lowrank import lowrank_dynamic_convolution, lowrank_dynamic_convolution_grouped


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
        z = self.proj_in(pre_z)
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
        z = self.proj_in(pre_z)  # [B, T, G*R]: one GEMM for every group
        zs = [z[..., g * R:(g + 1) * R].contiguous() for g in range(G)]
        Us = [self.proj_out[g] for g in range(G)]
        sws = [self.proj_out_bias[g] for g in range(G)]
        return lowrank_dynamic_convolution_grouped(x, zs, Us, static_w=sws, residual=True, head_dim=self.head_dim)
