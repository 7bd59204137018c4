"""HIP graph capture of the operators: forward + backward recorded once with torch.cuda.graph,
replayed on new inputs copied into the captured tensors, each replay bitwise equal to the same
step run eagerly.

The entry points launch on torch's current stream, allocate nothing outside torch's allocator
and record no memset nodes (outputs, partial sums and the padded z_eff copy are written whole by
kernels), so a training or serving step that captures them replays them.  Between replays the
test runs the eager step and synchronises, as a program would; every replay is compared, not only
the first.  Shapes are small; the launch plans are those of any other call of the same shape.
"""

import math

import pytest
import torch

from helpers import gen, randn, uniform
import headwise as hw_mod
import lowrank as lr_mod

pytestmark = pytest.mark.gpu

DEV = "cuda"
hw = hw_mod.headwise_dynamic_convolution
lr = lr_mod.lowrank_dynamic_convolution
lr_grouped = lr_mod.lowrank_dynamic_convolution_grouped


def _hw_case(Bn, Tn, Dn, H, W, static, dtype):
    def inputs(g):
        return [randn(g, Bn, Tn, Dn), randn(g, Bn, Tn, H, W, scale=1 / math.sqrt(W)),
                uniform(g, W, Dn, lo=-0.5, hi=0.5) if static else None]

    return inputs, (lambda x, w, s: hw(x, w, s, residual=True)), dtype, (Bn, Tn, Dn)


def _lr_case(Bn, Tn, Dn, R, W, static, dtype):
    def inputs(g):
        return [randn(g, Bn, Tn, Dn), randn(g, Bn, Tn, R), randn(g, R, W * Dn, scale=1 / math.sqrt((R + 1) * W)),
                uniform(g, W, Dn, lo=-0.5, hi=0.5) if static else None]

    return inputs, (lambda x, z, U, s: lr(x, z, U, s, residual=True)), dtype, (Bn, Tn, Dn)


def _grouped_case(G, Bn, Tn, Dn, R, W, head_dim, dtype):
    def inputs(g):
        t = [randn(g, Bn, Tn, G * Dn)]
        t += [randn(g, Bn, Tn, R) for _ in range(G)]
        t += [randn(g, R, W * Dn, scale=1 / math.sqrt((R + 1) * W)) for _ in range(G)]
        t += [uniform(g, W, Dn, lo=-0.5, hi=0.5) for _ in range(G)]
        return t

    def fn(x, *rest):
        zs, Us, ss = rest[:G], rest[G:2 * G], rest[2 * G:]
        return lr_grouped(x, list(zs), list(Us), list(ss), residual=True, head_dim=head_dim)

    shape = (Bn, Dn // head_dim, Tn, head_dim) if head_dim else (Bn, Tn, Dn)
    return inputs, fn, dtype, shape


CASES = {
    "hw_hs1": _hw_case(2, 300, 256, 256, 4, True, torch.bfloat16),
    "hw_hs32_fp16": _hw_case(2, 300, 512, 16, 4, True, torch.float16),
    "hw_hs8_fp32": _hw_case(1, 200, 256, 32, 3, False, torch.float32),
    "lr_r16": _lr_case(2, 300, 256, 16, 4, False, torch.bfloat16),          # z read directly
    "lr_r15s_fp16": _lr_case(2, 300, 256, 15, 4, True, torch.float16),      # padded z_eff from the forward
    "lr_r31s_w8": _lr_case(1, 200, 256, 31, 8, True, torch.bfloat16),       # two passes of taps
    "lr_r16_fp32": _lr_case(2, 300, 256, 16, 4, False, torch.float32),
    "lr_grouped_hd64": _grouped_case(3, 2, 200, 128, 15, 4, 64, torch.bfloat16),
    "lr_r15s_w20": _lr_case(1, 200, 256, 15, 20, True, torch.bfloat16),     # forward passes, fp32 dx rounded once
    "hw_hs4_w24": _hw_case(1, 200, 256, 64, 24, True, torch.bfloat16),      # wide kernels, one channel per lane
    "hw_hs32_w12": _hw_case(2, 300, 256, 8, 12, True, torch.bfloat16),      # head matrix-core kernels
    "lr_r127s": _lr_case(1, 200, 256, 127, 4, True, torch.bfloat16),        # passes of kernel ranks
    "lr_r16_w40": _lr_case(1, 100, 128, 16, 40, False, torch.float16),      # W 40: generic kernels
}


def _step(fn, leaves, dys):
    out = fn(*leaves)
    outs = list(out) if isinstance(out, (list, tuple)) else [out]
    grads = torch.autograd.grad(outs, [t for t in leaves if t is not None], dys)
    return outs + list(grads)


# the warm-up's autograd nodes ran on the side stream: torch notes the stream change, harmlessly
@pytest.mark.filterwarnings("ignore:The AccumulateGrad node's stream")
@pytest.mark.parametrize("name", list(CASES))
def test_graph_replays_match_eager(name):
    inputs, fn, dtype, yshape = CASES[name]
    g = gen(len(name) * 7919 + 13)
    leaves = [t.to(dtype).to(DEV).requires_grad_() if t is not None else None for t in inputs(g)]
    nout = 3 if name.startswith("lr_grouped") else 1
    dys = [randn(g, *yshape).to(dtype).to(DEV) for _ in range(nout)]

    # warm-up on a side stream (library handles, allocator), then capture
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            _step(fn, leaves, dys)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = _step(fn, leaves, dys)
    torch.cuda.synchronize()

    for rep in range(3):
        with torch.no_grad():
            for t, new in zip(leaves, inputs(g)):
                if t is not None:
                    t.copy_(new.to(dtype))
            for d in dys:
                d.copy_(randn(g, *yshape).to(dtype))
        graph.replay()
        eager = _step(fn, leaves, dys)
        torch.cuda.synchronize()
        assert len(eager) == len(captured)
        for i, (a, b) in enumerate(zip(captured, eager)):
            assert torch.equal(a, b), (name, rep, i, (a.float() - b.float()).abs().max().item())
