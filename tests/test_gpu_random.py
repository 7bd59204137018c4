"""GPU parity on seeded random shapes: the HIP kernels against the CPU oracle.

Each case draws B, T, D, the head size (headwise) or rank (lowrank), W,
static_w, residual and dtype from a fixed seed, so every dispatch path meets
shapes nobody picked by hand: the vector / MFMA kernels with partial channel
chunks and tiles, the lowrank passes of taps and of ranks (kernel ranks 33-256, and W 9-32), the
8-wavefront forward workgroups, the headwise wide
kernels (W 9-16), the fp32 matrix-core and VALU kernels, and the generic
kernels (D not a multiple of the vector width, head sizes that are not a power
of two, ranks and W outside the fast plans).  Criterion: the north-star
tolerance (tests/helpers.py) against the fp32 oracle on the same
dtype-rounded inputs.  Ranks the Python API rejects (kernel rank not a power
of two) go through the autograd Function directly, the C ABI's general case.
"""

import math
import random

import pytest
import torch

from helpers import assert_ns, check_reductions, gen, randn, run_fwd_bwd, uniform
from oracle.reference_cpu import (
    headwise_dynamic_convolution_ref as hw_ref,
    lowrank_dynamic_convolution_ref as lr_ref,
)
import headwise as hw_mod
import lowrank as lr_mod
from dynconv import lowrank as dlr

pytestmark = pytest.mark.gpu

DEV = "cuda"
DTYPES = [torch.bfloat16, torch.float16, torch.float32]
D_CHOICES = [4, 8, 12, 16, 24, 40, 64, 96, 128, 136, 200, 256, 272, 320]


def _to(t, dtype):
    return None if t is None else t.to(dtype).to(DEV)


def _lowrank_case(i):
    rnd = random.Random(7919 * i + 17)
    dtype = rnd.choice(DTYPES)
    Bn = rnd.randint(1, 3)
    Tn = rnd.choice([1, 2, 3, 5, 15, 16, 17, 31, 33, 64, 100, 129, 200])
    Dn = rnd.choice(D_CHOICES)
    W = rnd.randint(1, 8)
    static = rnd.random() < 0.5
    R = rnd.randint(1, 31)
    residual = rnd.random() < 0.5
    return Bn, Tn, Dn, R, W, static, residual, dtype


def _headwise_case(i):
    rnd = random.Random(104729 * i + 3)
    dtype = rnd.choice(DTYPES)
    Bn = rnd.randint(1, 3)
    Tn = rnd.choice([1, 2, 4, 7, 16, 33, 64, 100, 129, 200])
    Dn = rnd.choice(D_CHOICES)
    hs = rnd.choice([d for d in range(1, Dn + 1) if Dn % d == 0])
    W = rnd.randint(1, 8)
    static = rnd.random() < 0.5
    residual = rnd.random() < 0.5
    return Bn, Tn, Dn, Dn // hs, W, static, residual, dtype


def _lowrank_wide_case(i):
    """Kernel ranks 33-64 (3-4 rank chunks) at W 1-12 in 16-bit types: the matrix-core backward's
    passes of 32 ranks (49-64 from W 2 on, 33-48 from W 3 on) or its one pass of three or four
    rank chunks, with passes of taps (each pass's dx added to the earlier passes', its dz in slots
    of its own; past four passes in fp32), above W 8 the forward's passes of 8 taps."""
    rnd = random.Random(6113 * i + 29)
    dtype = rnd.choice([torch.bfloat16, torch.float16])
    Bn = rnd.randint(1, 2)
    Tn = rnd.choice([1, 15, 16, 17, 33, 64, 100, 129])
    Dn = rnd.choice([16, 64, 128, 144, 256])
    W = rnd.randint(1, 12)
    static = rnd.random() < 0.5
    R = rnd.randint(32, 63) if static else rnd.randint(33, 64)
    residual = rnd.random() < 0.5
    return Bn, Tn, Dn, R, W, static, residual, dtype


def _lowrank_widew_case(i):
    """W 9-32 at kernel ranks up to 32 in 16-bit types: the forward in one pass over up to 16 taps
    (above W 16 two passes, the second added to the first's y), the backward as passes of at most
    4 taps."""
    rnd = random.Random(4099 * i + 7)
    dtype = rnd.choice([torch.bfloat16, torch.float16])
    Bn = rnd.randint(1, 2)
    Tn = rnd.choice([1, 7, 16, 17, 33, 64, 100, 129])
    Dn = rnd.choice([8, 24, 64, 128, 200, 256])
    W = rnd.randint(9, 32)
    static = rnd.random() < 0.5
    R = rnd.randint(1, 31)
    residual = rnd.random() < 0.5
    return Bn, Tn, Dn, R, W, static, residual, dtype


def _headwise_wide_case(i):
    """9 <= W <= 32 with D a multiple of 128 and power-of-two head sizes up to 128: the wide
    row-ring kernels (two channels per lane up to W 16, one above; weight segments staged through
    LDS), or the generic ones where a wavefront's weight segment is not whole 16-byte pieces."""
    rnd = random.Random(3571 * i + 11)
    dtype = rnd.choice(DTYPES)
    Bn = rnd.randint(1, 3)
    Tn = rnd.choice([1, 2, 9, 16, 17, 33, 64, 100, 129, 300])
    Dn = rnd.choice([128, 256, 384, 640])
    hs = rnd.choice([h for h in (1, 2, 4, 8, 16, 32, 64, 128) if Dn % h == 0])
    W = rnd.randint(9, 32)
    static = rnd.random() < 0.5
    residual = rnd.random() < 0.5
    return Bn, Tn, Dn, Dn // hs, W, static, residual, dtype


def _lowrank_big_lds_case(i):
    """Forward shapes whose staged operands exceed 80 KiB (8-wavefront workgroups): W 5-8 at three
    or four rank chunks, W 11-16 at two, and kernel ranks 65-256 at W 1-4 (one pass of up to 128
    ranks, or two); their backward as passes of 32 ranks or of taps."""
    rnd = random.Random(27644437 * i + 1)
    dtype = rnd.choice([torch.bfloat16, torch.float16])
    Bn = rnd.randint(1, 2)
    Tn = rnd.choice([1, 16, 33, 100, 129])
    Dn = rnd.choice([8, 64, 128, 136, 256])
    static = rnd.random() < 0.5
    residual = rnd.random() < 0.5
    k = rnd.randint(0, 2)
    if k == 0:
        W, R = rnd.randint(5, 8), rnd.randint(33, 64)
    elif k == 1:
        W, R = rnd.randint(11, 16), rnd.randint(17, 32)
    else:
        W, R = rnd.randint(1, 4), rnd.randint(65, 256)
    R = max(1, min(R - (1 if static else 0), 255 if static else 256))
    return Bn, Tn, Dn, R, W, static, residual, dtype


LR_CASES = ([_lowrank_case(i) for i in range(64)] + [_lowrank_wide_case(i) for i in range(24)]
            + [_lowrank_widew_case(i) for i in range(24)] + [_lowrank_big_lds_case(i) for i in range(24)])
HW_CASES = [_headwise_case(i) for i in range(64)] + [_headwise_wide_case(i) for i in range(32)]


def _ids(cases, kind):
    return [f"{kind}{i}-B{c[0]}T{c[1]}D{c[2]}-{c[3]}-W{c[4]}-st{int(c[5])}-res{int(c[6])}-{str(c[7])[6:]}"
            for i, c in enumerate(cases)]


@pytest.mark.parametrize("Bn,Tn,Dn,R,W,static,residual,dtype", LR_CASES, ids=_ids(LR_CASES, "lr"))
def test_random_lowrank(Bn, Tn, Dn, R, W, static, residual, dtype):
    g = gen(Bn * 7 + Tn * 131 + Dn * 17 + R * 3 + W)
    x = randn(g, Bn, Tn, Dn)
    dy = randn(g, Bn, Tn, Dn)
    z = randn(g, Bn, Tn, R)
    U = randn(g, R, W * Dn, scale=1 / math.sqrt((R + 1) * W))
    sw = uniform(g, W, Dn, lo=-1 / math.sqrt(W), hi=1 / math.sqrt(W)) if static else None
    src = [x, z, U, sw]

    def kernel(a, b, c, d, residual):
        return lr_mod._LowrankDynamicConvolutionFn.apply(a, b, c, d, residual)

    src_q = [None if t is None else t.to(dtype).float() for t in src]
    y_q, g_q = run_fwd_bwd(lr_ref, src_q, dy.to(dtype).float(), residual)
    y_k, g_k = run_fwd_bwd(kernel, [_to(t, dtype) for t in src], _to(dy, dtype), residual)
    torch.cuda.synchronize()
    assert_ns(y_k, y_q, dtype, "y")
    for a, b, n in zip(g_k, g_q, ["dx", "dz", "dU", "dstatic_w"]):
        if b is not None:
            assert_ns(a, b, dtype, n, elementwise=n == "dx")
    check_reductions("lr", src_q, dy.to(dtype).float(), g_k, dtype)


@pytest.mark.parametrize("Bn,Tn,Dn,H,W,static,residual,dtype", HW_CASES, ids=_ids(HW_CASES, "hw"))
def test_random_headwise(Bn, Tn, Dn, H, W, static, residual, dtype):
    g = gen(Bn * 11 + Tn * 137 + Dn * 19 + H * 5 + W)
    x = randn(g, Bn, Tn, Dn)
    dy = randn(g, Bn, Tn, Dn)
    w = randn(g, Bn, Tn, H, W, scale=1 / math.sqrt(W))
    sw = uniform(g, W, Dn, lo=-1 / math.sqrt(W), hi=1 / math.sqrt(W)) if static else None
    src = [x, w, sw]
    src_q = [None if t is None else t.to(dtype).float() for t in src]
    y_q, g_q = run_fwd_bwd(hw_ref, src_q, dy.to(dtype).float(), residual)
    y_k, g_k = run_fwd_bwd(hw_mod.headwise_dynamic_convolution, [_to(t, dtype) for t in src], _to(dy, dtype),
                           residual)
    torch.cuda.synchronize()
    assert_ns(y_k, y_q, dtype, "y")
    for a, b, n in zip(g_k, g_q, ["dx", "dweight", "dstatic_w"]):
        if b is not None:
            assert_ns(a, b, dtype, n, elementwise=n != "dstatic_w")
    check_reductions("hw", src_q, dy.to(dtype).float(), g_k, dtype)


def _grouped_case(i):
    rnd = random.Random(15485863 * i + 11)
    dtype = rnd.choice(DTYPES)
    G = rnd.randint(1, 4)
    Bn = rnd.randint(1, 2)
    Tn = rnd.choice([1, 5, 16, 17, 40, 100])
    Dn = rnd.choice([8, 16, 40, 64, 128, 192])
    extra = rnd.choice([0, 0, 8, 24])  # x is a column slice of a wider tensor
    W = rnd.randint(1, 8)
    static = rnd.random() < 0.5
    R = rnd.randint(1, 31)
    hd = rnd.choice([None, None] + [d for d in (4, 8, 16, 32, 64) if Dn % d == 0])
    return G, Bn, Tn, Dn, extra, R, W, static, hd, dtype


GR_CASES = [_grouped_case(i) for i in range(32)]


@pytest.mark.parametrize("G,Bn,Tn,Dn,extra,R,W,static,hd,dtype", GR_CASES,
                         ids=[f"g{i}-G{c[0]}B{c[1]}T{c[2]}D{c[3]}x{c[4]}-R{c[5]}W{c[6]}-st{int(c[7])}-hd{c[8]}-"
                              f"{str(c[9])[6:]}" for i, c in enumerate(GR_CASES)])
def test_random_grouped(G, Bn, Tn, Dn, extra, R, W, static, hd, dtype):
    """The grouped operator (x read in place, optional head-major outputs) on random shapes."""
    g = gen(G * 101 + Bn * 7 + Tn * 131 + Dn * 17 + R * 3 + W + extra)
    xw = randn(g, Bn, Tn, G * Dn + extra)
    zs = [randn(g, Bn, Tn, R) for _ in range(G)]
    Us = [randn(g, R, W * Dn, scale=1 / math.sqrt((R + 1) * W)) for _ in range(G)]
    sws = [uniform(g, W, Dn, lo=-1 / math.sqrt(W), hi=1 / math.sqrt(W)) for _ in range(G)] if static else None
    dys = [randn(g, Bn, Tn, Dn) for _ in range(G)]
    x_k = xw.to(dtype).to(DEV)[..., :G * Dn].detach().requires_grad_()
    zk = [t.to(dtype).to(DEV).requires_grad_() for t in zs]
    Uk = [t.to(dtype).to(DEV).requires_grad_() for t in Us]
    sk = [t.to(dtype).to(DEV).requires_grad_() for t in sws] if static else None
    # the Python API keeps the reference's power-of-two rank rule; other ranks via the Function
    ys = dlr._GroupedLowrankDynamicConvolutionFn.apply(x_k, True, G, static, hd or 0,
                                                       *(zk + Uk + (sk if static else [])))
    H = Dn // hd if hd else None
    grads = [d.to(dtype).to(DEV) if hd is None else d.to(dtype).to(DEV).view(Bn, Tn, H, hd).transpose(1, 2)
             .contiguous() for d in dys]
    torch.autograd.backward(ys, grads)
    torch.cuda.synchronize()
    for gi in range(G):
        xs = xw[..., gi * Dn:(gi + 1) * Dn].to(dtype).float().requires_grad_()
        zr = zs[gi].to(dtype).float().requires_grad_()
        Ur = Us[gi].to(dtype).float().requires_grad_()
        sr = sws[gi].to(dtype).float().requires_grad_() if static else None
        yr = lr_ref(xs, zr, Ur, sr, residual=True)
        yr.backward(dys[gi].to(dtype).float())
        y = ys[gi] if hd is None else ys[gi].transpose(1, 2).reshape(Bn, Tn, Dn)
        assert_ns(y, yr, dtype, f"g{gi} y")
        assert_ns(x_k.grad[..., gi * Dn:(gi + 1) * Dn], xs.grad, dtype, f"g{gi} dx")
        assert_ns(zk[gi].grad, zr.grad, dtype, f"g{gi} dz", elementwise=False)
        assert_ns(Uk[gi].grad, Ur.grad, dtype, f"g{gi} dU", elementwise=False)
        if static:
            assert_ns(sk[gi].grad, sr.grad, dtype, f"g{gi} dstatic_w", elementwise=False)
        check_reductions("lr", [xs.detach(), zr.detach(), Ur.detach(), None if sr is None else sr.detach()],
                         dys[gi].to(dtype).float(), [None, zk[gi].grad, Uk[gi].grad, sk[gi].grad if static else None],
                         dtype, tag=f"g{gi} ")
