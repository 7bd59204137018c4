"""GPU parity of the grouped lowrank operator and the README modules.

lowrank_dynamic_convolution_grouped runs G lowrank convolutions of one shape
in one launch per direction, reading x as G column slices of one [B, T, G*D]
tensor in place (README.md:57-110 uses three calls on .contiguous() slices of
the fused q|k|v projection).  Checked here:

* every group's y, dx slice, dz, dU and dstatic_w against the CPU oracle
  (oracle/reference_cpu.py) on the same dtype-rounded inputs, to the
  north-star tolerance, for 1-4 groups, with and without the static filter,
  on the MFMA path (bf16, fp16) and the generic path (fp32), with x a column
  slice of a wider tensor (row stride above G*D);
* bitwise equality with G separate lowrank_dynamic_convolution calls (same
  kernels, same reduction order per group);
* a loss that uses only some groups' outputs (the others get zero gradients);
* GroupedLowRankDynamicShortConvolution against G LowRankDynamicShortConvolution
  modules holding the same parameters, and the README module against the oracle.
"""

import math

import pytest
import torch

from helpers import assert_ns, check_reductions, gen, randn, run_fwd_bwd, uniform
from oracle.reference_cpu import lowrank_dynamic_convolution_ref as lr_ref
import lowrank as lr_mod

pytestmark = pytest.mark.gpu

DEV = "cuda"
lr = lr_mod.lowrank_dynamic_convolution
lr_grouped = lr_mod.lowrank_dynamic_convolution_grouped


def _inputs(G, Bn, Tn, Dn, R, W, static, extra, seed):
    """fp32 CPU inputs: x [B, T, G*D + extra] (the grouped op reads its first G*D columns), dy per group."""
    g = gen(seed)
    xw = randn(g, Bn, Tn, G * Dn + extra)
    zs = [randn(g, Bn, Tn, R) for _ in range(G)]
    Us = [randn(g, R, W * Dn, scale=1 / math.sqrt((R + int(static)) * W)) for _ in range(G)]
    sws = [uniform(g, W, Dn, lo=-1 / math.sqrt(W), hi=1 / math.sqrt(W)) for _ in range(G)] if static else None
    dys = [randn(g, Bn, Tn, Dn) for _ in range(G)]
    return xw, zs, Us, sws, dys


def _leaf(t, dtype):
    return t.to(dtype).to(DEV).detach().requires_grad_()


CASES = [
    # G, B, T, D, R, W, static, extra columns, dtype
    (3, 2, 64, 128, 15, 4, True, 64, torch.bfloat16),   # q|k|v slice of a wider tensor, static as rank 16
    (3, 2, 80, 64, 16, 4, False, 0, torch.bfloat16),    # contiguous fused input, rank 16
    (4, 1, 48, 64, 31, 3, True, 8, torch.bfloat16),     # four groups, two rank chunks
    (2, 2, 33, 128, 8, 2, False, 16, torch.float16),    # odd T
    (1, 2, 40, 48, 7, 4, True, 0, torch.bfloat16),      # one group
    (2, 2, 24, 40, 3, 3, True, 12, torch.float32),      # fp32
    (3, 2, 50, 64, 15, 12, True, 8, torch.bfloat16),    # W 12: backward as three passes of 4 taps
    (2, 1, 70, 128, 31, 10, True, 0, torch.float16),    # W 10, two rank chunks
    (3, 2, 90, 128, 15, 20, True, 8, torch.bfloat16),   # W 20: one forward pass, three backward passes
    (3, 2, 70, 128, 127, 4, True, 8, torch.bfloat16),   # kernel rank 128: passes of ranks (2 forward, 4 backward)
    (2, 1, 50, 64, 63, 6, True, 0, torch.float16),      # kernel rank 64, W 6 (forward in one pass)
    (2, 2, 40, 64, 15, 40, True, 8, torch.bfloat16),    # W 40: the generic kernels, group by group
]


@pytest.mark.parametrize("G,Bn,Tn,Dn,R,W,static,extra,dtype", CASES)
def test_grouped_against_oracle(G, Bn, Tn, Dn, R, W, static, extra, dtype):
    xw, zs, Us, sws, dys = _inputs(G, Bn, Tn, Dn, R, W, static, extra, seed=G * 131 + Tn + Dn + R)
    # kernel: x is the column slice [:, :, :G*D] of the wider device tensor
    xw_k = xw.to(dtype).to(DEV)
    x_k = xw_k[..., :G * Dn].detach().requires_grad_()
    assert extra == 0 or not x_k.is_contiguous()
    zk = [_leaf(t, dtype) for t in zs]
    Uk = [_leaf(t, dtype) for t in Us]
    sk = [_leaf(t, dtype) for t in sws] if static else None
    ys = lr_grouped(x_k, zk, Uk, sk, residual=True)
    assert len(ys) == G
    torch.autograd.backward(ys, [d.to(dtype).to(DEV) for d in dys])
    torch.cuda.synchronize()
    for g in range(G):
        xs = xw[..., g * Dn:(g + 1) * Dn].to(dtype).float().requires_grad_()
        zr = zs[g].to(dtype).float().requires_grad_()
        Ur = Us[g].to(dtype).float().requires_grad_()
        sr = sws[g].to(dtype).float().requires_grad_() if static else None
        yr = lr_ref(xs, zr, Ur, sr, residual=True)
        yr.backward(dys[g].to(dtype).float())
        assert_ns(ys[g], yr, dtype, f"g{g} y")
        assert_ns(x_k.grad[..., g * Dn:(g + 1) * Dn], xs.grad, dtype, f"g{g} dx")
        assert_ns(zk[g].grad, zr.grad, dtype, f"g{g} dz", elementwise=False)
        assert_ns(Uk[g].grad, Ur.grad, dtype, f"g{g} dU", elementwise=False)
        if static:
            assert_ns(sk[g].grad, sr.grad, dtype, f"g{g} dstatic_w", elementwise=False)
        check_reductions("lr", [xs.detach(), zr.detach(), Ur.detach(), None if sr is None else sr.detach()],
                         dys[g].to(dtype).float(), [None, zk[g].grad, Uk[g].grad, sk[g].grad if static else None],
                         dtype, tag=f"g{g} ")


def test_grouped_long_sequence():
    """The grouped op on one long sequence, B1 T32768 D4096 x3 (the q|k|v of configs[4] at four times the
    length), R15 + static_w: x rows are 3 * 4096 elements apart, so the sequence's x spans 768 MiB.  The
    matrix-core kernels give each run of tiles its own buffer resources (before, sequences past 512 MiB,
    here T > 21813, took the generic kernels).  Local outputs on row windows at both ends, in the middle
    and around row 21813; every dz row and dU / dstatic_w entry of each group against float64 sums."""
    G, Bn, Tn, Dn, R, W = 3, 1, 32768, 4096, 15, 4
    dtype = torch.bfloat16
    print(f"[long grouped] G{G} B{Bn} T{Tn} D{Dn} R{R}+static W{W}", flush=True)
    g = gen(23)
    xw = randn(g, Bn, Tn, G * Dn).to(dtype)
    zs = [randn(g, Bn, Tn, R).to(dtype) for _ in range(G)]
    Us = [randn(g, R, W * Dn, scale=1 / math.sqrt((R + 1) * W)).to(dtype) for _ in range(G)]
    sws = [uniform(g, W, Dn, lo=-1 / math.sqrt(W), hi=1 / math.sqrt(W)).to(dtype) for _ in range(G)]
    dys = [randn(g, Bn, Tn, Dn).to(dtype) for _ in range(G)]
    x_k = xw.to(DEV).requires_grad_()
    zk = [t.to(DEV).requires_grad_() for t in zs]
    Uk = [t.to(DEV).requires_grad_() for t in Us]
    sk = [t.to(DEV).requires_grad_() for t in sws]
    ys = lr_grouped(x_k, zk, Uk, sk, residual=True)
    torch.autograd.backward(ys, [d.to(DEV) for d in dys])
    torch.cuda.synchronize()
    old_limit = (1 << 29) // (G * Dn * 2) - 32  # first row past the former per-sequence limit
    windows = [(0, 64), (Tn // 2 - 32, Tn // 2 + 32), (Tn - 64, Tn), (old_limit - 40, old_limit + 24)]
    dx_all = x_k.grad.cpu()
    for gi in range(G):
        xs = xw[..., gi * Dn:(gi + 1) * Dn].float()
        y_k, dz_k = ys[gi].cpu(), zk[gi].grad.cpu()
        for t0, t1 in windows:
            a, e = max(0, t0 - W + 1), min(Tn, t1 + W - 1)
            win = [xs[:, a:e].clone(), zs[gi][:, a:e].float(), Us[gi].float(), sws[gi].float()]
            y_w, g_w = run_fwd_bwd(lr_ref, win, dys[gi][:, a:e].float(), True)
            sl = slice(t0 - a, t1 - a)
            assert_ns(y_k[:, t0:t1], y_w[:, sl], dtype, f"g{gi} y[{t0}:{t1}]")
            assert_ns(dx_all[:, t0:t1, gi * Dn:(gi + 1) * Dn], g_w[0][:, sl], dtype, f"g{gi} dx[{t0}:{t1}]")
        check_reductions("lr", [xs, zs[gi].float(), Us[gi].float(), sws[gi].float()], dys[gi].float(),
                         [None, dz_k, Uk[gi].grad, sk[gi].grad], dtype, tag=f"g{gi} ")


@pytest.mark.parametrize("static", [False, True])
def test_grouped_bitwise_equals_separate_calls(static):
    G, Bn, Tn, Dn, R, W = 3, 2, 96, 256, 15 if static else 16, 4
    dtype = torch.bfloat16
    xw, zs, Us, sws, dys = _inputs(G, Bn, Tn, Dn, R, W, static, 32, seed=7 + int(static))
    xw_k = xw.to(dtype).to(DEV)
    dyk = [d.to(dtype).to(DEV) for d in dys]

    x_g = xw_k[..., :G * Dn].detach().requires_grad_()
    zg = [_leaf(t, dtype) for t in zs]
    Ug = [_leaf(t, dtype) for t in Us]
    sg = [_leaf(t, dtype) for t in sws] if static else None
    ys_g = lr_grouped(x_g, zg, Ug, sg, residual=True)
    torch.autograd.backward(ys_g, dyk)

    for g in range(G):
        x1 = xw_k[..., g * Dn:(g + 1) * Dn].contiguous().requires_grad_()
        z1, U1 = _leaf(zs[g], dtype), _leaf(Us[g], dtype)
        s1 = _leaf(sws[g], dtype) if static else None
        y1 = lr(x1, z1, U1, s1, residual=True)
        y1.backward(dyk[g])
        assert torch.equal(ys_g[g], y1), f"group {g}: y"
        assert torch.equal(x_g.grad[..., g * Dn:(g + 1) * Dn], x1.grad), f"group {g}: dx"
        assert torch.equal(zg[g].grad, z1.grad), f"group {g}: dz"
        assert torch.equal(Ug[g].grad, U1.grad), f"group {g}: dU"
        if static:
            assert torch.equal(sg[g].grad, s1.grad), f"group {g}: dstatic_w"


def test_grouped_partial_loss():
    """Outputs that do not reach the loss contribute zero gradients."""
    G, Bn, Tn, Dn, R, W = 3, 1, 64, 128, 15, 4
    dtype = torch.bfloat16
    xw, zs, Us, sws, dys = _inputs(G, Bn, Tn, Dn, R, W, True, 0, seed=3)
    x = _leaf(xw, dtype)
    zk = [_leaf(t, dtype) for t in zs]
    Uk = [_leaf(t, dtype) for t in Us]
    sk = [_leaf(t, dtype) for t in sws]
    q, k, v = lr_grouped(x, zk, Uk, sk, residual=True)
    (q.float() * dys[0].to(DEV)).sum().backward()
    assert torch.count_nonzero(x.grad[..., Dn:]) == 0
    for g in (1, 2):
        assert torch.count_nonzero(zk[g].grad) == 0 and torch.count_nonzero(Uk[g].grad) == 0
        assert torch.count_nonzero(sk[g].grad) == 0
    xs = xw[..., :Dn].to(dtype).float().requires_grad_()
    zr, Ur, sr = (t.to(dtype).float().requires_grad_() for t in (zs[0], Us[0], sws[0]))
    yr = lr_ref(xs, zr, Ur, sr, residual=True)
    (yr * dys[0]).sum().backward()
    assert_ns(x.grad[..., :Dn], xs.grad, dtype, "dq")
    assert_ns(zk[0].grad, zr.grad, dtype, "dz_q", elementwise=False)


def test_modules_grouped_matches_separate():
    from dynconv import GroupedLowRankDynamicShortConvolution, LowRankDynamicShortConvolution

    torch.manual_seed(0)
    Dm, R, W, G, Bn, Tn = 256, 15, 4, 3, 2, 128
    dtype = torch.bfloat16
    grouped = GroupedLowRankDynamicShortConvolution(Dm, R, W, groups=G).to(DEV, dtype)
    with torch.no_grad():
        grouped.proj_out.normal_(0, 1 / math.sqrt((R + 1) * W))  # the README initialises U to zero
    singles = []
    for g in range(G):
        m = LowRankDynamicShortConvolution(Dm, R, W).to(DEV, dtype)
        with torch.no_grad():
            m.proj_in.weight.copy_(grouped.proj_in.weight[g * R:(g + 1) * R])
            m.proj_out.copy_(grouped.proj_out[g])
            m.proj_out_bias.copy_(grouped.proj_out_bias[g])
        singles.append(m)
    pre_z = torch.randn(Bn, Tn, Dm, device=DEV, dtype=dtype)
    qkv = torch.randn(Bn, Tn, G * Dm, device=DEV, dtype=dtype)
    dys = [torch.randn(Bn, Tn, Dm, device=DEV, dtype=dtype) for _ in range(G)]

    x1 = qkv.clone().requires_grad_()
    outs = grouped(x1, pre_z)
    torch.autograd.backward(outs, dys)
    x2 = qkv.clone().requires_grad_()
    # README.md:99-110: split the fused projection, one module per slice
    parts = x2.split(Dm, dim=-1)
    outs2 = [m(p, pre_z) for m, p in zip(singles, parts)]
    torch.autograd.backward(outs2, dys)
    for g in range(G):
        # proj_in differs only by GEMM shape ([*, 3R] vs [*, R]); compare to bf16 tolerance
        assert_ns(outs[g], outs2[g], dtype, f"g{g} y")
        assert_ns(grouped.proj_out.grad[g], singles[g].proj_out.grad, dtype, f"g{g} dU", elementwise=False)
        assert_ns(grouped.proj_out_bias.grad[g], singles[g].proj_out_bias.grad, dtype, f"g{g} dstatic",
                  elementwise=False)
        assert_ns(grouped.proj_in.weight.grad[g * R:(g + 1) * R], singles[g].proj_in.weight.grad, dtype,
                  f"g{g} dW_in", elementwise=False)
    assert_ns(x1.grad, x2.grad, dtype, "dqkv")


def test_readme_module_against_oracle():
    from dynconv import LowRankDynamicShortConvolution

    torch.manual_seed(1)
    Dm, R, W, Bn, Tn = 128, 15, 4, 2, 64
    dtype = torch.bfloat16
    m = LowRankDynamicShortConvolution(Dm, R, W).to(DEV, dtype)
    with torch.no_grad():
        m.proj_out.normal_(0, 1 / math.sqrt((R + 1) * W))
    x = torch.randn(Bn, Tn, Dm, device=DEV, dtype=dtype, requires_grad=True)
    pre_z = torch.randn(Bn, Tn, Dm, device=DEV, dtype=dtype, requires_grad=True)
    dy = torch.randn(Bn, Tn, Dm, device=DEV, dtype=dtype)
    y = m(x, pre_z)
    y.backward(dy)
    # the whole module in fp32 on the CPU: z = pre_z @ W_in^T unrounded (proj_in and pre_z gradients)
    pz = pre_z.detach().float().cpu().requires_grad_()
    wi = m.proj_in.weight.detach().float().cpu().requires_grad_()
    y_full = lr_ref(x.detach().float().cpu(), pz @ wi.t(), m.proj_out.detach().float().cpu(),
                    m.proj_out_bias.detach().float().cpu(), residual=True)
    y_full.backward(dy.float().cpu())
    assert_ns(y, y_full, dtype, "y (fp32 z)")
    assert_ns(m.proj_in.weight.grad, wi.grad, dtype, "proj_in", elementwise=False)
    assert_ns(pre_z.grad, pz.grad, dtype, "d pre_z", elementwise=False)
    # oracle: the same bf16 z (the layer's own GEMM), then the fp32 restatement of reference.py
    z = m.proj_in(pre_z).detach()
    xr = x.detach().float().cpu().requires_grad_()
    zr = z.float().cpu().requires_grad_()
    Ur = m.proj_out.detach().float().cpu().requires_grad_()
    sr = m.proj_out_bias.detach().float().cpu().requires_grad_()
    yr = lr_ref(xr, zr, Ur, sr, residual=True)
    yr.backward(dy.float().cpu())
    assert_ns(y, yr, dtype, "y")
    assert_ns(x.grad, xr.grad, dtype, "dx")
    assert_ns(m.proj_out.grad, Ur.grad, dtype, "dU", elementwise=False)
    assert_ns(m.proj_out_bias.grad, sr.grad, dtype, "dstatic_w", elementwise=False)


@pytest.mark.parametrize("head_dim", [None, 64])
def test_grouped_module_against_oracle(head_dim):
    """GroupedLowRankDynamicShortConvolution end to end against an fp32 CPU oracle of the whole module:
    z = pre_z @ proj_in.weight^T in fp32, then reference.py's lowrank operator per group on its slice of
    the fused q|k|v projection (README.md:57-83, 99-110).  Every gradient: the fused projection x, pre_z,
    proj_in.weight, proj_out and proj_out_bias.  The kernel path rounds z to bf16 after the library's
    proj_in GEMM (dc_proj_in_fwd); the oracle keeps it in fp32, so the checks are the north-star ones
    (2e-2)."""
    from dynconv import GroupedLowRankDynamicShortConvolution

    torch.manual_seed(3)
    Dm, R, W, G, Bn, Tn = 256, 15, 4, 3, 2, 96
    dtype = torch.bfloat16
    m = GroupedLowRankDynamicShortConvolution(Dm, R, W, groups=G, head_dim=head_dim).to(DEV, dtype)
    with torch.no_grad():
        m.proj_out.normal_(0, 1 / math.sqrt((R + 1) * W))  # the README initialises U to zero
    qkv = torch.randn(Bn, Tn, G * Dm, device=DEV, dtype=dtype, requires_grad=True)
    pre_z = torch.randn(Bn, Tn, Dm, device=DEV, dtype=dtype, requires_grad=True)
    dys = [torch.randn(Bn, Tn, Dm, device=DEV, dtype=dtype) for _ in range(G)]
    outs = m(qkv, pre_z)
    if head_dim is None:
        torch.autograd.backward(outs, dys)
    else:
        H = Dm // head_dim
        torch.autograd.backward(outs, [d.view(Bn, Tn, H, head_dim).transpose(1, 2).contiguous() for d in dys])
        outs = [o.transpose(1, 2).reshape(Bn, Tn, Dm) for o in outs]
    torch.cuda.synchronize()

    def cpu_leaf(t):
        return t.detach().float().cpu().requires_grad_()

    xr, pzr = cpu_leaf(qkv), cpu_leaf(pre_z)
    win, uo, sb = cpu_leaf(m.proj_in.weight), cpu_leaf(m.proj_out), cpu_leaf(m.proj_out_bias)
    z = pzr @ win.t()  # [B, T, G*R] in fp32
    outs_r = [lr_ref(xr[..., g * Dm:(g + 1) * Dm], z[..., g * R:(g + 1) * R], uo[g], sb[g], residual=True)
              for g in range(G)]
    torch.autograd.backward(outs_r, [d.float().cpu() for d in dys])
    for g in range(G):
        assert_ns(outs[g], outs_r[g], dtype, f"g{g} y")
        assert_ns(m.proj_out.grad[g], uo.grad[g], dtype, f"g{g} proj_out", elementwise=False)
        assert_ns(m.proj_out_bias.grad[g], sb.grad[g], dtype, f"g{g} proj_out_bias", elementwise=False)
        assert_ns(m.proj_in.weight.grad[g * R:(g + 1) * R], win.grad[g * R:(g + 1) * R], dtype, f"g{g} proj_in",
                  elementwise=False)
    assert_ns(qkv.grad, xr.grad, dtype, "d qkv")
    assert_ns(pre_z.grad, pzr.grad, dtype, "d pre_z", elementwise=False)


# ------------------------------------------------------ head-major outputs
HEAD_CASES = [
    # G, B, T, D, R, W, static, head_dim, dtype, bitwise (fast kernels in both layouts)
    (3, 2, 70, 256, 15, 4, True, 64, torch.bfloat16, True),    # T % 16 != 0: the last tile's rows past T
    (3, 1, 96, 256, 16, 4, False, 128, torch.bfloat16, True),
    (2, 2, 50, 128, 31, 3, True, 64, torch.float16, True),     # two rank chunks
    (3, 2, 45, 128, 15, 4, True, 64, torch.float32, True),     # fp32 VALU kernels
    (3, 2, 40, 128, 15, 4, True, 32, torch.bfloat16, False),   # head dim 32: generic backward
    (2, 1, 33, 64, 7, 2, True, 16, torch.float32, False),      # fp32 head dim 16: generic kernels
    (3, 2, 60, 256, 15, 14, True, 64, torch.bfloat16, True),   # W 14: forward in one pass over the taps
    (3, 2, 60, 256, 15, 20, True, 64, torch.bfloat16, True),   # W 20, one rank chunk: forward in one pass
    (3, 2, 60, 256, 31, 20, True, 64, torch.bfloat16, True),   # W 20, two chunks: the second forward pass adds to y
    (2, 1, 40, 128, 63, 12, True, 64, torch.float16, True),    # kernel rank 64, W 12: forward passes 4 + 8
    # kernel rank 128: the second rank pass adds to y; head-major dy takes the backward's fp32 dx
    # accumulator, [B, T, D] dy the one-launch dx over all ranks (both round dx once: not bitwise)
    (3, 2, 60, 256, 127, 4, True, 64, torch.bfloat16, False),
    (2, 2, 45, 128, 15, 12, True, 64, torch.float32, True),    # fp32 W 12: forward passes 4 + 8
    (2, 1, 40, 128, 15, 36, True, 64, torch.bfloat16, False),  # W 36: generic kernels, head-major y
]


@pytest.mark.parametrize("G,Bn,Tn,Dn,R,W,static,hd,dtype,bitwise", HEAD_CASES)
def test_grouped_head_major(G, Bn, Tn, Dn, R, W, static, hd, dtype, bitwise):
    """head_dim writes y as y.view(B, T, H, hd).transpose(1, 2) and takes dy in that layout."""
    H = Dn // hd
    xw, zs, Us, sws, dys = _inputs(G, Bn, Tn, Dn, R, W, static, 0, seed=Tn * 7 + hd + Dn)
    dyk = [d.to(dtype).to(DEV) for d in dys]

    def run(head_dim):
        x = _leaf(xw, dtype)
        zk = [_leaf(t, dtype) for t in zs]
        Uk = [_leaf(t, dtype) for t in Us]
        sk = [_leaf(t, dtype) for t in sws] if static else None
        ys = lr_grouped(x, zk, Uk, sk, residual=True, head_dim=head_dim)
        if head_dim is None:
            grads = dyk
        else:
            grads = [d.view(Bn, Tn, H, hd).transpose(1, 2).contiguous() for d in dyk]
        torch.autograd.backward(ys, grads)
        torch.cuda.synchronize()
        return ys, x.grad, [t.grad for t in zk], [t.grad for t in Uk], [t.grad for t in sk] if static else []

    ys_h, dx_h, dz_h, dU_h, ds_h = run(hd)
    for y in ys_h:
        assert y.shape == (Bn, H, Tn, hd) and y.is_contiguous()
    if bitwise:
        ys_t, dx_t, dz_t, dU_t, ds_t = run(None)
        for g in range(G):
            assert torch.equal(ys_h[g], ys_t[g].view(Bn, Tn, H, hd).transpose(1, 2)), f"group {g}: y"
            assert torch.equal(dz_h[g], dz_t[g]), f"group {g}: dz"
            assert torch.equal(dU_h[g], dU_t[g]), f"group {g}: dU"
            if static:
                assert torch.equal(ds_h[g], ds_t[g]), f"group {g}: dstatic_w"
        assert torch.equal(dx_h, dx_t), "dx"
        return
    for g in range(G):
        xs = xw[..., g * Dn:(g + 1) * Dn].to(dtype).float().requires_grad_()
        zr = zs[g].to(dtype).float().requires_grad_()
        Ur = Us[g].to(dtype).float().requires_grad_()
        sr = sws[g].to(dtype).float().requires_grad_() if static else None
        yr = lr_ref(xs, zr, Ur, sr, residual=True)
        yr.backward(dys[g].to(dtype).float())
        assert_ns(ys_h[g].transpose(1, 2).reshape(Bn, Tn, Dn), yr, dtype, f"g{g} y")
        assert_ns(dx_h[..., g * Dn:(g + 1) * Dn], xs.grad, dtype, f"g{g} dx")
        assert_ns(dz_h[g], zr.grad, dtype, f"g{g} dz", elementwise=False)
        assert_ns(dU_h[g], Ur.grad, dtype, f"g{g} dU", elementwise=False)
        if static:
            assert_ns(ds_h[g], sr.grad, dtype, f"g{g} dstatic_w", elementwise=False)
        check_reductions("lr", [xs.detach(), zr.detach(), Ur.detach(), None if sr is None else sr.detach()],
                         dys[g].to(dtype).float(), [None, dz_h[g], dU_h[g], ds_h[g] if static else None], dtype,
                         tag=f"g{g} ")


def test_module_head_major():
    """GroupedLowRankDynamicShortConvolution(head_dim=...) returns the README's q.view(...).transpose(1, 2)."""
    from dynconv import GroupedLowRankDynamicShortConvolution

    torch.manual_seed(2)
    Dm, R, W, G, Bn, Tn, hd = 256, 15, 4, 3, 2, 64, 64
    dtype = torch.bfloat16
    a = GroupedLowRankDynamicShortConvolution(Dm, R, W, groups=G).to(DEV, dtype)
    b = GroupedLowRankDynamicShortConvolution(Dm, R, W, groups=G, head_dim=hd).to(DEV, dtype)
    with torch.no_grad():
        a.proj_out.normal_(0, 1 / math.sqrt((R + 1) * W))
        b.load_state_dict(a.state_dict())
    pre_z = torch.randn(Bn, Tn, Dm, device=DEV, dtype=dtype)
    qkv = torch.randn(Bn, Tn, G * Dm, device=DEV, dtype=dtype)
    outs_a, outs_b = a(qkv, pre_z), b(qkv, pre_z)
    for g in range(G):
        assert torch.equal(outs_b[g], outs_a[g].view(Bn, Tn, Dm // hd, hd).transpose(1, 2))
