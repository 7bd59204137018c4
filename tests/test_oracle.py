"""Pins the CPU oracle (oracle/reference_cpu.py) before anything is compared with it.

Each check is chosen so that a plausible slip in the restatement fails it:
  * known-answer values computed by hand from README.md:12-17;
  * float64 index loops with hand-derived backward (oracle/brute.py);
  * zero dynamic weight + static filter == depthwise causal F.conv1d (a
    library routine), which fixes the tap direction and padding side;
  * W = 1 == elementwise product;
  * lowrank == headwise(hs=1) on (z@U).view(B,T,W,D).transpose(-1,-2);
  * one-hot z selects a row of U;
  * gradcheck in float64 and the adjoint identity <dy, J v> = <J^T dy, v>.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import brute
from oracle.reference_cpu import (
    headwise_dynamic_convolution_ref as hw_ref,
    lowrank_dynamic_convolution_ref as lr_ref,
)


def _t(a):
    return torch.tensor(a, dtype=torch.float64)


# ---------------------------------------------------------------- known answer
def test_headwise_known_answer():
    # B=1, T=3, D=2, H=1 (head_size 2), W=2; values worked out by hand.
    x = _t([[[1, 2], [3, 4], [5, 6]]])
    w = _t([[[[0.5, 1.0]], [[2.0, -1.0]], [[1.5, 0.25]]]])
    sw = _t([[0.1, 0.2], [0.3, 0.4]])
    y = hw_ref(x, w, sw)
    exp = _t([[[0.6, 1.4], [5.6, 7.6], [9.65, 12.8]]])
    torch.testing.assert_close(y, exp, atol=1e-12, rtol=0)
    yr = hw_ref(x, w, sw, residual=True)
    torch.testing.assert_close(yr, exp + x, atol=1e-12, rtol=0)

    xs, ws, sws = (t.clone().requires_grad_() for t in (x, w, sw))
    hw_ref(xs, ws, sws).sum().backward()
    torch.testing.assert_close(xs.grad, _t([[[-0.1, 0.1], [2.65, 2.85], [1.6, 1.7]]]), atol=1e-12, rtol=0)
    torch.testing.assert_close(ws.grad, _t([[[[3, 0]], [[7, 3]], [[11, 7]]]]), atol=1e-12, rtol=0)
    torch.testing.assert_close(sws.grad, _t([[9, 12], [4, 6]]), atol=1e-12, rtol=0)


# ----------------------------------------------------------------- brute force
HW_CASES = [
    # B, T, D, H, W, static, residual
    (1, 5, 4, 4, 1, False, False),
    (2, 7, 6, 3, 3, True, False),   # head_size 2
    (1, 9, 6, 2, 4, True, True),    # head_size 3 (not a power of two)
    (2, 6, 8, 1, 5, False, True),   # one head over all channels, W > T/2
    (1, 3, 4, 2, 4, True, False),   # W > T
]


@pytest.mark.parametrize("B,T,D,H,W,static,residual", HW_CASES)
def test_headwise_vs_brute(B, T, D, H, W, static, residual):
    g = np.random.default_rng(1000 + B * 100 + T * 10 + W)
    x = g.standard_normal((B, T, D))
    w = g.standard_normal((B, T, H, W))
    sw = g.standard_normal((W, D)) if static else None
    dy = g.standard_normal((B, T, D))

    y_b = brute.headwise_fwd(x, w, sw, residual)
    dx_b, dw_b, dsw_b = brute.headwise_bwd(x, w, sw, dy, residual)

    xs, ws = _t(x).requires_grad_(), _t(w).requires_grad_()
    sws = _t(sw).requires_grad_() if static else None
    y = hw_ref(xs, ws, sws, residual=residual)
    y.backward(_t(dy))
    np.testing.assert_allclose(y.detach().numpy(), y_b, atol=1e-12)
    np.testing.assert_allclose(xs.grad.numpy(), dx_b, atol=1e-12)
    np.testing.assert_allclose(ws.grad.numpy(), dw_b, atol=1e-12)
    if static:
        np.testing.assert_allclose(sws.grad.numpy(), dsw_b, atol=1e-12)


LR_CASES = [
    # B, T, D, R, W, static, residual
    (1, 5, 4, 1, 1, False, False),
    (2, 6, 3, 2, 3, True, True),
    (1, 8, 4, 4, 4, True, False),
    (2, 4, 2, 3, 2, False, True),
]


@pytest.mark.parametrize("B,T,D,R,W,static,residual", LR_CASES)
def test_lowrank_vs_brute(B, T, D, R, W, static, residual):
    g = np.random.default_rng(2000 + B * 100 + T * 10 + R)
    x = g.standard_normal((B, T, D))
    z = g.standard_normal((B, T, R))
    U = g.standard_normal((R, W * D))
    sw = g.standard_normal((W, D)) if static else None
    dy = g.standard_normal((B, T, D))

    y_b = brute.lowrank_fwd(x, z, U, sw, residual)
    dx_b, dz_b, dU_b, dsw_b = brute.lowrank_bwd(x, z, U, sw, dy, residual)

    xs, zs, Us = (_t(a).requires_grad_() for a in (x, z, U))
    sws = _t(sw).requires_grad_() if static else None
    y = lr_ref(xs, zs, Us, sws, residual=residual)
    y.backward(_t(dy))
    np.testing.assert_allclose(y.detach().numpy(), y_b, atol=1e-12)
    np.testing.assert_allclose(xs.grad.numpy(), dx_b, atol=1e-12)
    np.testing.assert_allclose(zs.grad.numpy(), dz_b, atol=1e-12)
    np.testing.assert_allclose(Us.grad.numpy(), dU_b, atol=1e-12)
    if static:
        np.testing.assert_allclose(sws.grad.numpy(), dsw_b, atol=1e-12)


# ------------------------------------------------------------ library identity
@pytest.mark.parametrize("W", [1, 2, 4, 7])
def test_static_only_equals_depthwise_conv1d(W):
    g = torch.Generator().manual_seed(W)
    B, T, D = 2, 33, 12
    x = torch.randn(B, T, D, generator=g, dtype=torch.float64)
    sw = torch.randn(W, D, generator=g, dtype=torch.float64)
    w0 = torch.zeros(B, T, D, W, dtype=torch.float64)
    y = hw_ref(x, w0, sw)
    # F.conv1d is a cross-correlation: out[t] = sum_j ker[j] * in[t + j].  With
    # W-1 zeros on the left and the taps flipped, ker[j] = sw[W-1-j] and
    # in[t + j] = x[t - (W-1-j)], i.e. out[t] = sum_k sw[k] x[t-k].
    ker = sw.flip(0).t().unsqueeze(1)  # [D, 1, W]
    ref = F.conv1d(F.pad(x.transpose(1, 2), (W - 1, 0)), ker, groups=D).transpose(1, 2)
    torch.testing.assert_close(y, ref, atol=1e-12, rtol=0)


def test_w1_is_elementwise_product():
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, 9, 8, generator=g, dtype=torch.float64)
    w = torch.randn(2, 9, 4, 1, generator=g, dtype=torch.float64)
    y = hw_ref(x, w, residual=True)
    torch.testing.assert_close(y, x * w[..., 0].repeat_interleave(2, dim=2) + x, atol=1e-12, rtol=0)


def test_zero_weight_residual_is_identity():
    x = torch.randn(2, 9, 8, dtype=torch.float64)
    torch.testing.assert_close(hw_ref(x, torch.zeros(2, 9, 8, 3, dtype=torch.float64), residual=True), x)
    z = torch.randn(2, 9, 4, dtype=torch.float64)
    torch.testing.assert_close(lr_ref(x, z, torch.zeros(4, 3 * 8, dtype=torch.float64), residual=True), x)


def test_lowrank_equals_headwise_hs1():
    g = torch.Generator().manual_seed(3)
    B, T, D, R, W = 2, 17, 8, 5, 3
    x = torch.randn(B, T, D, generator=g, dtype=torch.float64)
    z = torch.randn(B, T, R, generator=g, dtype=torch.float64)
    U = torch.randn(R, W * D, generator=g, dtype=torch.float64)
    sw = torch.randn(W, D, generator=g, dtype=torch.float64)
    w = (z @ U).view(B, T, W, D).transpose(-1, -2).contiguous()  # [B,T,D,W]: H = D
    torch.testing.assert_close(lr_ref(x, z, U, sw, True), hw_ref(x, w, sw, True), atol=1e-12, rtol=0)


def test_lowrank_one_hot_selects_row():
    B, T, D, R, W = 1, 6, 4, 3, 2
    x = torch.randn(B, T, D, dtype=torch.float64)
    U = torch.randn(R, W * D, dtype=torch.float64)
    z = torch.zeros(B, T, R, dtype=torch.float64)
    z[..., 2] = 1.0
    y = lr_ref(x, z, U)
    sw = U[2].view(W, D)
    torch.testing.assert_close(y, hw_ref(x, torch.zeros(B, T, D, W, dtype=torch.float64), sw), atol=1e-12, rtol=0)


# ------------------------------------------------------------------- gradients
def test_gradcheck_headwise():
    g = torch.Generator().manual_seed(11)
    x = torch.randn(1, 6, 4, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(1, 6, 2, 3, generator=g, dtype=torch.float64, requires_grad=True)
    sw = torch.randn(3, 4, generator=g, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda a, b, c: hw_ref(a, b, c, True), (x, w, sw))


def test_gradcheck_lowrank():
    g = torch.Generator().manual_seed(12)
    x = torch.randn(1, 5, 3, generator=g, dtype=torch.float64, requires_grad=True)
    z = torch.randn(1, 5, 2, generator=g, dtype=torch.float64, requires_grad=True)
    U = torch.randn(2, 2 * 3, generator=g, dtype=torch.float64, requires_grad=True)
    sw = torch.randn(2, 3, generator=g, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda a, b, c, d: lr_ref(a, b, c, d, False), (x, z, U, sw))


def test_adjoint_identity_headwise_x():
    # y is linear in x for fixed weights: <dy, J v> == <J^T dy, v>.
    g = torch.Generator().manual_seed(13)
    B, T, D, H, W = 2, 11, 8, 2, 4
    w = torch.randn(B, T, H, W, generator=g, dtype=torch.float64)
    sw = torch.randn(W, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, T, D, generator=g, dtype=torch.float64)
    dy = torch.randn(B, T, D, generator=g, dtype=torch.float64)
    x = torch.zeros(B, T, D, dtype=torch.float64, requires_grad=True)
    y = hw_ref(x, w, sw)
    (jt_dy,) = torch.autograd.grad(y, x, dy)
    lhs = (dy * hw_ref(v, w, sw)).sum()
    rhs = (jt_dy * v).sum()
    torch.testing.assert_close(lhs, rhs)
