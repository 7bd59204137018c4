"""CPU pins of the per-entry reduction bound (helpers.assert_sum / SUM_TOL) that the GPU tests
apply to dU, dz and dstatic_w.

An emulation of the 16-bit lowrank backward's arithmetic (dy*x rounded to the I/O type, exact
products, fp32 sums, one rounding of the output) must pass it, also where fp16 products fall into
the subnormal range; the same emulation with a planted mistake of the kind a kernel could make (a
16-row tile left out of the sum, a tap shifted by one row, the static rank's row dropped) must
fail it.  The mistakes are planted here, in the emulation on the CPU.
"""

import math

import pytest
import torch

from helpers import assert_sum, dstatic_sums, lowrank_sums


def _shift(x, k):
    out = torch.zeros_like(x)
    if k == 0:
        return x.clone()
    out[:, k:] = x[:, :-k]
    return out


def _emulate(x, z, U, dy, dtype, drop_rows=None, tap_err=0):
    """dU and dz as the 16-bit kernels form them: G_k = dtype(dy * x shifted by k), products of
    dtype values accumulated in fp32, outputs rounded to dtype.  drop_rows: rows left out of dU's
    sum (a lost tile); tap_err: an extra row shift of every tap (a wrong tap index)."""
    Bn, Tn, Dn = x.shape
    R = z.shape[-1]
    W = U.shape[1] // Dn
    dU, dz = [], torch.zeros(Bn, Tn, R)
    zf = z.reshape(-1, R)
    for k in range(W):
        G = (dy * _shift(x, k + tap_err)).to(dtype).float()
        Gf = G.reshape(-1, Dn)
        if drop_rows is not None:
            keep = torch.ones(Bn * Tn, dtype=torch.bool)
            keep[drop_rows] = False
            dU.append(zf[keep].t() @ Gf[keep])
        else:
            dU.append(zf.t() @ Gf)
        dz += (Gf @ U[:, k * Dn:(k + 1) * Dn].t()).reshape(Bn, Tn, R)
    return torch.cat(dU, dim=1).to(dtype), dz.to(dtype)


def _inputs(dtype, scale=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    Bn, Tn, Dn, R, W = 2, 64, 32, 8, 4
    x = (torch.randn(Bn, Tn, Dn, generator=g) * scale).to(dtype).float()
    dy = (torch.randn(Bn, Tn, Dn, generator=g) * scale).to(dtype).float()
    z = torch.randn(Bn, Tn, R, generator=g).to(dtype).float()
    U = (torch.randn(R, W * Dn, generator=g) / math.sqrt(R * W)).to(dtype).float()
    return x, z, U, dy


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scale", [1.0, 3e-3])  # 3e-3: fp16 products of about 1e-5, subnormal
def test_emulated_kernel_passes(dtype, scale):
    x, z, U, dy = _inputs(dtype, scale)
    ref = lowrank_sums(x, z, U, dy)
    dU, dz = _emulate(x, z, U, dy, dtype)
    assert_sum(dU, ref["dU"], dtype, "dU", floor=ref["floor_dU"])
    assert_sum(dz, ref["dz"], dtype, "dz", floor=ref["floor_dz"])


def test_fp16_subnormal_products_need_the_floor():
    """Without the subnormal floor the fp16 emulation fails at small magnitudes: the floor is
    what admits it, not a loose relative bound."""
    dtype = torch.float16
    x, z, U, dy = _inputs(dtype, 3e-3)
    ref = lowrank_sums(x, z, U, dy)
    dU, _ = _emulate(x, z, U, dy, dtype)
    with pytest.raises(AssertionError):
        assert_sum(dU, ref["dU"], dtype, "dU")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_lost_tile_fails(dtype):
    x, z, U, dy = _inputs(dtype)
    ref = lowrank_sums(x, z, U, dy)
    dU, _ = _emulate(x, z, U, dy, dtype, drop_rows=list(range(16, 32)))
    with pytest.raises(AssertionError):
        assert_sum(dU, ref["dU"], dtype, "dU", floor=ref["floor_dU"])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_wrong_tap_fails(dtype):
    x, z, U, dy = _inputs(dtype)
    ref = lowrank_sums(x, z, U, dy)
    dU, dz = _emulate(x, z, U, dy, dtype, tap_err=1)
    with pytest.raises(AssertionError):
        assert_sum(dU, ref["dU"], dtype, "dU", floor=ref["floor_dU"])
    with pytest.raises(AssertionError):
        assert_sum(dz, ref["dz"], dtype, "dz", floor=ref["floor_dz"])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dropped_static_row_fails(dtype):
    """dstatic_w is the dU row of a ones-column of z (lowrank.py:223-225, 297): zeroing that row,
    as a static rank left out of the kernel rank would, fails the bound."""
    x, _, _, dy = _inputs(dtype)
    W = 4
    ref = dstatic_sums(x, dy, W)
    good = ref[0].to(dtype)
    assert_sum(good, ref, dtype, "dstatic_w", floor=4 * 2.0**-25 * math.sqrt(x.shape[0] * x.shape[1]))
    bad = good.clone()
    bad[W - 1] = 0
    with pytest.raises(AssertionError):
        assert_sum(bad, ref, dtype, "dstatic_w")
