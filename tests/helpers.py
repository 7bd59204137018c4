"""Shared test helpers: seeded inputs, tolerance checks, library loading."""

import math
import os
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "dynamic-conv1d_amd")
if PKG not in sys.path:
    sys.path.insert(0, PKG)

# test.py:17 -- the reference's own tolerance, applied as in test.py:59-69
# (oracle on the unrounded fp32 inputs, kernel on inputs cast to dtype).
REF_TOL = {torch.float32: (1e-4, 1e-3), torch.bfloat16: (4e-1, 5e-1), torch.float16: (4e-1, 5e-1)}

# North-star tolerance (oracle in fp32 on the same dtype-rounded inputs):
#   elementwise |a - b| <= atol + rtol * |b|   for outputs that are local sums
#   (y, dx, dweight) and
#   max|a - b| / max|b| <= nrm                  for every output, including the
#   long reductions (dstatic_w, dU, dz) whose bf16 rounding is relative to the
#   largest entries.
NS_TOL = {
    torch.bfloat16: dict(atol=2e-2, rtol=2e-2, nrm=2e-2),
    torch.float16: dict(atol=2e-2, rtol=2e-2, nrm=2e-2),
    torch.float32: dict(atol=1e-5, rtol=1e-5, nrm=1e-5),
}


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def randn(g, *shape, scale=1.0):
    return torch.randn(*shape, generator=g, dtype=torch.float32) * scale


def uniform(g, *shape, lo, hi):
    return torch.rand(*shape, generator=g, dtype=torch.float32) * (hi - lo) + lo


def max_rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().float().cpu()
    b = b.detach().float().cpu()
    den = b.abs().max().item()
    num = (a - b).abs().max().item()
    return num / den if den > 0 else num


def assert_ns(a, b, dtype, name="", elementwise=True):
    """North-star check of kernel output `a` against oracle output `b`."""
    tol = NS_TOL[dtype]
    r = max_rel(a, b)
    assert r <= tol["nrm"], f"{name}: max|a-b|/max|b| = {r:.3e} > {tol['nrm']:.1e}"
    if elementwise:
        torch.testing.assert_close(a.detach().float().cpu(), b.detach().float().cpu(),
                                   atol=tol["atol"], rtol=tol["rtol"], msg=lambda m: f"{name}: {m}")


def assert_ns_full(a, b, dtype, name="", elementwise=True, rows=4096):
    """assert_ns over whole (possibly multi-GB) tensors without moving them to the CPU: the
    norm-wise ratio and, when elementwise, |a - b| <= atol + rtol |b| for every entry, computed
    on a's device in chunks of `rows` along dim 1 (dim 0 for 2-D tensors).  On failure, names
    the worst entry."""
    tol = NS_TOL[dtype]
    a = a.detach()
    b = b.detach().to(a.device)
    assert a.shape == b.shape, f"{name}: shape {tuple(a.shape)} != {tuple(b.shape)}"
    dim = 1 if a.dim() >= 3 else 0
    n = a.shape[dim]
    num = den = 0.0
    worst, where = 0.0, None
    for c0 in range(0, n, rows):
        ac = a.narrow(dim, c0, min(rows, n - c0)).float()
        bc = b.narrow(dim, c0, min(rows, n - c0)).float()
        d = (ac - bc).abs()
        num = max(num, d.max().item())
        den = max(den, bc.abs().max().item())
        if elementwise:
            ratio = d / (tol["atol"] + tol["rtol"] * bc.abs())
            r = ratio.max().item()
            if r > worst:
                i = int(ratio.argmax())
                idx = [int(v) for v in torch.unravel_index(torch.tensor(i), ac.shape)]
                idx[dim] += c0
                worst, where = r, (idx, ac.flatten()[i].item(), bc.flatten()[i].item(), int((ratio > 1).sum()))
    r = num / den if den > 0 else num
    assert r <= tol["nrm"], f"{name}: max|a-b|/max|b| = {r:.3e} > {tol['nrm']:.1e}"
    if elementwise and worst > 1.0:
        idx, av, bv, nbad = where
        raise AssertionError(f"{name}: |a-b| > {tol['atol']} + {tol['rtol']}|b| at {idx}: a={av:.6g} b={bv:.6g} "
                             f"({worst:.3g}x the bound; {nbad}+ entries over it)")


class fp32_matmul_exact:
    """Context: torch's fp32 GEMMs at full fp32 precision (TF32 / reduced-precision paths off)."""

    def __enter__(self):
        self.prev = (torch.backends.cuda.matmul.allow_tf32, torch.get_float32_matmul_precision())
        torch.backends.cuda.matmul.allow_tf32 = False
        torch.set_float32_matmul_precision("highest")
        return self

    def __exit__(self, *exc):
        torch.backends.cuda.matmul.allow_tf32 = self.prev[0]
        torch.set_float32_matmul_precision(self.prev[1])
        return False


# Per-entry bound for the long reductions (lowrank dU, dz, dstatic_w; headwise
# dstatic_w) against b, the float64 sum of the terms formed from the same
# dtype-rounded inputs:
#     |a - b| <= k_in * L2 + k_acc * L1 + k_out * |b|
# with L1 = sum |term| and L2 = sqrt(sum term^2), both in float64.
#   k_in:  the per-term rounding before the sum.  The 16-bit lowrank backward
#          rounds dy*x to the I/O type before its products, as the reference
#          does for bf16 (lowrank.py:127-130; for fp16 the reference keeps fp32
#          products, lowrank.py:131-134, so there the rounding is this build's):
#          relative errors of at most u = 2^-8 (bf16) / 2^-11 (fp16) whose
#          standard deviation is below u/2, independent across terms, so their
#          sum is bounded statistically by L2: k_in = 4u is over 7 standard
#          deviations.  Headwise dstatic_w and fp32 have no such rounding.
#   k_acc: fp32 accumulation, 2^-20 of L1 (sequential fp32 sums of 512 to
#          131072 products stay within 1e-7 of L1, 10x below it).
#   k_out: the final rounding to the output dtype, 2u.
#   fp16's subnormal range (below 2^-14) rounds to absolute steps of 2^-24,
#   not relative ones: a rounded product dy*x there is off by at most 2^-25
#   times the other factor of its term (z for dU, U for dz), and an output by
#   at most 2^-25.  The fp16 bound adds 4 sqrt(n) 2^-25 max|other factor| over
#   the entry's n terms (the `floor` of lowrank_sums) and 2^-25.  bf16's
#   subnormals start at 2^-126 and do not matter at these magnitudes.
# A plausible kernel mistake fails it: a dropped 16-row tile of a 16384-row
# bf16 reduction moves an entry by about 4 rms(term); the bound there is about
# 2 rms(term) + |b| / 128.
SUM_TOL = {
    torch.bfloat16: dict(k_in=2.0**-6, k_acc=2.0**-20, k_out=2.0**-7),
    torch.float16: dict(k_in=2.0**-9, k_acc=2.0**-20, k_out=2.0**-10),
    torch.float32: dict(k_in=0.0, k_acc=2.0**-20, k_out=2.0**-23),
}


def assert_sum(a, ref, dtype, name, rounded_terms=True, floor=None):
    """Per-entry check of a long reduction `a` against ref = (b, L1, L2) (float64, CPU; see SUM_TOL).
    floor: fp16 only, the subnormal rounding of the terms (broadcast against b)."""
    b, l1, l2 = ref
    t = SUM_TOL[dtype]
    a = a.detach().double().cpu().reshape(b.shape)
    k_in = t["k_in"] if rounded_terms else 0.0
    bound = k_in * l2 + t["k_acc"] * l1 + t["k_out"] * b.abs()
    if dtype == torch.float16:
        bound = bound + 2.0**-25
        if rounded_terms and floor is not None:
            bound = bound + floor
    err = (a - b).abs()
    ratio = err / bound.clamp_min(1e-300)
    worst = ratio.max().item()
    if not worst <= 1.0:
        i = int(ratio.argmax())
        idx = [int(v) for v in torch.unravel_index(torch.tensor(i), b.shape)]
        raise AssertionError(
            f"{name}: |a-b| above the per-entry bound at {idx}: a={a.flatten()[i].item():.6g} "
            f"b={b.flatten()[i].item():.6g} bound={bound.flatten()[i].item():.3g} (err/bound {worst:.3g}; "
            f"{int((ratio > 1).sum())} of {ratio.numel()} entries)")


def _shift(x, k):
    if k == 0:
        return x
    out = torch.zeros_like(x)
    out[:, k:] = x[:, :-k]
    return out


def _sum3(parts):
    """(sum, L1, L2) of a list of (sum, L1, sum of squares) triples."""
    s = sum(p[0] for p in parts)
    return s, sum(p[1] for p in parts), torch.sqrt(sum(p[2] for p in parts))


def dstatic_sums(x, dy, W):
    """(b, L1, L2) of dstatic_w[k, d] = sum_{b,t} dy[b,t,d] x[b,t-k,d], float64 (inputs: rounded, CPU)."""
    x64, dy64 = x.detach().double().cpu(), dy.detach().double().cpu()
    rows = []
    for k in range(W):
        g = dy64 * _shift(x64, k)
        rows.append((g.sum((0, 1)), g.abs().sum((0, 1)), (g * g).sum((0, 1))))
    return (torch.stack([r[0] for r in rows]), torch.stack([r[1] for r in rows]),
            torch.sqrt(torch.stack([r[2] for r in rows])))


def lowrank_sums(x, z, U, dy):
    """(b, L1, L2) of the lowrank backward's reductions, float64 on the CPU from the rounded inputs:
    dU[r, kD+d] = sum_{b,t} z[b,t,r] G_k[b,t,d] and dz[b,t,r] = sum_{k,d} G_k[b,t,d] U[r, kD+d], where
    G_k = dy * x shifted by k rows (reference.py:23-39 differentiated)."""
    x64, dy64 = x.detach().double().cpu(), dy.detach().double().cpu()
    z64, U64 = z.detach().double().cpu(), U.detach().double().cpu()
    Bn, Tn, Dn = x64.shape
    R = z64.shape[-1]
    W = U64.shape[1] // Dn
    zf = z64.reshape(-1, R)
    dU, dz = [], []
    for k in range(W):
        G = (dy64 * _shift(x64, k)).reshape(-1, Dn)
        Ga, G2 = G.abs(), G * G
        dU.append((zf.t() @ G, zf.abs().t() @ Ga, (zf * zf).t() @ G2))
        Uk = U64[:, k * Dn:(k + 1) * Dn]
        dz.append((G @ Uk.t(), Ga @ Uk.abs().t(), G2 @ (Uk * Uk).t()))
        del G, Ga, G2
    dU = tuple(torch.cat([p[i] for p in dU], dim=1) for i in range(3))
    dU = (dU[0], dU[1], torch.sqrt(dU[2]))
    dz = _sum3(dz)
    # fp16 subnormal floor of the rounded products (see SUM_TOL): dU[r, :] has B*T terms whose other
    # factor is z[:, r]; dz[b, t, r] has W*D terms whose other factor is U[r, :]
    sub = 4 * 2.0**-25
    floor_du = (sub * math.sqrt(Bn * Tn) * zf.abs().amax(0)).reshape(R, 1)
    floor_dz = (sub * math.sqrt(W * Dn) * U64.abs().amax(1)).reshape(1, 1, R)
    return {"dU": dU, "dz": tuple(t.reshape(Bn, Tn, R) for t in dz), "floor_dU": floor_du, "floor_dz": floor_dz}


def check_reductions(kind, src_q, dyq, grads, dtype, tag=""):
    """Per-entry bounds (assert_sum) on the long reductions of one case: headwise ("hw") dstatic_w,
    lowrank ("lr") dz, dU and dstatic_w.  src_q: the dtype-rounded inputs (fp32, CPU) in the
    operator's argument order; grads: the kernel's gradients in the same order."""
    x = src_q[0]
    if kind == "hw":
        W = src_q[1].shape[-1]
        if src_q[2] is not None:
            assert_sum(grads[2], dstatic_sums(x, dyq, W), dtype, tag + "dstatic_w", rounded_terms=False)
        return
    z, U, sw = src_q[1], src_q[2], src_q[3]
    ref = lowrank_sums(x, z, U, dyq)
    assert_sum(grads[1], ref["dz"], dtype, tag + "dz", floor=ref["floor_dz"])
    assert_sum(grads[2], ref["dU"], dtype, tag + "dU", floor=ref["floor_dU"])
    if sw is not None:
        W = U.shape[1] // x.shape[-1]
        # the static rank's other factor is 1: B*T terms
        assert_sum(grads[3], dstatic_sums(x, dyq, W), dtype, tag + "dstatic_w",
                   floor=4 * 2.0**-25 * math.sqrt(x.shape[0] * x.shape[1]))


def run_fwd_bwd(fn, inputs, dy, residual):
    """Run fn(*inputs) forward+backward; return (y, [grads]) (grads None for None inputs)."""
    leaves = [t.detach().clone().requires_grad_() if t is not None else None for t in inputs]
    y = fn(*leaves, residual=residual)
    y.backward(dy)
    return y.detach(), [t.grad if t is not None else None for t in leaves]
