"""Shared test helpers: seeded inputs, tolerance checks, library loading."""

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


def run_fwd_bwd(fn, inputs, dy, residual):
    """Run fn(*inputs) forward+backward; return (y, [grads]) (grads None for None inputs)."""
    leaves = [t.detach().clone().requires_grad_() if t is not None else None for t in inputs]
    y = fn(*leaves, residual=residual)
    y.backward(dy)
    return y.detach(), [t.grad if t is not None else None for t in leaves]
