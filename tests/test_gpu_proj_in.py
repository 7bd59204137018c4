"""The proj_in GEMM kernels (dc_proj_in_fwd / dc_proj_in_bwd) against float64 sums on the CPU.

README.md:67, 75: z = proj_in(pre_z) with proj_in = nn.Linear(d_model, R, bias=False), for G
modules at once (the grouped q / k / v module: W_in rows g*R .. g*R+R-1 are group g's).  With
pre_z [M, K], W_in [N = G*R, K] and dz the G gradients side by side:

    z = pre_z W_in^T,   dpre_z = dz W_in,   dW_in = dz^T pre_z

Each output entry is checked against the float64 sum of its terms from the same 16-bit inputs with
helpers.assert_sum (no per-term rounding: a product of two 16-bit values is exact in fp32; fp32
accumulation; the output's rounding).  Shapes cover configs[4]'s (B2 T8192 D4096, 3 x 31 ranks),
the README module's, M and K off the tile sizes, N up to the 128 maximum, fp16.  The autograd
Function (dynconv.modules._ProjInFn) is checked against the same references, and dW_in twice for
bitwise determinism.
"""

import pytest
import torch

from helpers import assert_sum, gen, randn
from dynconv import _capi
from dynconv.modules import _ProjInFn, _proj_in_native

pytestmark = pytest.mark.gpu

DEV = "cuda"

CASES = [
    # G, B, T, K, R, dtype
    (3, 2, 8192, 4096, 31, torch.bfloat16),   # configs[4]: the grouped q|k|v module
    (1, 4, 4096, 2048, 15, torch.bfloat16),   # one README module at the B4 shape
    (3, 1, 37, 256, 15, torch.bfloat16),      # M not a multiple of 16
    (2, 3, 50, 200, 7, torch.float16),        # K not a multiple of 128 (K % 8 == 0), fp16
    (4, 1, 100, 1032, 32, torch.bfloat16),    # N = 128, the maximum
    (1, 2, 33, 8, 1, torch.bfloat16),         # one 8-channel piece, rank 1
    (3, 2, 300, 512, 21, torch.float16),      # N = 63
]


def _sums(a, b):
    """(a @ b, |a| @ |b|, sqrt(a^2 @ b^2)) in float64."""
    return a @ b, a.abs() @ b.abs(), torch.sqrt((a * a) @ (b * b))


@pytest.mark.parametrize("G,Bn,Tn,K,R,dtype", CASES)
def test_proj_in_against_float64(G, Bn, Tn, K, R, dtype):
    print(f"[proj_in] G{G} B{Bn} T{Tn} K{K} R{R} {dtype}", flush=True)
    g = gen(G * 7 + Tn + K + R)
    M, N = Bn * Tn, G * R
    pre = randn(g, Bn, Tn, K).to(dtype)
    w = randn(g, N, K, scale=K ** -0.5).to(dtype)
    dzs = [randn(g, Bn, Tn, R).to(dtype) for _ in range(G)]
    pre_d, w_d = pre.to(DEV), w.to(DEV)
    dz_d = [d.to(DEV) for d in dzs]
    assert _proj_in_native(pre_d, w_d, G, R)
    lib = _capi.load()
    p = _capi.ptr
    dt = _capi.dtype_code(dtype)
    st = _capi.stream_of(pre_d)
    zs = [torch.empty(Bn, Tn, R, dtype=dtype, device=DEV) for _ in range(G)]
    _capi.check(lib.dc_proj_in_fwd(p(pre_d), p(w_d), _capi.ptr_array(zs), G, M, K, R, dt, st), "fwd")
    dpre = torch.empty_like(pre_d)
    dws = []
    for _ in range(2):
        dw = torch.empty_like(w_d)
        nws = lib.dc_proj_in_bwd_ws_bytes(G, M, K, R, dt)
        ws = torch.full((nws,), 0x5A, dtype=torch.uint8, device=DEV)  # contents on entry do not matter
        _capi.check(lib.dc_proj_in_bwd(p(pre_d), p(w_d), _capi.ptr_array(dz_d), p(dpre), p(dw), p(ws), nws,
                                       G, M, K, R, dt, st), "bwd")
        dws.append(dw)
    torch.cuda.synchronize()
    assert torch.equal(dws[0], dws[1]), "dW_in differs between two identical calls"

    pre64 = pre.double().reshape(M, K)
    w64 = w.double()
    dz64 = torch.cat([d.double().reshape(M, R) for d in dzs], dim=1)
    zref = _sums(pre64, w64.t())
    z_k = torch.cat([z.reshape(M, R) for z in zs], dim=1)
    assert_sum(z_k, zref, dtype, "z", rounded_terms=False)
    assert_sum(dpre.reshape(M, K), _sums(dz64, w64), dtype, "dpre_z", rounded_terms=False)
    assert_sum(dws[0], _sums(dz64.t(), pre64), dtype, "dW_in", rounded_terms=False)

    # the autograd Function: same kernels, same values
    pre_a = pre_d.clone().requires_grad_()
    w_a = w_d.clone().requires_grad_()
    za = _ProjInFn.apply(pre_a, w_a, G, R)
    torch.autograd.backward(za, dz_d)
    torch.cuda.synchronize()
    for a, b in zip(za, zs):
        assert torch.equal(a, b)
    assert torch.equal(pre_a.grad, dpre)
    assert torch.equal(w_a.grad, dws[0])
