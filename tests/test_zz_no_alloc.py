"""The allocation-free headwise backward, dc_headwise_bwd_noalloc, against dc_headwise_bwd.

dc_headwise_bwd_noalloc runs the same kernels with the workspace (the fp32
dstatic_w partial sums) in a fixed device array of the library instead of a
caller's allocation.  Through the C ABI, on consecutive calls whose second
input is smaller than the first (the array keeps the last call's contents),
its outputs must equal dc_headwise_bwd's bitwise: with and without static_w,
on the vector kernels, the wide ones (W 9-32), the head matrix-core ones (head
size 32 at W 12) and the generic ones (head size 3, W 48).
"""

import pytest
import torch

from helpers import gen, randn
from dynconv import _capi

pytestmark = pytest.mark.gpu

DEV = "cuda"

# B, T, D, H, W, static, residual: each list runs its calls in order, larger first
SEQUENCES = [
    [(4, 1024, 2048, 64, 4, True, True), (2, 300, 512, 512, 3, True, False)],   # vector kernels
    [(2, 500, 1024, 1024, 4, True, True), (1, 77, 96, 32, 5, True, True)],     # then head size 3: generic
    [(2, 256, 512, 16, 4, False, True), (1, 64, 256, 8, 2, False, False)],     # no static_w: no scratch
    [(2, 300, 512, 512, 12, True, True), (1, 70, 256, 8, 9, True, False),      # W 9-32: wide kernels
     (1, 50, 128, 32, 24, True, True)],
    [(2, 300, 512, 16, 12, True, True), (1, 90, 256, 8, 48, True, False)],    # head matrix cores, then W 48: generic
]


def _inputs(Bn, Tn, Dn, H, W, static, dtype, seed):
    g = gen(seed)
    x = randn(g, Bn, Tn, Dn).to(dtype).to(DEV)
    w = randn(g, Bn, Tn, H, W, scale=0.5).to(dtype).to(DEV)
    sw = randn(g, W, Dn, scale=0.3).to(dtype).to(DEV) if static else None
    dy = randn(g, Bn, Tn, Dn).to(dtype).to(DEV)
    return x, w, sw, dy


def _outputs(x, w, sw):
    return torch.empty_like(x), torch.empty_like(w), (torch.empty_like(sw) if sw is not None else None)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("seq", range(len(SEQUENCES)))
def test_noalloc_matches_workspace_entry_point(seq, dtype):
    lib = _capi.load()
    p = _capi.ptr
    dt = _capi.dtype_code(dtype)
    st = _capi.stream_of(torch.empty(1, device=DEV))
    for i, (Bn, Tn, Dn, H, W, static, residual) in enumerate(SEQUENCES[seq]):
        print(f"[noalloc] seq {seq} call {i}: B{Bn} T{Tn} D{Dn} H{H} W{W} static={static} {dtype}", flush=True)
        x, w, sw, dy = _inputs(Bn, Tn, Dn, H, W, static, dtype, seed=100 * seq + i)
        need = lib.dc_headwise_bwd_ws_bytes(Bn, Tn, Dn, H, W, dt, int(static))
        assert 0 <= need <= 8 << 20
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=DEV)
        ref = _outputs(x, w, sw)
        _capi.check(lib.dc_headwise_bwd(p(x), p(w), p(sw), p(dy), p(ref[0]), p(ref[1]), p(ref[2]), p(ws), need,
                                        Bn, Tn, Dn, H, W, dt, int(residual), st), "dc_headwise_bwd")
        got = _outputs(x, w, sw)
        _capi.check(lib.dc_headwise_bwd_noalloc(p(x), p(w), p(sw), p(dy), p(got[0]), p(got[1]), p(got[2]),
                                                Bn, Tn, Dn, H, W, dt, int(residual), st), "dc_headwise_bwd_noalloc")
        torch.cuda.synchronize()
        for name, a, b in zip(("dx", "dweight", "dstatic_w"), got, ref):
            if b is not None:
                assert torch.equal(a, b), f"call {i}: {name} differs from dc_headwise_bwd"
