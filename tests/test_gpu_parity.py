"""GPU parity: the HIP kernels against the CPU oracle (oracle/reference_cpu.py).

* test_reference_sweep reproduces test.py's 48-config sweep (test.py:9-58):
  dtype {bf16, fp32} x residual x W {2, 4} x {headwise hs {1, 16} x static;
  lowrank R=16 x static}, B,T,D = 2,512,256, inputs scaled as test.py:36-54.
  Each case is checked twice:
    1. test.py's own criterion (test.py:17, 59-69): oracle on the unrounded
       fp32 inputs, kernel on inputs cast to dtype, assert_close(TOL[dtype]);
    2. the north-star criterion: oracle in fp32 on the same dtype-rounded
       inputs; max|a-b|/max|b| <= 2e-2 (bf16) / 1e-5 (fp32) for every output
       and |a-b| <= 2e-2 + 2e-2|b| elementwise for y, dx, dweight.
* test_edge_shapes covers head sizes 1..1024 (vector and generic paths),
  W = 1..8, W > T, T = 1, odd T, D not a multiple of the vector width, fp16,
  ranks 1..63 (+ static) including ranks the Python API rejects (reached
  through the autograd Function directly, i.e. the C ABI's general case).
* test_baseline_configs runs BASELINE.json configs 2-5 at full size and
  checks every row of the local outputs (y, dx, dweight) elementwise against
  the oracle run over the whole tensors on the GPU (fp32, TF32 off), dz
  norm-wise against it, and the global reductions (dz, dU, dstatic_w) entry
  by entry against float64 sums.
* test_headwise_mixed_dtypes: weight / static_w in other dtypes than x, each
  gradient in its own tensor's dtype, against the oracle.
* test_generic_lowrank_rows_past_2_24: the generic lowrank backward over more
  than 2^24 rows (its capped dz grid).
* test_deterministic: two backward passes are bitwise identical.
"""

import itertools
import math
import zlib

import pytest
import torch

from helpers import (REF_TOL, assert_ns, assert_ns_full, assert_sum, check_reductions, dstatic_sums, fp32_matmul_exact,
                     gen, lowrank_sums, max_rel, randn, run_fwd_bwd, uniform)
from oracle.reference_cpu import (
    headwise_dynamic_convolution_ref as hw_ref,
    lowrank_dynamic_convolution_ref as lr_ref,
)
import headwise as hw_mod
import lowrank as lr_mod

hw = hw_mod.headwise_dynamic_convolution
lr = lr_mod.lowrank_dynamic_convolution

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _to(t, dtype):
    return None if t is None else t.to(dtype).to(DEV)


def _f32cpu(t):
    return None if t is None else t.detach().float().cpu()


def _check_case(kernel, ref, src, dy, dtype, residual, names, local, kind):
    """Run both criteria for one case.  src: fp32 CPU tensors (None allowed)."""
    # 1. test.py criterion
    atol, rtol = REF_TOL[dtype]
    y_r, g_r = run_fwd_bwd(ref, src, dy, residual)
    y_k, g_k = run_fwd_bwd(kernel, [_to(t, dtype) for t in src], _to(dy, dtype), residual)
    pairs = [(y_k, y_r, "y")] + [(a, b, n) for a, b, n in zip(g_k, g_r, names) if b is not None]
    for a, b, n in pairs:
        torch.testing.assert_close(a.float().cpu(), b.float(), atol=atol, rtol=rtol, msg=lambda m: f"[test.py] {n}: {m}")
    # 2. north-star criterion on the rounded inputs
    src_q = [None if t is None else t.to(dtype).float() for t in src]
    y_q, g_q = run_fwd_bwd(ref, src_q, dy.to(dtype).float(), residual)
    assert_ns(y_k, y_q, dtype, "y")
    for a, b, n in zip(g_k, g_q, names):
        if b is not None:
            assert_ns(a, b, dtype, n, elementwise=n in local)
    # 3. per-entry bounds on the long reductions (float64 sums of the same rounded terms)
    check_reductions(kind, src_q, dy.to(dtype).float(), [None] + g_k[1:], dtype)


# ----------------------------------------------------------- test.py sweep
B, T, D = 2, 512, 256
SWEEP = list(itertools.product([torch.bfloat16, torch.float32], [False, True], [2, 4],
                               ["hw1", "hw16", "lr16"], [False, True]))


@pytest.mark.parametrize("dtype,residual,W,kind,static", SWEEP,
                         ids=[f"{str(d)[6:]}-res{int(r)}-W{w}-{k}-st{int(s)}" for d, r, w, k, s in SWEEP])
def test_reference_sweep(dtype, residual, W, kind, static):
    g = gen(zlib.crc32(f"{dtype}-{residual}-{W}-{kind}-{static}".encode()))
    x = randn(g, B, T, D)
    dy = randn(g, B, T, D)
    sw = randn(g, W, D, scale=0.1) if static else None
    if kind.startswith("hw"):
        hs = int(kind[2:])
        w = randn(g, B, T, D // hs, W, scale=0.1)
        _check_case(hw, hw_ref, [x, w, sw], dy, dtype, residual, ["dx", "dweight", "dstatic_w"], {"dx", "dweight"},
                    "hw")
    else:
        R = 16
        z = randn(g, B, T, R, scale=0.1 / R**0.5)
        U = randn(g, R, W * D)
        if static:
            z, U = z[..., :-1].contiguous(), U[:-1].contiguous()
        _check_case(lr, lr_ref, [x, z, U, sw], dy, dtype, residual, ["dx", "dz", "dU", "dstatic_w"], {"dx"}, "lr")


# -------------------------------------------------------------- edge shapes
HW_EDGE = [
    # B, T, D, H, W, static, residual, dtype
    (1, 37, 64, 64, 3, True, True, torch.bfloat16),     # hs 1, odd T, W 3
    (2, 100, 128, 4, 5, False, True, torch.bfloat16),   # hs 32, W 5
    (1, 64, 256, 128, 4, True, False, torch.bfloat16),  # hs 2
    (1, 64, 256, 64, 4, True, False, torch.bfloat16),   # hs 4
    (1, 64, 256, 32, 6, True, True, torch.bfloat16),    # hs 8
    (1, 64, 1024, 2, 8, True, False, torch.bfloat16),   # hs 512: a head spans a whole wavefront
    (1, 40, 2048, 2, 4, True, True, torch.bfloat16),    # hs 1024: generic path
    (2, 50, 96, 96, 4, True, True, torch.float16),      # fp16, D not a multiple of 64*VEC
    (1, 20, 12, 4, 2, True, True, torch.bfloat16),      # D % 8 != 0 and hs 3: generic path
    (2, 33, 64, 16, 1, True, True, torch.float32),      # W 1
    # fp32 W 8: a lane's dweight piece is 32 bytes; heads over 2 and 8 lanes
    # must sum across lanes before the store (found by the random sweep)
    (1, 40, 128, 16, 8, True, False, torch.float32),
    (2, 33, 256, 8, 8, False, True, torch.float32),
    (1, 37, 128, 32, 8, True, True, torch.float32),     # hs 4: one lane per head, transposed store
    (1, 5, 64, 64, 8, True, True, torch.bfloat16),      # W > T
    (1, 1, 64, 8, 4, True, True, torch.bfloat16),       # T 1
    (3, 129, 200, 50, 7, True, True, torch.float32),    # hs 4 fp32, W 7, D % 64*4 != 0
    # one 320-channel head (generic kernels), fp32: dweight's head sum must stay
    # within the elementwise 1e-5 bar (found by the random sweep)
    (3, 200, 320, 1, 8, False, True, torch.float32),
    # whole wavefronts with lanes that own whole heads: weight rows loaded as
    # contiguous 1 KiB instructions and handed to the lanes through LDS
    # (pieces of NP = 2, 3, 4 units), runs of several chunks
    (2, 300, 512, 512, 3, True, True, torch.float16),   # hs 1, W 3: NP 3
    (1, 260, 256, 256, 2, False, True, torch.float32),  # hs 1 fp32, W 2: NP 2
    (2, 181, 512, 256, 4, True, False, torch.bfloat16), # hs 2, W 4: NP 2
    (1, 333, 1024, 1024, 4, True, True, torch.bfloat16),  # hs 1, W 4: NP 4, two wavefront columns
    # widths above 8 (the reference accepts any W, headwise.py:226): 9 <= W <= 16 on the wide
    # row-ring kernels when D % 128 == 0 and a head lies in one wavefront, else the generic ones
    (1, 50, 64, 16, 12, True, True, torch.bfloat16),   # W 12, D 64: generic
    (2, 40, 128, 128, 16, True, False, torch.float32),  # W 16, head size 1: wide
    (1, 10, 64, 32, 32, True, True, torch.bfloat16),   # W 32 (the maximum) > T: wide, one channel per lane
    # 17 <= W <= 32: one channel per lane (64-channel wavefronts), head sums over a run-time group
    (2, 77, 128, 128, 17, True, True, torch.bfloat16),  # hs 1
    (1, 100, 256, 64, 20, False, True, torch.float16),  # hs 4
    (2, 61, 256, 8, 24, True, False, torch.float32),    # hs 32
    (1, 130, 128, 2, 32, True, True, torch.bfloat16),   # hs 64: a head is a whole wavefront
    (1, 90, 128, 64, 25, True, True, torch.bfloat16),   # hs 2, odd W
    (1, 1, 64, 16, 28, True, True, torch.float16),      # T 1
    (1, 50, 96, 96, 20, True, True, torch.bfloat16),    # D % 64 != 0: generic
    (2, 77, 256, 256, 9, True, True, torch.bfloat16),   # wide: hs 1, odd W (ring of W + 1 rows)
    (1, 100, 128, 64, 10, False, True, torch.float16),  # wide: hs 2
    (2, 61, 384, 96, 11, True, False, torch.float32),   # wide: hs 4, three wavefront columns
    (1, 130, 256, 8, 12, True, True, torch.bfloat16),   # wide: hs 32
    (2, 45, 256, 2, 13, True, True, torch.float32),     # wide: hs 128 (a head is a whole wavefront)
    (1, 90, 128, 16, 14, False, False, torch.float32),  # wide: hs 8 (16-bit types: matrix cores)
    (1, 7, 128, 128, 15, True, True, torch.float16),    # wide: T < W
    (2, 200, 256, 32, 16, True, True, torch.float32),   # wide: hs 8, W 16
    (1, 1, 128, 64, 16, True, True, torch.bfloat16),    # wide: T 1
    (1, 50, 256, 2, 9, True, True, torch.bfloat16),     # hs 128 bf16 W 9: 18-byte weight segments, generic
    # fp16 W 16 head size 1 without a static filter: the dx of every row 16k + 15 came out wrong.
    # The row resources were built from vector registers, every access went through a per-lane
    # descriptor loop, and two register copies landed where no lane was enabled (found by a random
    # sweep; resources now uniform by construction).  Also the same shape with the residual and in bf16.
    (1, 40, 256, 256, 16, False, False, torch.float16),
    (2, 64, 128, 128, 16, False, True, torch.float16),
    (1, 40, 256, 256, 16, False, True, torch.bfloat16),
    # the head matrix-core kernels (head sizes 8, 16, 32, 64 at 9 <= W <= 32, whole 16-byte pieces of
    # a wavefront's weight-row segment): dw on MFMA over the head's channels, the head weights' part
    # of dx as a banded product, the static filter by row pairs; runs of 16-row tiles, T not a
    # multiple of 16, T below one tile, runs ending at T
    (2, 77, 256, 8, 24, True, True, torch.bfloat16),    # hs 32, W 24 (two look-back blocks)
    (1, 100, 128, 4, 12, False, True, torch.float16),   # hs 32, W 12, no static filter
    (1, 33, 128, 8, 10, True, False, torch.bfloat16),   # hs 16, W 10 (one look-back block)
    (2, 50, 192, 12, 32, True, True, torch.float16),    # hs 16, W 32, three wavefront columns
    # head size 8: two heads per 16-channel block, one product per head with the other head's
    # channels zeroed (dw: its K quarters, dx / y: its output columns)
    (1, 90, 128, 16, 14, False, False, torch.bfloat16), # hs 8, W 14
    (2, 200, 256, 32, 16, True, True, torch.float16),   # hs 8, W 16
    (1, 77, 256, 32, 9, True, True, torch.bfloat16),    # hs 8, W 9 (odd)
    (2, 61, 192, 24, 17, True, False, torch.float16),   # hs 8, W 17: two look-back blocks, three columns
    (1, 130, 256, 32, 24, False, True, torch.bfloat16), # hs 8, W 24: three wavefronts per CU by LDS
    (1, 10, 128, 16, 32, True, True, torch.bfloat16),   # hs 8, W 32 > T
    (1, 70, 128, 2, 16, True, True, torch.bfloat16),    # hs 64, W 16
    (1, 9, 64, 1, 24, True, True, torch.bfloat16),      # hs 64, W 24 > T
    (1, 1, 128, 4, 28, True, False, torch.bfloat16),    # hs 32, T 1
    (3, 300, 128, 8, 18, False, True, torch.bfloat16),  # hs 16, W 18: two look-ahead blocks, runs of tiles
    (1, 1000, 64, 2, 32, True, True, torch.float16),    # hs 32, W 32, runs of one tile
    (2, 2000, 2048, 64, 32, True, True, torch.float16), # hs 32, W 32, runs of 7-8 tiles, 32 wavefront columns
    (2, 64, 128, 4, 20, True, True, torch.bfloat16),    # hs 32, W 20, T a multiple of 16
    # W 33 .. DC_MAX_W (the reference takes any W, headwise.py:226): the generic kernels
    (1, 70, 128, 128, 33, True, True, torch.bfloat16),  # hs 1, W 33
    (2, 50, 128, 4, 48, True, False, torch.float16),    # hs 32, W 48
    (1, 40, 64, 2, 64, False, True, torch.float32),     # hs 32 fp32, W 64 > T
    (1, 300, 64, 16, 100, True, True, torch.bfloat16),  # hs 4, W 100
]


@pytest.mark.parametrize("Bn,Tn,Dn,H,W,static,residual,dtype", HW_EDGE)
def test_edge_shapes_headwise(Bn, Tn, Dn, H, W, static, residual, dtype):
    g = gen(Bn * 1000003 + Tn * 1009 + Dn * 7 + H + W)
    want = ("vector" if W <= 8 and _hw_vector_shape(Dn, H, dtype)
            else "wide" if _hw_wide_shape(Dn, H, W, dtype) else "generic")
    if want != "vector" and _hw_mma_shape(Dn, H, W, dtype):
        want = "head_mfma"
    for bwd in (0, 1):
        assert _path("hw", Bn, Tn, Dn, H, W, dtype, static, bwd) == want
    x = randn(g, Bn, Tn, Dn)
    dy = randn(g, Bn, Tn, Dn)
    w = randn(g, Bn, Tn, H, W, scale=1 / math.sqrt(W))
    sw = uniform(g, W, Dn, lo=-1 / math.sqrt(W), hi=1 / math.sqrt(W)) if static else None
    src = [x, w, sw]
    src_q = [None if t is None else t.to(dtype).float() for t in src]
    y_q, g_q = run_fwd_bwd(hw_ref, src_q, dy.to(dtype).float(), residual)
    y_k, g_k = run_fwd_bwd(hw, [_to(t, dtype) for t in src], _to(dy, dtype), residual)
    assert_ns(y_k, y_q, dtype, "y")
    for a, b, n in zip(g_k, g_q, ["dx", "dweight", "dstatic_w"]):
        if b is not None:
            assert_ns(a, b, dtype, n, elementwise=n != "dstatic_w")
    check_reductions("hw", src_q, dy.to(dtype).float(), g_k, dtype)


HW_MIXED = [
    # B, T, D, H, W, static, residual, x dtype, weight dtype, static_w dtype
    (2, 70, 256, 256, 4, True, True, torch.bfloat16, torch.float32, torch.bfloat16),   # hs 1
    (1, 64, 512, 32, 3, True, False, torch.bfloat16, torch.float32, torch.float32),    # hs 16
    (2, 33, 128, 32, 4, False, True, torch.float32, torch.bfloat16, None),             # hs 4, fp32 x
    (1, 50, 256, 32, 4, True, True, torch.float16, torch.bfloat16, torch.float32),     # two 16-bit types
]


@pytest.mark.parametrize("Bn,Tn,Dn,H,W,static,residual,xd,wd,sd", HW_MIXED)
def test_headwise_mixed_dtypes(Bn, Tn, Dn, H, W, static, residual, xd, wd, sd):
    """weight / static_w in other dtypes than x, as the reference accepts (it loads them in fp32,
    headwise.py:63, 78, 180, 187, and returns dweight and dstatic_w in their own dtypes,
    headwise.py:268, 305): the oracle in fp32 on the same rounded inputs; every output carries
    its own tensor's dtype and is checked to that dtype's bar."""
    g = gen(Bn * 7919 + Tn * 31 + Dn + H + W)
    x = randn(g, Bn, Tn, Dn)
    dy = randn(g, Bn, Tn, Dn)
    w = randn(g, Bn, Tn, H, W, scale=1 / math.sqrt(W))
    sw = uniform(g, W, Dn, lo=-1 / math.sqrt(W), hi=1 / math.sqrt(W)) if static else None
    dts = [xd, wd, sd]
    src_q = [None if t is None else t.to(d).float() for t, d in zip([x, w, sw], dts)]
    y_q, g_q = run_fwd_bwd(hw_ref, src_q, dy.to(xd).float(), residual)
    y_k, g_k = run_fwd_bwd(hw, [None if t is None else t.to(d).to(DEV) for t, d in zip([x, w, sw], dts)],
                           _to(dy, xd), residual)
    assert y_k.dtype == xd
    assert_ns(y_k, y_q, xd, "y")
    for a, b, n, d in zip(g_k, g_q, ["dx", "dweight", "dstatic_w"], dts):
        if b is not None:
            assert a.dtype == d, f"{n}: {a.dtype} != {d}"
            assert_ns(a, b, d, n, elementwise=n != "dstatic_w")


def _hw_vector_shape(Dn, H, dtype):
    """Shapes the headwise vector kernels take (contiguous, aligned tensors): D a multiple of the
    16-byte lane width, a power-of-two head size of at most 64 lanes."""
    vec = 16 // torch.tensor([], dtype=dtype).element_size()
    hs = Dn // H
    return Dn % vec == 0 and hs & (hs - 1) == 0 and hs <= 64 * vec


def _hw_mma_shape(Dn, H, W, dtype):
    """Shapes the head matrix-core kernels take (contiguous, aligned tensors): bf16 / fp16, head
    sizes 8, 16, 32, 64 at 9 <= W <= 32 with whole 16-byte pieces of a 64-channel wavefront's
    weight-row segment ((64 / hs) * W a multiple of 8), D a multiple of 64."""
    hs = Dn // H
    return (dtype in (torch.bfloat16, torch.float16) and hs in (8, 16, 32, 64) and 9 <= W <= 32
            and (64 // hs) * W % 8 == 0 and Dn % 64 == 0)


def _hw_wide_shape(Dn, H, W, dtype):
    """Shapes the headwise wide kernels take (contiguous, aligned tensors): 9 <= W <= 32, D a multiple
    of a wavefront's channels (128: two per lane up to W 16; 64 above), a power-of-two head size of at
    most that, and weight-row segments (a wavefront's heads, and a whole row) of whole 16-byte pieces."""
    es = torch.tensor([], dtype=dtype).element_size()
    hs = Dn // H
    cols = 128 if W <= 16 else 64
    return (9 <= W <= 32 and Dn % cols == 0 and hs & (hs - 1) == 0 and hs <= cols
            and (cols // hs) * W * es % 16 == 0 and H * W * es % 16 == 0)


def _path(kind, Bn, Tn, Dn, HR, W, dtype, static, bwd):
    """Kernel family (dc_headwise_path / dc_lowrank_path) a call of this shape runs on."""
    from dynconv import _capi

    lib = _capi.load()
    fn = lib.dc_headwise_path if kind == "hw" else lib.dc_lowrank_path
    code = fn(Bn, Tn, Dn, HR, W, _capi.dtype_code(dtype), int(static), bwd)
    assert code >= 0, _capi.status_string(code)
    return _capi.PATHS[code]


LR_EDGE = [
    # B, T, D, R, W, static, residual, dtype, (forward, backward) kernel family
    (1, 37, 256, 16, 3, False, True, torch.bfloat16),
    (2, 70, 128, 31, 4, True, True, torch.bfloat16),    # kernel rank 32
    (1, 64, 256, 32, 2, False, False, torch.bfloat16),
    (1, 48, 128, 63, 4, True, True, torch.bfloat16),    # kernel rank 64 (the maximum)
    (2, 40, 64, 7, 5, True, False, torch.float16),      # kernel rank 8
    (1, 33, 96, 1, 8, False, True, torch.bfloat16),     # rank 1, W 8
    (1, 3, 128, 16, 4, False, True, torch.bfloat16),    # W > T
    (2, 21, 40, 4, 3, True, True, torch.float32),       # D % 8 != 0
    (1, 50, 64, 3, 4, False, True, torch.bfloat16),     # rank 3: C-ABI general case
    (1, 50, 64, 5, 2, True, True, torch.float32),       # kernel rank 6: C-ABI general case
    # backward plans with an odd run count (the last 8-wavefront workgroup's
    # second run is empty) and a short last run: 201 tiles in runs of 2
    (3, 3216, 256, 16, 4, False, True, torch.bfloat16),
    (3, 3216, 256, 31, 4, True, True, torch.bfloat16),  # two rank chunks: 32-channel tiles
    (2, 1000, 272, 15, 3, True, False, torch.float16),  # D not a multiple of 256: partial channel groups
    # fp32 kernels: ranks padded to 8 / 16 / 32, partial channel groups, runs of 16+ rows
    (2, 1000, 272, 15, 3, True, False, torch.float32),
    (1, 70, 128, 31, 4, True, True, torch.float32),     # kernel rank 32
    (2, 300, 64, 1, 1, False, True, torch.float32),     # rank 1, W 1
    (1, 9, 100, 7, 4, False, True, torch.float32),      # T below one run, D % 64 != 0
    (1, 40, 64, 40, 4, False, False, torch.float32, ("f32_mfma", "f32_mfma")),   # kernel rank 40: rank passes
    (2, 100, 128, 63, 6, True, True, torch.float32, ("f32_mfma", "f32_mfma")),   # kernel rank 64, 3 + 3 taps
    # static rank alone in the second rank pass of the forward, W 12 (its later tap pass has no U rows:
    # their buffer range must be empty, not negative)
    (1, 60, 64, 32, 12, True, True, torch.float32, ("f32_mfma", "f32_mfma")),
    # fp32 kernel ranks 17-32: the matrix-core backward as two rank passes (ranks 0-15, then the
    # rest; the second pass adds its dx to the first's and its dz columns / dU rows are its own)
    (2, 300, 256, 31, 4, True, True, torch.float32, ("f32_mfma", "f32_mfma")),   # static rank in pass 2
    (1, 100, 128, 20, 3, False, True, torch.float32, ("f32_mfma", "f32_mfma")),  # pass 2 of 4 ranks
    (2, 1000, 272, 16, 2, True, False, torch.float32, ("f32_mfma", "f32_mfma")),  # pass 2: the static rank alone
    (1, 64, 64, 32, 4, False, True, torch.float32, ("f32_mfma", "f32_mfma")),    # kernel rank 32, no static
    # fp32 W 5-8: the matrix-core forward at any W <= 8; the backward as two tap passes (x shifted by
    # the second pass's first tap, dx added, dz partials per pass), with rank passes above 16
    (2, 300, 256, 16, 8, False, True, torch.float32, ("f32_mfma", "f32_mfma")),   # W 8: 4 + 4
    (1, 100, 128, 31, 5, True, True, torch.float32, ("f32_mfma", "f32_mfma")),    # W 5: 3 + 2, x 2 rank passes
    (2, 1000, 272, 7, 6, True, False, torch.float32, ("f32_mfma", "f32_mfma")),   # W 6: 3 + 3, long runs
    (1, 40, 64, 20, 7, False, True, torch.float32, ("f32_mfma", "f32_mfma")),     # W 7: 4 + 3, rank passes
    # fp32 W 9-32: the forward as passes of 8 taps (the first W - 8(n-1), later ones added to the
    # stored y), the backward as ceil(W / 4) passes of 2-4 taps (dx in fp32 throughout)
    (2, 300, 256, 16, 12, False, True, torch.float32, ("f32_mfma", "f32_mfma")),  # forward 4 + 8, 4+4+4
    (1, 100, 128, 31, 20, True, True, torch.float32, ("f32_mfma", "f32_mfma")),   # 5 tap x 2 rank passes
    (1, 3300, 64, 7, 32, True, False, torch.float32, ("f32_mfma", "f32_mfma")),   # W 32, long runs
    (1, 5, 64, 3, 9, False, True, torch.float32, ("f32_mfma", "f32_mfma")),       # W 9 > T
    # matrix-core plans with three and four rank chunks (kernel ranks 33-64 at W 1-2); from W 2 on,
    # kernel ranks 49-64 take the backward as passes of 32 ranks on the two-chunk kernels
    (1, 70, 128, 64, 1, False, True, torch.bfloat16, ("mfma", "mfma")),      # <W1, 4 chunks>
    (2, 50, 256, 63, 2, True, True, torch.bfloat16, ("mfma", "mfma")),       # <W2, kernel rank 64>: 2 rank passes
    (1, 40, 128, 40, 2, False, False, torch.float16, ("mfma", "mfma")),      # <W2, 3 chunks>
    (2, 60, 128, 40, 1, True, True, torch.bfloat16, ("mfma", "mfma")),       # <W1, 3 chunks>, kernel rank 41
    (1, 90, 128, 48, 4, True, True, torch.bfloat16, ("mfma", "mfma")),       # kernel rank 49: 32 + 16 and the static
    (2, 40, 256, 64, 3, False, False, torch.float16, ("mfma", "mfma")),      # 64 dynamic ranks: z itself, 2 passes
    (1, 77, 128, 52, 6, False, True, torch.bfloat16, ("mfma", "mfma")),      # kernel rank 52, W 6: 2 x 2 passes
    # wide W x rank: the backward runs passes of taps (x shifted by each pass's first tap,
    # dx accumulated, dz partials per pass), the forward stages every tap's operands
    (2, 70, 128, 31, 8, True, True, torch.bfloat16, ("mfma", "mfma")),       # W 8, 2 chunks: 2 passes
    (1, 100, 256, 20, 6, False, False, torch.bfloat16, ("mfma", "mfma")),    # W 6, 2 chunks: passes of 4 + 2
    (2, 45, 128, 40, 5, False, True, torch.float16, ("mfma", "mfma")),       # W 5, 3 chunks: passes 2 + 2 + 1
    (1, 60, 256, 63, 8, True, True, torch.bfloat16, ("mfma", "mfma")),       # W 8, 4 chunks: 8 passes of 1
    (1, 3216, 256, 31, 7, True, True, torch.bfloat16, ("mfma", "mfma")),     # W 7: passes of 4 + 3, long runs
    (2, 37, 64, 47, 3, True, False, torch.bfloat16, ("mfma", "mfma")),       # W 3, 3 chunks: passes 2 + 1
    # D a multiple of 8 but not of 16 on the matrix-core backward: the last 16-channel group and
    # 32-channel dz block half inside D (their other channels read 0 and store nothing)
    (2, 100, 200, 16, 4, False, True, torch.bfloat16, ("mfma", "mfma")),      # 64-channel tiles
    (1, 70, 40, 31, 4, True, True, torch.bfloat16, ("mfma", "mfma")),         # two rank chunks: 32-channel tiles
    (1, 50, 1000, 15, 3, True, False, torch.float16, ("mfma", "mfma")),       # partial channel group
    (2, 33, 24, 7, 8, True, True, torch.bfloat16, ("mfma", "mfma")),          # W 8 gather form
    (1, 64, 72, 63, 2, False, True, torch.bfloat16, ("mfma", "mfma")),        # four rank chunks, tap passes
    # 9 <= W <= 16 at one or two rank chunks: the forward in one pass (x rows back to 4q-15), the
    # backward as passes of at most 8 taps (one rank chunk) or 4 (two)
    (1, 9, 64, 8, 16, False, True, torch.bfloat16, ("mfma", "mfma")),          # W 16 > T
    (2, 300, 256, 16, 12, False, True, torch.bfloat16, ("mfma", "mfma")),      # passes 8 + 4
    (1, 520, 128, 15, 9, True, False, torch.float16, ("mfma", "mfma")),        # passes 8 + 1
    (2, 77, 200, 31, 16, True, True, torch.bfloat16, ("mfma", "mfma")),        # two rank chunks: 4 x 4 taps
    (1, 3300, 256, 3, 13, False, True, torch.bfloat16, ("mfma", "mfma")),      # long runs, padded z
    (1, 64, 512, 20, 10, True, True, torch.float16, ("mfma", "mfma")),         # kernel rank 21: passes 4 + 4 + 2
    # 17 <= W <= 32 at one or two rank chunks: the forward in one pass at one chunk (x rows up to
    # 4q-31, U chunks of all W taps in LDS), as two at two (taps 0 .. W-17, then the last 16 added
    # to the stored y, x read W-16 rows earlier), the backward as passes of 8 taps (one
    # rank chunk: at most 4, dx rounded after each) or 4 (two: 5-8 passes into the fp32 dx
    # accumulator); long runs reach back up to 31 rows before their first tile (the runs' 32-row halo)
    (1, 25, 64, 8, 20, False, True, torch.bfloat16, ("mfma", "mfma")),         # W 20 > T
    (2, 300, 256, 16, 17, True, True, torch.bfloat16, ("mfma", "mfma")),       # forward 1 + 16 taps
    (1, 3300, 256, 15, 32, True, True, torch.bfloat16, ("mfma", "mfma")),      # W 32: forward one pass, backward 4 x 8
    (2, 200, 128, 31, 24, True, False, torch.float16, ("mfma", "mfma")),       # two rank chunks, 8 + 16
    (1, 520, 200, 20, 28, False, True, torch.bfloat16, ("mfma", "mfma")),      # D % 16 != 0, 12 + 16
    (1, 3216, 64, 31, 25, True, True, torch.float16, ("mfma", "mfma")),        # long runs, two rank chunks
    # kernel ranks 33-64 above W 8: the forward as passes of 8 taps (the first W - 8(n-1), each later
    # one added to the stored y), the backward as passes of 32 ranks x passes of up to 4 taps into
    # the fp32 dx accumulator (the forward's z_eff rows of 64 ranks even where its first pass holds 1 tap)
    (1, 40, 64, 40, 9, False, True, torch.bfloat16, ("mfma", "mfma")),         # forward 1 + 8, 2 x 3 passes
    (1, 100, 128, 40, 12, False, True, torch.bfloat16, ("mfma", "mfma")),      # forward 4 + 8, 2 x 3 passes
    (2, 70, 256, 63, 9, True, True, torch.float16, ("mfma", "mfma")),          # four chunks: 9 passes of 1
    (1, 300, 64, 47, 20, True, False, torch.bfloat16, ("mfma", "mfma")),       # forward 4 + 8 + 8
    (1, 25, 64, 40, 20, False, True, torch.bfloat16, ("mfma", "mfma")),        # W 20 > T
    (1, 50, 64, 64, 32, False, True, torch.bfloat16, ("mfma", "mfma")),        # W 32: forward 4 x 8, 32 passes
    # kernel ranks 65-256 (the reference takes any power-of-two rank, lowrank.py:331-333): the forward
    # as passes of 128 ranks up to W 4 (8-wavefront workgroups), of 64 above (z columns and U rows from
    # the pass's first rank, the static rank in the pass
    # that holds index R, each pass split into passes of at most 8 taps, every pass after the first added
    # to the stored y; at most 4 passes), the backward as passes of 32 ranks on the two-chunk kernels
    # (dz partial columns and dU partial rows of the whole problem, dx accumulated; past 4 rank x tap
    # passes in fp32)
    (2, 300, 256, 127, 4, True, True, torch.bfloat16, ("mfma", "mfma")),      # kernel rank 128: 1 + 4 passes
    (1, 100, 128, 64, 3, True, False, torch.float16, ("mfma", "mfma")),       # rank 65: static alone in bwd pass 3
    (1, 60, 128, 64, 6, True, True, torch.bfloat16, ("mfma", "mfma")),        # W 6, rank 65: fwd 64 + static alone
    (1, 80, 128, 255, 4, True, True, torch.bfloat16, ("mfma", "mfma")),       # rank 256, W 4: forward 128 + 128
    (1, 3216, 256, 96, 2, False, True, torch.bfloat16, ("mfma", "mfma")),     # rank 96: z itself, long runs
    (2, 64, 128, 255, 8, True, True, torch.float16, ("mfma", "mfma")),        # rank 256, W 8: 4 + 8 x 2 passes
    (1, 50, 64, 200, 1, False, True, torch.bfloat16, ("mfma", "mfma")),       # rank 200, W 1: fwd 128 + 72
    (1, 37, 64, 100, 16, True, True, torch.bfloat16, ("mfma", "mfma")),       # rank 101, W 16: 2 x 2, 4 x 4
    (1, 45, 64, 127, 12, True, True, torch.bfloat16, ("mfma", "mfma")),       # W 12: forward 2 x (4 + 8)
    (1, 520, 200, 70, 5, False, False, torch.float16, ("mfma", "mfma")),      # D % 16 != 0, rank 70, W 5
    # z rows of R % 4 != 0 ranks at two or five to eight rank chunks: 8-byte loads at the rows'
    # 2-byte alignment, the last chunk's boundary group loaded as the 4 ranks that end at R (m = R -
    # 4q - 16(RC-1) dynamic ranks in it, then the static rank, then zeros)
    (2, 70, 64, 17, 4, False, True, torch.bfloat16, ("mfma", "mfma")),        # m = 1
    (1, 90, 128, 18, 3, True, False, torch.bfloat16, ("mfma", "mfma")),       # m = 2, static after
    (1, 61, 64, 19, 2, True, True, torch.float16, ("mfma", "mfma")),          # m = 3, static after
    (1, 50, 128, 29, 4, False, True, torch.bfloat16, ("mfma", "mfma")),       # m = 1 in group 3
    (1, 45, 64, 93, 4, True, True, torch.bfloat16, ("mfma", "mfma")),         # six chunks, m = 1
    (1, 40, 64, 118, 3, False, False, torch.float16, ("mfma", "mfma")),       # eight chunks, m = 2
    # the forward past 4 passes takes the generic kernels (its y would be rounded more often)
    (1, 64, 256, 127, 20, True, True, torch.bfloat16, ("generic", "mfma")),   # 2 x 3 forward passes
    (1, 30, 32, 255, 3, True, False, torch.float32, ("generic", "generic")),  # fp32 kernel rank 256
    # W 33 .. DC_MAX_W (the reference takes any W, lowrank.py:220): the generic kernels, whose dx
    # stages z rows per chunk of 32 taps (and per 256 channels) above W 32
    (1, 70, 128, 16, 33, False, True, torch.bfloat16, ("generic", "generic")),    # W 33: chunks 32 + 1
    (2, 50, 64, 15, 48, True, True, torch.float16, ("generic", "generic")),       # W 48 > T
    (1, 100, 128, 3, 64, True, False, torch.float32, ("generic", "generic")),     # fp32, W 64
    (1, 300, 64, 8, 100, True, True, torch.bfloat16, ("generic", "generic")),     # W 100: 4 chunks
    (1, 40, 320, 4, 70, False, True, torch.bfloat16, ("generic", "generic")),     # D 320: two channel steps
]


@pytest.mark.parametrize("case", LR_EDGE, ids=[f"lr{i}" for i in range(len(LR_EDGE))])
def test_edge_shapes_lowrank(case):
    Bn, Tn, Dn, R, W, static, residual, dtype = case[:8]
    if len(case) > 8:  # the kernel family the dispatch must pick for this shape
        for bwd, want in enumerate(case[8]):
            assert _path("lr", Bn, Tn, Dn, R, W, dtype, static, bwd) == want, ("bwd" if bwd else "fwd", want)
    g = gen(Bn * 1000003 + Tn * 1009 + Dn * 7 + R + W)
    x = randn(g, Bn, Tn, Dn)
    dy = randn(g, Bn, Tn, Dn)
    z = randn(g, Bn, Tn, R)
    U = randn(g, R, W * Dn, scale=1 / math.sqrt((R + 1) * W))
    sw = uniform(g, W, Dn, lo=-1 / math.sqrt(W), hi=1 / math.sqrt(W)) if static else None
    src = [x, z, U, sw]
    rk = R + (1 if static else 0)
    if rk & (rk - 1) == 0:
        kernel = lr
    else:  # the reference API asserts a power-of-two rank; the C ABI accepts any rank
        kernel = lambda a, b, c, d, residual: lr_mod._LowrankDynamicConvolutionFn.apply(a, b, c, d, residual)  # noqa: E731
    src_q = [None if t is None else t.to(dtype).float() for t in src]
    y_q, g_q = run_fwd_bwd(lr_ref, src_q, dy.to(dtype).float(), residual)
    y_k, g_k = run_fwd_bwd(kernel, [_to(t, dtype) for t in src], _to(dy, dtype), residual)
    assert_ns(y_k, y_q, dtype, "y")
    for a, b, n in zip(g_k, g_q, ["dx", "dz", "dU", "dstatic_w"]):
        if b is not None:
            assert_ns(a, b, dtype, n, elementwise=n == "dx")
    check_reductions("lr", src_q, dy.to(dtype).float(), g_k, dtype)


@pytest.mark.parametrize("R,static,dtype,off", [(16, False, torch.bfloat16, 1), (12, True, torch.bfloat16, 1),
                                                (32, False, torch.float16, 1), (15, True, torch.bfloat16, 1),
                                                (32, False, torch.bfloat16, 4), (16, False, torch.bfloat16, 4)])
def test_lowrank_misaligned_z(R, static, dtype, off):
    """z `off` elements into a buffer: the backward pads z (with the static column) into its workspace
    when its rows cannot be read whole (8-byte rows; 16-byte for two rank chunks), whatever R is."""
    g = gen(31 * R + static + 7 * off)
    Bn, Tn, Dn, W = 2, 72, 128, 4
    x, dy, z = randn(g, Bn, Tn, Dn), randn(g, Bn, Tn, Dn), randn(g, Bn, Tn, R)
    U = randn(g, R, W * Dn, scale=1 / math.sqrt((R + 1) * W))
    sw = uniform(g, W, Dn, lo=-1 / math.sqrt(W), hi=1 / math.sqrt(W)) if static else None
    buf = torch.empty(Bn * Tn * R + off, dtype=dtype, device=DEV)
    z_off = buf[off:].view(Bn, Tn, R)
    z_off.copy_(z.to(dtype))
    assert z_off.data_ptr() % 16 != 0 and z_off.is_contiguous()
    kernel = lambda a, b, c, d, residual: lr_mod._LowrankDynamicConvolutionFn.apply(a, b, c, d, residual)  # noqa: E731
    src_q = [None if t is None else t.to(dtype).float() for t in (x, z, U, sw)]
    y_q, g_q = run_fwd_bwd(lr_ref, src_q, dy.to(dtype).float(), True)
    leaves = [_to(x, dtype), z_off.detach(), _to(U, dtype), _to(sw, dtype)]  # no clone: z keeps its offset
    leaves = [None if t is None else t.requires_grad_() for t in leaves]
    assert leaves[1].data_ptr() % 16 != 0
    y_k = kernel(*leaves, residual=True)
    y_k.backward(_to(dy, dtype))
    g_k = [None if t is None else t.grad for t in leaves]
    assert_ns(y_k, y_q, dtype, "y")
    for a, b, n in zip(g_k, g_q, ["dx", "dz", "dU", "dstatic_w"]):
        if b is not None:
            assert_ns(a, b, dtype, n, elementwise=n == "dx")
    check_reductions("lr", src_q, dy.to(dtype).float(), g_k, dtype)


# --------------------------------------------------------- BASELINE configs
@pytest.mark.parametrize("loss", ["sum", "randn"])
def test_config0(loss):
    """BASELINE.json configs[0] on the GPU: headwise fp32, B2 T1024 D512 H512 (head size 1) W4, no static_w,
    no residual, x ~ N(0, 1), weights ~ N(0, 1/W); loss y.sum() (dy = 1) as the CPU baseline runs it, and a
    random dy.  test.py's criterion (test.py:17, 59-69) and the north-star one (1e-5 elementwise)."""
    Bn, Tn, Dn, H, W = 2, 1024, 512, 512, 4
    assert _path("hw", Bn, Tn, Dn, H, W, torch.float32, False, 0) == "vector"
    assert _path("hw", Bn, Tn, Dn, H, W, torch.float32, False, 1) == "vector"
    g = gen(0)
    x = randn(g, Bn, Tn, Dn)
    w = randn(g, Bn, Tn, H, W, scale=1 / math.sqrt(W))
    dy = torch.ones(Bn, Tn, Dn) if loss == "sum" else randn(g, Bn, Tn, Dn)
    _check_case(hw, hw_ref, [x, w, None], dy, torch.float32, False, ["dx", "dweight", "dstatic_w"],
                {"dx", "dweight"}, "hw")


def _baseline_inputs(cfg, seed=0):
    g = gen(seed)
    if cfg in ("cfg2", "cfg3"):
        Bn, Tn, Dn, W = 4, 4096, 2048, 4
        H = 2048 if cfg == "cfg2" else 64
        x = randn(g, Bn, Tn, Dn)
        w = randn(g, Bn, Tn, H, W, scale=1 / math.sqrt(W))
        sw = uniform(g, W, Dn, lo=-1 / math.sqrt(W), hi=1 / math.sqrt(W))
        dy = randn(g, Bn, Tn, Dn)
        return "hw", [x, w, sw], dy, True
    if cfg == "cfg4":
        Bn, Tn, Dn, W, R = 4, 4096, 2048, 4, 16
        x = randn(g, Bn, Tn, Dn)
        z = randn(g, Bn, Tn, R)
        U = randn(g, R, W * Dn, scale=1 / math.sqrt(16 * W))
        dy = randn(g, Bn, Tn, Dn)
        return "lr", [x, z, U, None], dy, True
    Bn, Tn, Dn, W, R = 2, 8192, 4096, 4, 31
    x = randn(g, Bn, Tn, Dn)
    z = randn(g, Bn, Tn, R)
    U = randn(g, R, W * Dn, scale=1 / math.sqrt(32 * W))
    sw = uniform(g, W, Dn, lo=-1 / math.sqrt(W), hi=1 / math.sqrt(W))
    dy = randn(g, Bn, Tn, Dn)
    return "lr", [x, z, U, sw], dy, True


def _oracle_on_device(ref, q, dyq, residual):
    """The oracle's fp32 restatement of reference.py, run over whole tensors on the GPU with
    torch's fp32 GEMMs at full precision (z @ U; TF32 off), from the same dtype-rounded inputs.
    It is still the oracle's own code (oracle/reference_cpu.py), only on another device."""
    with fp32_matmul_exact():
        return run_fwd_bwd(ref, [None if t is None else t.to(DEV) for t in q], dyq.to(DEV), residual)


@pytest.mark.parametrize("cfg", ["cfg2", "cfg3", "cfg4", "cfg5"])
def test_baseline_configs(cfg):
    """BASELINE.json configs 2-5 at full size, every row: y, dx and the local gradient (headwise
    dweight) elementwise against the oracle over the whole tensors (|a-b| <= 2e-2 +
    2e-2|b|), dz norm-wise against it, and the long reductions (lowrank dz and dU, dstatic_w) entry
    by entry against float64 sums of the same rounded terms (a per-entry bound tighter than the
    elementwise bar; see SUM_TOL).  configs[4] (cfg5) is one of its three q / k / v calls."""
    dtype = torch.bfloat16
    kind, src, dy, residual = _baseline_inputs(cfg)
    dev_in = [_to(t, dtype) for t in src]
    dy_d = _to(dy, dtype)
    fn = hw if kind == "hw" else lr
    y_k, g_k = run_fwd_bwd(fn, dev_in, dy_d, residual)
    del dev_in
    q = [None if t is None else t.to(dtype).float() for t in src]  # rounded inputs, fp32, CPU
    dyq = dy.to(dtype).float()
    ref = hw_ref if kind == "hw" else lr_ref
    y_o, g_o = _oracle_on_device(ref, q, dyq, residual)
    assert_ns_full(y_k, y_o, dtype, f"{cfg} y")
    assert_ns_full(g_k[0], g_o[0], dtype, f"{cfg} dx")
    assert_ns_full(g_k[1], g_o[1], dtype, f"{cfg} {'dweight' if kind == 'hw' else 'dz'}", elementwise=kind == "hw")
    del y_o, g_o
    torch.cuda.empty_cache()
    # the long reductions over the whole tensors: per-entry bounds against float64 sums
    # (dz of every row, every dU / dstatic_w entry)
    check_reductions(kind, q, dyq, g_k, dtype)


# ---------------------------------------------------------- long sequence
# One sequence of x spans more than 512 MiB (131172 rows of 2048 bf16): the
# headwise and lowrank kernels give each run of tiles buffer resources that
# start at the run's own first rows, so they stay on the vector / matrix-core
# kernels.  Local outputs are checked on every row (the oracle over the whole
# sequence on the GPU), the reductions over the whole sequence entry by entry.
# lr16n (rank 16, no static_w: the forward without the z_eff writer) runs
# 2048 forward wavefronts with runs of 65 tiles.  lr16f and lr32f8 are the
# fp32 tier's matrix-core kernels (rows of 8 and 16 KiB); lr32f8's backward
# runs as two rank passes x two tap passes (x read from 4 rows before each
# run's first tile in the second tap pass).
LONG = {  # kind: dtype, T, D, W, R (lowrank), static_w
    "hw32": (torch.bfloat16, 131172, 2048, 4, None, True),
    "hw32w12": (torch.bfloat16, 131172, 2048, 12, None, True),  # the wide kernels: a resource per row
    "lr16": (torch.bfloat16, 131172, 2048, 4, 15, True),
    "lr16n": (torch.bfloat16, 131172, 2048, 4, 16, False),
    "lr16f": (torch.float32, 65600, 2048, 4, 15, True),
    "lr32f8": (torch.float32, 32800, 4096, 8, 31, True),
}


@pytest.mark.parametrize("kind", list(LONG))
def test_long_sequence(kind):
    dtype, Tn, Dn, W, R, static = LONG[kind]
    Bn = 1
    for bwd in (0, 1):
        if kind.startswith("hw"):
            want = "vector" if W <= 8 else "head_mfma"
            assert _path("hw", Bn, Tn, Dn, Dn // 32, W, dtype, True, bwd) == want
        else:
            want = "f32_mfma" if dtype == torch.float32 else "mfma"
            assert _path("lr", Bn, Tn, Dn, R, W, dtype, static, bwd) == want
    g = gen(11)
    x = randn(g, Bn, Tn, Dn)
    dy = randn(g, Bn, Tn, Dn)
    sw = uniform(g, W, Dn, lo=-1 / math.sqrt(W), hi=1 / math.sqrt(W))
    if kind.startswith("hw"):
        src, fn, ref = [x, randn(g, Bn, Tn, Dn // 32, W, scale=1 / math.sqrt(W)), sw], hw, hw_ref
    else:
        src, fn, ref = [x, randn(g, Bn, Tn, R), randn(g, R, W * Dn, scale=1 / math.sqrt((R + 1) * W)),
                        sw if static else None], lr, lr_ref
    y_k, g_k = run_fwd_bwd(fn, [_to(t, dtype) for t in src], _to(dy, dtype), True)
    q = [t.to(dtype).float() if t is not None else None for t in src]
    dyq = dy.to(dtype).float()
    # every row (the run boundaries of the full launch plan and the rows around 512 MiB included)
    y_o, g_o = _oracle_on_device(ref, q, dyq, True)
    assert_ns_full(y_k, y_o, dtype, f"{kind} y")
    assert_ns_full(g_k[0], g_o[0], dtype, f"{kind} dx")
    assert_ns_full(g_k[1], g_o[1], dtype, f"{kind} d1", elementwise=kind.startswith("hw"))
    del y_o, g_o
    torch.cuda.empty_cache()
    # the global reductions over the whole sequence (headwise dstatic_w; lowrank dz, dU,
    # dstatic_w): per-entry bounds against float64 sums
    check_reductions("hw" if kind.startswith("hw") else "lr", q, dyq, g_k, dtype)


HUGE = {  # kind: T, D, heads (headwise) or rank (lowrank), W, static_w
    "hw32": ((1 << 20) + 100, 2048, 64, 4, True),
    "hw1": ((1 << 20) + 100, 2048, 2048, 4, True),   # weight and dweight of 2^33 + elements
    "lr16": ((1 << 20) + 100, 2048, 16, 4, False),
    "lr31s": ((1 << 19) + 50, 4096, 31, 4, True),    # the z_eff writer, two rank chunks
}


@pytest.mark.parametrize("kind", list(HUGE))
def test_past_2_31_elements(kind):
    """x (and y, dy, dx) past 2^31 elements, headwise weights past 2^33 (about 60 GB of device
    memory at hs1): the vector and matrix-core kernels address every row through per-run buffer
    resources whose bases are 64-bit.  Rows at both ends and around element 2^31 against the CPU
    oracle on windows of the same inputs (with the W-1 rows of halo on each side)."""
    dtype = torch.bfloat16
    Tn, Dn, HR, W, static = HUGE[kind]
    assert Tn * Dn > 1 << 31
    g = torch.Generator(device=DEV).manual_seed(7)
    x = torch.randn(1, Tn, Dn, device=DEV, generator=g, dtype=dtype)
    dy = torch.randn(1, Tn, Dn, device=DEV, generator=g, dtype=dtype)
    sw = ((torch.rand(W, Dn, device=DEV, generator=g) * 2 - 1) / math.sqrt(W)).to(dtype) if static else None
    if kind.startswith("hw"):
        mid = [(torch.randn(1, Tn, HR, W, device=DEV, generator=g) / math.sqrt(W)).to(dtype)]
        fn, ref, per_row = hw, hw_ref, [True]
        assert _path("hw", 1, Tn, Dn, HR, W, dtype, static, 1) == "vector"
    else:
        mid = [torch.randn(1, Tn, HR, device=DEV, generator=g, dtype=dtype),
               (torch.randn(HR, W * Dn, device=DEV, generator=g) / math.sqrt((HR + 1) * W)).to(dtype)]
        fn, ref, per_row = lr, lr_ref, [True, False]
        assert _path("lr", 1, Tn, Dn, HR, W, dtype, static, 1) == "mfma"
    src = [x] + mid + [sw]
    leaves = [None if t is None else t.detach().requires_grad_() for t in src]
    y = fn(*leaves, residual=True)
    y.backward(dy)
    torch.cuda.synchronize()
    rows = [True] + per_row + [False]  # inputs cut to the window (z with x; U and static_w whole)
    edge = (1 << 31) // Dn
    for w0, w1 in [(0, 64), (edge - 40, edge + 40), (Tn - 64, Tn)]:
        a, e = max(0, w0 - W + 1), min(Tn, w1 + W - 1)
        win = [None if t is None else (t[:, a:e] if r else t).float().cpu() for t, r in zip(src, rows)]
        y_w, g_w = run_fwd_bwd(ref, win, dy[:, a:e].float().cpu(), True)
        sl = slice(w0 - a, w1 - a)
        assert_ns(y[:, w0:w1], y_w[:, sl], dtype, f"{kind} y[{w0}:{w1}]")
        assert_ns(leaves[0].grad[:, w0:w1], g_w[0][:, sl], dtype, f"{kind} dx[{w0}:{w1}]")
        assert_ns(leaves[1].grad[:, w0:w1], g_w[1][:, sl], dtype, f"{kind} d1[{w0}:{w1}]",
                  elementwise=kind.startswith("hw"))
    del x, dy, sw, mid, src, leaves, y
    torch.cuda.empty_cache()


def test_generic_lowrank_rows_past_2_24():
    """The generic lowrank kernels (D = 4 is off the matrix-core paths, which take whole
    8-channel pieces) over more than 2^24 rows: the per-row dz launch loops over rows with a capped
    grid (one workgroup per row would ask for more than 2^32 work-items).  Row windows at both
    ends against the oracle; dz, dU and dstatic_w entry by entry against float64 sums over the
    whole sequence."""
    dtype = torch.bfloat16
    Bn, Tn, Dn, R, W = 1, (1 << 24) + 40, 4, 3, 4  # R + static = 4 (the API's power of two)
    assert _path("lr", Bn, Tn, Dn, R, W, dtype, True, 0) == "generic"
    assert _path("lr", Bn, Tn, Dn, R, W, dtype, True, 1) == "generic"
    g = gen(13)
    x = randn(g, Bn, Tn, Dn)
    dy = randn(g, Bn, Tn, Dn)
    sw = uniform(g, W, Dn, lo=-1 / math.sqrt(W), hi=1 / math.sqrt(W))
    src = [x, randn(g, Bn, Tn, R), randn(g, R, W * Dn, scale=1 / math.sqrt(R * W)), sw]
    y_k, g_k = run_fwd_bwd(lr, [_to(t, dtype) for t in src], _to(dy, dtype), True)
    y_k, g_k = y_k.cpu(), [t.cpu() for t in g_k]
    q = [t.to(dtype).float() for t in src]
    dyq = dy.to(dtype).float()
    for t0, t1 in [(0, 64), (Tn - 64, Tn)]:
        a, e = max(0, t0 - W + 1), min(Tn, t1 + W - 1)
        win = [q[0][:, a:e], q[1][:, a:e], q[2], q[3]]
        y_w, g_w = run_fwd_bwd(lr_ref, win, dyq[:, a:e], True)
        sl = slice(t0 - a, t1 - a)
        assert_ns(y_k[:, t0:t1], y_w[:, sl], dtype, f"y[{t0}:{t1}]")
        assert_ns(g_k[0][:, t0:t1], g_w[0][:, sl], dtype, f"dx[{t0}:{t1}]")
    check_reductions("lr", q, dyq, g_k, dtype)


# ------------------------------------------------------------ inference
@pytest.mark.parametrize("R,static,W,dtype", [(15, True, 4, torch.bfloat16), (31, True, 4, torch.float16),
                                              (16, False, 4, torch.bfloat16), (15, True, 12, torch.bfloat16)])
def test_lowrank_inference_forward(R, static, W, dtype):
    """Without gradients the forward skips the padded z copy for the backward (other kernel
    instantiations): y is bitwise the training forward's, single and grouped."""
    g = gen(23 + R + W)
    Bn, Tn, Dn = 2, 300, 256
    x = randn(g, Bn, Tn, Dn).to(dtype).to(DEV)
    z = randn(g, Bn, Tn, R).to(dtype).to(DEV)
    U = randn(g, R, W * Dn, scale=1 / math.sqrt((R + 1) * W)).to(dtype).to(DEV)
    sw = uniform(g, W, Dn, lo=-0.5, hi=0.5).to(dtype).to(DEV) if static else None
    with torch.no_grad():
        y_inf = lr(x, z, U, sw, residual=True)
    y_trn = lr(x.clone().requires_grad_(), z, U, sw, residual=True).detach()
    assert torch.equal(y_inf, y_trn)
    xs = randn(g, Bn, Tn, 3 * Dn).to(dtype).to(DEV)
    zs = [z, z.flip(1).contiguous(), (z * 0.5).contiguous()]
    with torch.no_grad():
        ys_inf = lr_mod.lowrank_dynamic_convolution_grouped(xs, zs, [U] * 3, [sw] * 3 if static else None,
                                                            residual=True)
    ys_trn = lr_mod.lowrank_dynamic_convolution_grouped(xs.clone().requires_grad_(), zs, [U] * 3,
                                                        [sw] * 3 if static else None, residual=True)
    for a, b in zip(ys_inf, ys_trn):
        assert torch.equal(a, b.detach())


@pytest.mark.parametrize("R,static,W,dtype,passes", [(63, True, 32, torch.bfloat16, 4), (63, True, 32, torch.float16, 4),
                                                     (64, False, 32, torch.bfloat16, 4), (31, True, 32, torch.bfloat16, 2),
                                                     (127, True, 16, torch.bfloat16, 4), (127, True, 16, torch.float16, 4)])
def test_lowrank_forward_pass_rounding(R, static, W, dtype, passes):
    """The 16-bit forward above W 16 (kernel rank <= 32), above W 8 (ranks 33-64) and above kernel
    rank 64 runs as `passes` launches, each adding to the y the previous one stored in x's type, so
    y is rounded `passes` times where the reference rounds once.  Bound on |y - y64| against the
    oracle's float64 result from the same inputs: u|y64| (the last rounding) + (passes - 1) u S
    (each earlier rounding of a partial sum, |partial| <= S = |x| + sum_k |K[k]| |x[t-k]|) +
    (W (R + 1) + 2) 2^-23 S' (fp32 sums, S' as S with |z| |U| for K); u = 2^-8 (bf16), 2^-11 (fp16)."""
    from oracle.reference_cpu import lowrank_weights_ref

    g = gen(97 + R + W)
    Bn, Tn, Dn = 2, 256, 256
    x = randn(g, Bn, Tn, Dn).to(dtype).to(DEV)
    z = randn(g, Bn, Tn, R).to(dtype).to(DEV)
    U = randn(g, R, W * Dn, scale=1 / math.sqrt((R + 1) * W)).to(dtype).to(DEV)
    sw = uniform(g, W, Dn, lo=-1 / math.sqrt(W), hi=1 / math.sqrt(W)).to(dtype).to(DEV) if static else None
    assert _path("lr", Bn, Tn, Dn, R, W, dtype, static, False) == "mfma"  # the matrix-core passes
    with torch.no_grad():
        y = lr_mod._LowrankDynamicConvolutionFn.apply(x, z, U, sw, True).double()
    d = [None if t is None else t.double() for t in (x, z, U, sw)]
    y64 = lr_ref(*d, residual=True)
    K = lowrank_weights_ref(d[1], d[2], Dn) + (0 if sw is None else d[3])
    Ka = lowrank_weights_ref(d[1].abs(), d[2].abs(), Dn) + (0 if sw is None else d[3].abs())
    xa = d[0].abs()
    S, S2 = xa.clone(), xa.clone()
    for k in range(W):
        xk = torch.zeros_like(xa)
        xk[:, k:] = xa[:, :Tn - k]
        S += K[:, :, k].abs() * xk
        S2 += Ka[:, :, k] * xk
    u = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    bound = u * y64.abs() + (passes - 1) * u * S + (W * (R + 1) + 2) * 2.0 ** -23 * S2
    err = (y - y64).abs()
    worst = (err / bound).max().item()
    single = u * y64.abs() + (W * (R + 1) + 2) * 2.0 ** -23 * S2  # what one rounding allows
    over = (err > single).double().mean().item()
    print(f"R{R}{'+s' if static else ''} W{W} {dtype}: max err/bound {worst:.3f}, max err/(u S) "
          f"{(err / (u * S)).max().item():.3f}, share past the one-rounding bound {over:.2e}")
    assert worst <= 1.0


@pytest.mark.parametrize("R,static,W,dtype,passes", [(40, True, 5, torch.bfloat16, 3), (40, True, 7, torch.bfloat16, 4),
                                                     (64, True, 1, torch.bfloat16, 3), (16, False, 16, torch.bfloat16, 2),
                                                     (31, True, 8, torch.float16, 2), (40, True, 7, torch.float16, 4)])
def test_lowrank_backward_pass_rounding(R, static, W, dtype, passes):
    """The 16-bit backward of 2-4 passes (taps, or ranks above kernel rank 64) adds each pass's dx
    to what the previous one stored in x's type (more passes go through an fp32 accumulator), so dx
    is rounded `passes` times where the reference rounds once.  Bound on |dx - dx64| against the
    oracle's float64 gradient from the same inputs: u|dx64| + (passes - 1) u S + (W (R + 1) + 2)
    2^-23 S, with S = |dy| + sum_k |dy[t+k]| (|z| |U| + |static_w|)[t+k, k] (every partial sum of
    ranks and taps is at most S); u = 2^-8 (bf16), 2^-11 (fp16).  A random sweep of large shapes
    met single entries (of 10^6-10^7) just past the elementwise 2e-2 bar this way, where the exact
    dx is near zero and the partials are several units: within this bound and the reference's own
    bf16 tolerance (test.py:17)."""
    from oracle.reference_cpu import lowrank_weights_ref

    g = gen(193 + R + W)
    Bn, Tn, Dn = 2, 256, 256
    x = randn(g, Bn, Tn, Dn).to(dtype).to(DEV)
    z = randn(g, Bn, Tn, R).to(dtype).to(DEV)
    U = randn(g, R, W * Dn, scale=1 / math.sqrt((R + 1) * W)).to(dtype).to(DEV)
    sw = uniform(g, W, Dn, lo=-1 / math.sqrt(W), hi=1 / math.sqrt(W)).to(dtype).to(DEV) if static else None
    dy = randn(g, Bn, Tn, Dn).to(dtype).to(DEV)
    for bwd in (0, 1):
        assert _path("lr", Bn, Tn, Dn, R, W, dtype, static, bwd) == "mfma"
    xk = x.clone().requires_grad_()
    lr_mod._LowrankDynamicConvolutionFn.apply(xk, z, U, sw, True).backward(dy)
    dx = xk.grad.double()
    d = [None if t is None else t.double() for t in (x, z, U, sw)]
    xr = d[0].clone().requires_grad_()
    lr_ref(xr, *d[1:], residual=True).backward(dy.double())
    dx64 = xr.grad
    Ka = lowrank_weights_ref(d[1].abs(), d[2].abs(), Dn) + (0 if sw is None else d[3].abs())
    dya = dy.double().abs()
    S = dya.clone()  # the residual's term
    for k in range(W):
        t = torch.zeros_like(dya)
        t[:, :Tn - k] = dya[:, k:] * Ka[:, k:, k]
        S += t
    u = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    bound = u * dx64.abs() + (passes - 1) * u * S + (W * (R + 1) + 2) * 2.0 ** -23 * S
    err = (dx - dx64).abs()
    worst = (err / bound).max().item()
    print(f"R{R}{'+s' if static else ''} W{W} {dtype} ({passes} passes): max err/bound {worst:.3f}, "
          f"max err/(u S) {(err / (u * S)).max().item():.3f}")
    assert worst <= 1.0


# ------------------------------------------------------------ determinism
DET_CASES = [  # op, head size (headwise) or kernel rank with the static filter (lowrank), W
    ("hw", 1, 4), ("hw", 32, 4), ("lr", 16, 4),
    ("hw", 32, 12), ("hw", 4, 24),  # the head matrix-core kernels (hs 32), the wide kernels (hs 4)
    ("hw", 16, 30),
    ("lr", 16, 20),                 # passes of 8 taps (one rank chunk)
    ("lr", 32, 20),                 # passes of 4 taps (two rank chunks) into the fp32 dx accumulator
    ("lr", 128, 4), ("lr", 128, 8),  # passes of ranks (at W 8 into the fp32 dx accumulator)
]


@pytest.mark.parametrize("op,n,W", DET_CASES, ids=[f"{o}{n}w{w}" for o, n, w in DET_CASES])
def test_deterministic(op, n, W):
    """Two runs give bitwise equal outputs and gradients: no float atomics anywhere, partial sums in a
    fixed order (W 12 / 24: the wide headwise kernels; lowrank W 20: passes of taps, at kernel rank 32
    into the fp32 dx accumulator; kernel rank 128: passes of ranks, at W 8 into the fp32 dx
    accumulator)."""
    g = gen(5)
    Bn, Tn, Dn = 2, 1024, 512
    x = randn(g, Bn, Tn, Dn).to(torch.bfloat16).to(DEV)
    dy = randn(g, Bn, Tn, Dn).to(torch.bfloat16).to(DEV)
    sw = randn(g, W, Dn, scale=0.3).to(torch.bfloat16).to(DEV)
    if op == "hw":
        w = randn(g, Bn, Tn, Dn // n, W, scale=0.5).to(torch.bfloat16).to(DEV)
        src, fn = [x, w, sw], hw
        want = "vector" if W <= 8 else "head_mfma" if _hw_mma_shape(Dn, Dn // n, W, torch.bfloat16) else "wide"
        assert _path("hw", Bn, Tn, Dn, Dn // n, W, torch.bfloat16, True, 1) == want
    else:
        R = n - 1  # dynamic ranks; the static filter is the last kernel rank
        z = randn(g, Bn, Tn, R).to(torch.bfloat16).to(DEV)
        U = randn(g, R, W * Dn, scale=0.1).to(torch.bfloat16).to(DEV)
        src, fn = [x, z, U, sw], lr
        assert _path("lr", Bn, Tn, Dn, R, W, torch.bfloat16, True, 1) == "mfma"
    outs = [run_fwd_bwd(fn, src, dy, True) for _ in range(2)]
    assert torch.equal(outs[0][0], outs[1][0])
    for a, b in zip(outs[0][1], outs[1][1]):
        assert torch.equal(a, b)


def test_generic_matches_vector_path():
    """A 2-byte-offset view forces the element-aligned kernels; both paths agree with the oracle."""
    g = gen(9)
    Bn, Tn, Dn, H, W = 2, 96, 256, 64, 4
    dtype = torch.bfloat16
    x = randn(g, Bn, Tn, Dn)
    w = randn(g, Bn, Tn, H, W, scale=0.5)
    sw = randn(g, W, Dn, scale=0.3)
    dy = randn(g, Bn, Tn, Dn)
    buf = torch.empty(Bn * Tn * Dn + 1, dtype=dtype, device=DEV)
    x_off = buf[1:].view(Bn, Tn, Dn)  # 2-byte offset: not 16-byte aligned
    x_off.copy_(x.to(dtype))
    assert x_off.data_ptr() % 16 != 0 and x_off.is_contiguous()
    y_v, g_v = run_fwd_bwd(hw, [_to(x, dtype), _to(w, dtype), _to(sw, dtype)], _to(dy, dtype), True)
    x_off.requires_grad_()
    leaves = [_to(w, dtype).requires_grad_(), _to(sw, dtype).requires_grad_()]
    y_g = hw(x_off, *leaves, residual=True)
    y_g.backward(_to(dy, dtype))
    g_g = [x_off.grad] + [t.grad for t in leaves]
    assert max_rel(y_v, y_g) < 1e-2
    for a, b in zip(g_v, g_g):
        assert max_rel(a, b) < 1e-2


# ------------------------------------------------- padded z copy from the forward
@pytest.mark.parametrize("R,static,xoff,zoff", [(15, True, 0, 0), (31, True, 0, 0), (3, False, 0, 0), (28, False, 0, 0),
                                                (15, True, 4, 0), (63, True, 0, 0), (37, False, 4, 0), (15, True, 0, 1),
                                                (31, True, 4, 1), (50, True, 0, 0), (52, False, 0, 1)])
def test_lowrank_zeff_saved(R, static, xoff, zoff):
    """The forward's padded z copy (z, the static column as 1, zero ranks up to RP) feeds the
    backward exactly as the copy the backward builds itself: bitwise equal gradients.  xoff = 4
    puts x 8 bytes off 16-byte alignment: the forward takes its element-aligned kernels and
    fills the copy in a launch of its own (the padding kernel), the backward stays on matrix
    cores.  zoff = 1 starts z 2 bytes into its buffer (rows not 4-byte aligned); at W 4 every
    kernel rank above 32 pads to a multiple of 32 (the backward's passes of 32 ranks read 16
    bytes of a row per lane, so even R % 4 == 0 takes the copy): R 63, 37, 50 + static, 52."""
    from dynconv import _capi

    lib = _capi.load()
    Bn, Tn, Dn, W = 2, 300, 256, 4
    g = gen(17 + R)
    bf = torch.bfloat16
    xb = randn(g, Bn * Tn * Dn + xoff).to(bf).to(DEV)
    x = xb[xoff:].view(Bn, Tn, Dn)
    zb = randn(g, Bn * Tn * R + zoff).to(bf).to(DEV)
    z = zb[zoff:].view(Bn, Tn, R)
    U = randn(g, R, W * Dn, scale=1 / math.sqrt((R + 1) * W)).to(bf).to(DEV)
    sw = uniform(g, W, Dn, lo=-0.5, hi=0.5).to(bf).to(DEV) if static else None
    dy = randn(g, Bn, Tn, Dn).to(bf).to(DEV)
    rk = R + (1 if static else 0)
    rp = 32 if 16 < rk <= 32 else ((rk + 31) // 32 * 32 if rk > 32 else (rk + 3) // 4 * 4)  # W 4
    nz = lib.dc_lowrank_zeff_bytes(Bn, Tn, Dn, R, W, 0, int(static))
    assert nz == Bn * Tn * rp * 2
    zeff = torch.full((nz,), 0xAB, dtype=torch.uint8, device=DEV)  # the forward overwrites all of it
    y = torch.empty_like(x)
    p = _capi.ptr
    st = torch.cuda.current_stream().cuda_stream
    _capi.check(lib.dc_lowrank_fwd(p(x), p(z), p(U), p(sw), p(y), p(zeff), nz, Bn, Tn, Dn, R, W, 0, 1, st), "fwd")
    want = torch.zeros(Bn * Tn, rp, dtype=bf, device=DEV)
    want[:, :R] = z.reshape(-1, R)
    if static:
        want[:, R] = 1.0
    torch.cuda.synchronize()
    assert torch.equal(zeff.view(bf).view(Bn * Tn, rp), want)
    nws = lib.dc_lowrank_bwd_ws_bytes(Bn, Tn, Dn, R, W, 0, int(static))
    outs = []
    for zp in (None, zeff):
        ws = torch.empty(nws, dtype=torch.uint8, device=DEV)
        dx, dz, dU = torch.empty_like(x), torch.empty_like(z), torch.empty_like(U)
        dsw = torch.empty_like(sw) if static else None
        _capi.check(lib.dc_lowrank_bwd(p(x), p(z), p(U), p(sw), p(zp), nz if zp is not None else 0, p(dy), p(dx),
                                       p(dz), p(dU), p(dsw), p(ws), nws, Bn, Tn, Dn, R, W, 0, 1, st), "bwd")
        outs.append([dx, dz, dU] + ([dsw] if static else []))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
