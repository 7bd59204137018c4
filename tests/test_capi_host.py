"""C-ABI tests that run without a GPU.

The library must load, export every function include/dynconv.h declares, and
reject every invalid argument with its documented status before touching
the HIP runtime.  Valid arguments on a machine without a device must give
DC_ERR_DEVICE (a status, not a crash).  No compute call is made here: the
pointers passed are never dereferenced on any of these paths.
"""

import ctypes
import os
import re

import pytest
import torch

from helpers import ROOT  # noqa: F401  (sets sys.path)
from dynconv import _capi

HEADER = os.path.join(ROOT, "include", "dynconv.h")

OK, E_NULL, E_SHAPE, E_DTYPE, E_UNSUP, E_WS, E_ALIGN, E_DEV, E_LAUNCH, E_SCRATCH = 0, -1, -2, -3, -4, -5, -6, -7, -8, -9
P = 0x10000  # a fake, 256-byte aligned "device pointer"; never dereferenced on these paths


@pytest.fixture(scope="module")
def lib():
    return _capi.load()


def header_functions():
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\*\s]+?\b(dc_\w+)\s*\(", txt, re.M)))


def test_exports_every_declared_symbol(lib):
    names = header_functions()
    assert len(names) == 19, names
    raw = ctypes.CDLL(_capi.LIB_PATH)
    for n in names:
        assert hasattr(raw, n), f"{n} declared in dynconv.h but not exported"
    assert set(names) == set(_capi.SIGNATURES), "ctypes signatures out of sync with the header"


def test_abi_version_and_strings(lib):
    assert lib.dc_abi_version() == 7
    for s in (OK, E_NULL, E_SHAPE, E_DTYPE, E_UNSUP, E_WS, E_ALIGN, E_DEV, E_LAUNCH, E_SCRATCH):
        assert len(lib.dc_status_string(s)) > 0
    assert b"unknown" in lib.dc_status_string(-99)


def hw_fwd(lib, x=P, w=P, sw=None, y=P, B=2, T=8, D=16, H=4, W=4, dt=0, res=0):
    return lib.dc_headwise_fwd(x, w, sw, y, B, T, D, H, W, dt, res, None)


def test_headwise_fwd_validation(lib):
    no_dev = not torch.cuda.is_available()
    assert hw_fwd(lib, dt=7) == E_DTYPE
    assert hw_fwd(lib, B=0) == E_SHAPE
    assert hw_fwd(lib, T=-1) == E_SHAPE
    assert hw_fwd(lib, H=3) == E_SHAPE           # 16 % 3 != 0
    assert hw_fwd(lib, H=0) == E_SHAPE
    assert hw_fwd(lib, W=1025) == E_UNSUP        # > DC_MAX_W
    assert hw_fwd(lib, W=1024, D=1 << 21, H=1 << 21) == E_SHAPE  # W * D columns past int32
    assert hw_fwd(lib, T=1 << 31) == E_SHAPE     # int32 row indexing bound
    assert hw_fwd(lib, x=None) == E_NULL
    assert hw_fwd(lib, y=None) == E_NULL
    assert hw_fwd(lib, x=P + 1) == E_ALIGN       # bf16 needs 2-byte alignment
    assert hw_fwd(lib, x=P + 2, dt=2) == E_ALIGN  # fp32 needs 4
    if no_dev:
        assert hw_fwd(lib) == E_DEV
        assert hw_fwd(lib, sw=P, res=1, W=1) == E_DEV
        assert hw_fwd(lib, W=32) == E_DEV         # widths above 8 take the generic kernels


def hw_bwd(lib, sw=None, dsw=None, ws=None, nws=0, B=2, T=8, D=16, H=4, W=4, dt=0, dy=P):
    return lib.dc_headwise_bwd(P, P, sw, dy, P, P, dsw, ws, nws, B, T, D, H, W, dt, 0, None)


def test_headwise_bwd_validation(lib):
    no_dev = not torch.cuda.is_available()
    assert lib.dc_headwise_bwd_ws_bytes(2, 8, 16, 4, 4, 0, 0) == 0
    need = lib.dc_headwise_bwd_ws_bytes(2, 8, 16, 4, 4, 0, 1)
    assert need > 0 and need % 4 == 0
    assert lib.dc_headwise_bwd_ws_bytes(2, 8, 16, 3, 4, 0, 1) == E_SHAPE
    assert lib.dc_headwise_bwd_ws_bytes(2, 8, 16, 4, 4, 5, 1) == E_DTYPE
    assert hw_bwd(lib, dy=None) == E_NULL
    assert hw_bwd(lib, sw=P, dsw=None) == E_NULL   # static_w / dstatic_w must agree
    assert hw_bwd(lib, sw=None, dsw=P) == E_NULL
    assert hw_bwd(lib, sw=P, dsw=P, ws=None, nws=need) == E_WS
    assert hw_bwd(lib, sw=P, dsw=P, ws=P, nws=need - 4) == E_WS
    assert hw_bwd(lib, sw=P, dsw=P, ws=P + 4, nws=need) == E_WS   # workspace below 16-byte alignment
    if no_dev:
        assert hw_bwd(lib) == E_DEV
        assert hw_bwd(lib, sw=P, dsw=P, ws=P, nws=need) == E_DEV


def lr_fwd(lib, x=P, z=P, U=P, sw=None, zeff=None, nzeff=1 << 20, B=2, T=8, D=16, R=4, W=4, dt=0):
    return lib.dc_lowrank_fwd(x, z, U, sw, P, zeff, nzeff, B, T, D, R, W, dt, 0, None)


def test_lowrank_validation(lib):
    no_dev = not torch.cuda.is_available()
    assert lr_fwd(lib, dt=-1) == E_DTYPE
    assert lr_fwd(lib, R=0) == E_SHAPE
    assert lr_fwd(lib, R=256, sw=P) == E_UNSUP   # kernel rank 257 > DC_MAX_R
    assert lr_fwd(lib, R=257) == E_UNSUP
    assert lr_fwd(lib, W=1025) == E_UNSUP
    assert lr_fwd(lib, W=0) == E_SHAPE
    assert lr_fwd(lib, z=None) == E_NULL
    assert lr_fwd(lib, U=P + 1) == E_ALIGN
    assert lr_fwd(lib, zeff=P + 8) == E_ALIGN      # the padded z copy: 16-byte aligned
    # a padded z copy shorter than its size query (R 3 + static: 2*8 rows of 4 ranks)
    assert lr_fwd(lib, R=3, sw=P, zeff=P, nzeff=2 * 8 * 4 * 2 - 2) == E_WS
    # the padded z copy the backward would build: none when z's own rows serve (R % 4 == 0,
    # or 32 dynamic ranks for two rank chunks), else B*T rows of 4*k (one chunk) or 32 ranks
    zb = lib.dc_lowrank_zeff_bytes
    assert zb(2, 8, 16, 4, 4, 0, 1) == 0
    assert zb(2, 8, 16, 3, 4, 0, 1) == 2 * 8 * 4 * 2
    assert zb(2, 8, 16, 15, 4, 1, 1) == 2 * 8 * 16 * 2
    assert zb(2, 8, 16, 31, 4, 0, 1) == 2 * 8 * 32 * 2
    assert zb(2, 8, 16, 32, 4, 0, 0) == 0
    assert zb(2, 8, 16, 28, 4, 0, 0) == 2 * 8 * 32 * 2
    # kernel ranks 49-64 from W 2 on and 33-48 from W 3 on: passes of 32 ranks, rows of 64 unless z
    # holds a multiple of 32 dynamic ranks; below those widths one pass of three or four rank chunks
    # (8-byte loads: R % 4 == 0 reads z itself, else rows of RK rounded up to 4)
    assert zb(2, 8, 16, 63, 4, 0, 1) == 2 * 8 * 64 * 2
    assert zb(2, 8, 16, 60, 2, 0, 0) == 2 * 8 * 64 * 2
    assert zb(2, 8, 16, 64, 4, 0, 0) == 0
    assert zb(2, 8, 16, 60, 1, 0, 0) == 0
    assert zb(2, 8, 16, 63, 1, 0, 1) == 2 * 8 * 64 * 2
    assert zb(2, 8, 16, 47, 4, 0, 1) == 2 * 8 * 64 * 2
    assert zb(2, 8, 16, 40, 3, 0, 0) == 2 * 8 * 64 * 2
    assert zb(2, 8, 16, 47, 2, 0, 1) == 2 * 8 * 48 * 2  # W 2: one pass of three rank chunks
    assert zb(2, 8, 16, 40, 2, 0, 0) == 0
    assert zb(2, 8, 16, 37, 9, 0, 0) == 2 * 8 * 64 * 2  # W 9: the forward's first pass of taps holds 1
    assert zb(2, 8, 16, 3, 4, 2, 1) == 0              # fp32: the backward reads z itself
    assert zb(2, 8, 20, 3, 4, 0, 1) == 0              # D % 8 != 0: no matrix-core backward
    assert zb(2, 8, 24, 3, 4, 0, 1) == 2 * 8 * 4 * 2  # D % 8 == 0 suffices
    assert zb(2, 8, 16, 0, 4, 0, 1) == E_SHAPE
    need = lib.dc_lowrank_bwd_ws_bytes(2, 8, 16, 4, 4, 0, 1)
    assert need > 0
    assert lib.dc_lowrank_bwd_ws_bytes(2, 8, 16, 4, 1025, 0, 1) == E_UNSUP
    assert lib.dc_lowrank_bwd_ws_bytes(2, 8, 16, 127, 12, 0, 1) > 0   # generic kernels: W 12, kernel rank 128

    def bwd(zeff=None, nzeff=0, ws=P, nws=need, sw=P, R=4):
        return lib.dc_lowrank_bwd(P, P, P, sw, zeff, nzeff, P, P, P, P, sw, ws, nws, 2, 8, 16, R, 4, 0, 0, None)

    assert bwd(ws=None, nws=0) == E_WS
    assert bwd(ws=P + 8) == E_WS  # workspace below 16-byte alignment
    assert lib.dc_lowrank_bwd(P, P, P, None, None, 0, P, P, P, P, P, P, need, 2, 8, 16, 4, 4, 0, 0, None) == E_NULL
    assert bwd(zeff=P + 8, nzeff=1 << 20) == E_ALIGN  # the padded z copy below 16-byte alignment
    need3 = lib.dc_lowrank_bwd_ws_bytes(2, 8, 16, 3, 4, 0, 1)
    nz3 = zb(2, 8, 16, 3, 4, 0, 1)
    assert bwd(zeff=P, nzeff=nz3 - 1, R=3, nws=need3) == E_WS  # padded z copy below its size query
    if no_dev:
        assert lr_fwd(lib) == E_DEV
        assert lr_fwd(lib, R=3, sw=P, zeff=P) == E_DEV
        assert lr_fwd(lib, R=3, sw=P, zeff=P, nzeff=nz3) == E_DEV
        assert lr_fwd(lib, R=4, zeff=P, nzeff=0) == E_DEV   # no copy for this shape: the buffer is not used
        assert lr_fwd(lib, R=127, sw=P, W=12) == E_DEV      # generic kernels
        assert bwd() == E_DEV
        assert bwd(zeff=P, nzeff=nz3, R=3, nws=need3) == E_DEV


def arr(*ptrs):
    """A host array of fake device pointers (a `const void* const*` argument)."""
    return (ctypes.c_void_p * len(ptrs))(*ptrs)


def lr_fwd_g(lib, G=3, x=P, x_ld=48, z="ok", U="ok", sw=None, y="ok", zeff=None, nzeff=1 << 20, y_hd=0, B=2, T=8,
             D=16, R=4, W=4, dt=0):
    z = arr(*[P] * G) if z == "ok" else z
    U = arr(*[P] * G) if U == "ok" else U
    y = arr(*[P] * G) if y == "ok" else y
    return lib.dc_lowrank_fwd_grouped(G, x, x_ld, z, U, sw, y, zeff, nzeff, y_hd, B, T, D, R, W, dt, 0, None)


def test_lowrank_grouped_fwd_validation(lib):
    no_dev = not torch.cuda.is_available()
    assert lr_fwd_g(lib, G=0) == E_UNSUP
    assert lr_fwd_g(lib, G=5, x_ld=80) == E_UNSUP          # > DC_MAX_GROUPS
    assert lr_fwd_g(lib, x_ld=47) == E_SHAPE               # rows narrower than G*D
    assert lr_fwd_g(lib, x_ld=1 << 31) == E_SHAPE
    assert lr_fwd_g(lib, dt=9) == E_DTYPE
    assert lr_fwd_g(lib, W=1025) == E_UNSUP
    assert lr_fwd_g(lib, x=None) == E_NULL
    assert lr_fwd_g(lib, z=None) == E_NULL
    assert lr_fwd_g(lib, y=arr(P, None, P)) == E_NULL      # a NULL entry
    assert lr_fwd_g(lib, sw=arr(P, P, None)) == E_NULL      # static_w for every group or none
    assert lr_fwd_g(lib, U=arr(P, P + 1, P)) == E_ALIGN
    assert lr_fwd_g(lib, zeff=arr(P, None, P)) == E_NULL    # padded z copies for every group or none
    assert lr_fwd_g(lib, zeff=arr(P, P + 8, P)) == E_ALIGN
    assert lr_fwd_g(lib, R=3, sw=arr(P, P, P), zeff=arr(P, P, P), nzeff=2 * 8 * 4 * 2 - 1) == E_WS
    assert lr_fwd_g(lib, x=P + 1) == E_ALIGN
    assert lr_fwd_g(lib, y_hd=-1) == E_SHAPE               # head dims: D % y_hd == 0, y_hd <= D
    assert lr_fwd_g(lib, y_hd=5) == E_SHAPE
    assert lr_fwd_g(lib, y_hd=32) == E_SHAPE
    if no_dev:
        assert lr_fwd_g(lib) == E_DEV
        assert lr_fwd_g(lib, y_hd=4) == E_DEV               # head-major y [B, 4, T, 4]
        assert lr_fwd_g(lib, y_hd=16) == E_DEV
        assert lr_fwd_g(lib, G=1, x_ld=16, sw=arr(P)) == E_DEV
        assert lr_fwd_g(lib, G=4, x_ld=100, sw=arr(P, P, P, P)) == E_DEV


def test_lowrank_grouped_bwd_validation(lib):
    no_dev = not torch.cuda.is_available()
    one = lib.dc_lowrank_bwd_ws_bytes(2, 8, 16, 4, 4, 0, 1)
    need = lib.dc_lowrank_bwd_grouped_ws_bytes(3, 2, 8, 16, 4, 4, 0, 1)
    assert need == 3 * ((one + 255) // 256 * 256)
    assert lib.dc_lowrank_bwd_grouped_ws_bytes(0, 2, 8, 16, 4, 4, 0, 1) == E_UNSUP
    assert lib.dc_lowrank_bwd_grouped_ws_bytes(3, 2, 8, 16, 0, 4, 0, 1) == E_SHAPE
    g3 = arr(P, P, P)

    def call(G=3, x_ld=48, dx_ld=48, sw=None, dsw=None, ws=P, nws=need, dz=g3, dy=g3, dy_hd=0, zeff=None,
             nzeff=1 << 20, R=4):
        return lib.dc_lowrank_bwd_grouped(G, P, x_ld, g3, g3, sw, zeff, nzeff, dy, dy_hd, P, dx_ld, dz, g3, dsw, ws,
                                          nws, 2, 8, 16, R, 4, 0, 0, None)

    assert call(G=5) == E_UNSUP
    assert call(dx_ld=40) == E_SHAPE
    assert call(x_ld=40) == E_SHAPE
    assert call(sw=g3, dsw=None) == E_NULL
    assert call(sw=None, dsw=g3) == E_NULL
    assert call(dz=arr(P, None, P)) == E_NULL
    assert call(dy=None) == E_NULL
    assert call(zeff=arr(P, P, None)) == E_NULL
    assert call(zeff=arr(P + 8, P, P)) == E_ALIGN
    need3 = lib.dc_lowrank_bwd_grouped_ws_bytes(3, 2, 8, 16, 3, 4, 0, 1)
    assert call(R=3, sw=g3, dsw=g3, nws=need3, zeff=g3, nzeff=2 * 8 * 4 * 2 - 1) == E_WS
    assert call(sw=g3, dsw=g3, ws=None) == E_WS
    assert call(sw=g3, dsw=g3, nws=need - 256) == E_WS
    assert call(sw=g3, dsw=g3, ws=P + 16) == E_WS           # workspace shares start 256-byte aligned
    assert call(dy_hd=3) == E_SHAPE                         # D % dy_hd != 0
    assert call(dy_hd=-2) == E_SHAPE
    if no_dev:
        assert call(sw=g3, dsw=g3) == E_DEV
        assert call(sw=g3, dsw=g3, dy_hd=8) == E_DEV


def test_headwise_bwd_noalloc_validation(lib):
    """The allocation-free backward: the checks of dc_headwise_bwd, and DC_ERR_SCRATCH for problems whose
    dstatic_w partials exceed the fixed scratch array (the workspace size query's bytes)."""
    no_dev = not torch.cuda.is_available()
    limit = 8 << 20  # DC_NOALLOC_SCRATCH_BYTES

    def call(sw=None, dsw=None, B=2, T=8, D=16, H=4, W=4, dt=0, dy=P):
        return lib.dc_headwise_bwd_noalloc(P, P, sw, dy, P, P, dsw, B, T, D, H, W, dt, 0, None)

    assert call(dt=5) == E_DTYPE
    assert call(H=3) == E_SHAPE
    assert call(W=1025) == E_UNSUP
    assert call(dy=None) == E_NULL
    assert call(sw=P, dsw=None) == E_NULL
    assert call(sw=P + 1, dsw=P) == E_ALIGN
    # the largest shapes: the partials of a wide, long problem exceed the scratch array
    big = dict(B=64, T=1 << 16, D=1 << 15, H=1 << 15, W=16)
    assert lib.dc_headwise_bwd_ws_bytes(big["B"], big["T"], big["D"], big["H"], big["W"], 0, 1) > limit
    assert call(sw=P, dsw=P, **big) == E_SCRATCH
    assert lib.dc_headwise_bwd_ws_bytes(2, 8, 16, 4, 4, 0, 1) <= limit
    if no_dev:
        assert call() == E_DEV
        assert call(sw=P, dsw=P) == E_DEV
        assert call(**big) == E_DEV  # no static filter: no scratch needed, any size


def test_kernel_paths(lib):
    """dc_headwise_path / dc_lowrank_path: the kernel family each BASELINE shape and a few edge shapes
    take (0 generic, 1 vector, 2 matrix cores, 3 fp32 matrix cores, 4 fp32 VALU, 5 headwise wide,
    6 headwise matrix cores);
    host logic only."""
    bf, f16, f32 = 0, 1, 2
    hp, lp = lib.dc_headwise_path, lib.dc_lowrank_path
    for bwd in (0, 1):
        assert hp(2, 1024, 512, 512, 4, f32, 0, bwd) == 1      # configs[0]
        assert hp(4, 4096, 2048, 2048, 4, bf, 1, bwd) == 1     # configs[1]
        assert hp(4, 4096, 2048, 64, 4, bf, 1, bwd) == 1       # configs[2]
        assert lp(4, 4096, 2048, 16, 4, bf, 0, bwd) == 2       # configs[3]
        assert lp(2, 8192, 4096, 31, 4, bf, 1, bwd) == 2       # configs[4]
        assert lp(4, 4096, 2048, 16, 4, f32, 0, bwd) == 3      # the fp32 tier on matrix cores
        assert hp(1, 40, 2048, 2, 4, bf, 1, bwd) == 0          # head size 1024: generic
        assert hp(1, 50, 64, 16, 12, bf, 1, bwd) == 0          # W 12, D 64: generic
        assert hp(4, 4096, 2048, 2048, 12, bf, 1, bwd) == 5    # W 12, head size 1: wide
        assert hp(4, 4096, 2048, 64, 16, f32, 0, bwd) == 5     # W 16, head size 32: wide
        assert hp(4, 4096, 2048, 64, 24, bf, 1, bwd) == 6      # W 24, hs 32: matrix cores (hs 8-64)
        assert hp(4, 4096, 2048, 128, 10, f16, 0, bwd) == 6    # W 10, hs 16
        assert hp(4, 4096, 2048, 256, 12, bf, 1, bwd) == 6     # hs 8: matrix cores (two heads per 16 channels)
        assert hp(4, 4096, 2048, 256, 9, f16, 0, bwd) == 6     # hs 8 at every W 9-32
        assert hp(4, 4096, 2048, 512, 12, bf, 1, bwd) == 5     # hs 4: the wide kernels in both directions
        assert hp(4, 4096, 2048, 64, 9, bf, 1, bwd) == 0       # hs 32, W 9: segments not in 16-byte pieces
        assert hp(1, 50, 96, 96, 20, bf, 1, bwd) == 0          # W 20, D % 64 != 0: generic
        assert hp(1, 50, 256, 2, 9, bf, 1, bwd) == 0           # head size 128, W 9: 18-byte segments
        assert hp(4, 4096, 2048, 64, 33, bf, 1, bwd) == 0      # W 33-1024: generic kernels
        assert hp(1, 64, 256, 256, 1024, f32, 0, bwd) == 0
        assert hp(1, 64, 256, 256, 1025, bf, 0, bwd) < 0       # above DC_MAX_W
        assert lp(1, 45, 64, 127, 12, bf, 1, bwd) == 2         # W 12, kernel rank 128: 2 x 2 forward passes
        assert lp(1, 70, 128, 64, 1, bf, 0, bwd) == 2          # kernel rank 64, W 1
        assert lp(1, 40, 128, 40, 2, f16, 0, bwd) == 2         # kernel rank 40, W 2
    assert lp(1, 300, 64, 1, 1, f32, 0, 0) == 3                # fp32 W 1: forward on fp32 matrix cores,
    assert lp(1, 300, 64, 1, 1, f32, 0, 1) == 4                # backward on the VALU kernels
    for bwd in (0, 1):                                         # fp32 kernel ranks 17-32: the backward
        assert lp(2, 8192, 4096, 31, 4, f32, 1, bwd) == 3      # as two rank passes on matrix cores
        assert lp(1, 100, 256, 32, 2, f32, 0, bwd) == 3
    assert lp(1, 100, 256, 33, 4, f32, 0, 1) == 3              # kernel rank 33: three rank passes
    assert lp(1, 100, 256, 33, 4, f32, 0, 0) == 3              # its forward: two rank passes
    assert lp(1, 100, 256, 65, 4, f32, 0, 1) == 0              # kernel rank 65: the generic kernels
    for bwd in (0, 1):                                         # fp32 sequences past 512 MiB of rows:
        assert lp(1, 65600, 2048, 15, 4, f32, 1, bwd) == 3     # per-run buffer ranges
        assert lp(1, 1 << 20, 4096, 31, 8, f32, 1, bwd) == 3
    for bwd in (0, 1):                                         # fp32 W 5-32: forward passes of 8 taps
        assert lp(1, 100, 256, 16, 20, f32, 1, bwd) == 3       # above W 8, backward passes of 2-4 taps
        assert lp(1, 100, 256, 31, 32, f32, 0, bwd) == 3
        assert lp(4, 4096, 2048, 16, 8, f32, 0, bwd) == 3
        assert lp(1, 100, 256, 31, 5, f32, 1, bwd) == 3
    for bwd in (0, 1):                                         # every W <= 8 at every kernel rank <= 64:
        assert lp(2, 50, 256, 63, 2, bf, 1, bwd) == 2          # the backward as passes of taps
        assert lp(2, 8192, 4096, 31, 8, bf, 1, bwd) == 2       # W 8, two rank chunks
        assert lp(1, 64, 256, 40, 5, f16, 0, bwd) == 2         # W 5, three rank chunks
        assert lp(1, 64, 256, 63, 8, bf, 1, bwd) == 2          # W 8, four rank chunks
        assert lp(1, 64, 256, 64, 8, bf, 1, bwd) == 2          # kernel rank 65: passes of ranks
        assert lp(2, 300, 256, 16, 12, bf, 0, bwd) == 2        # W 9-16 at kernel ranks <= 32
        assert lp(2, 77, 200, 31, 16, bf, 1, bwd) == 2
        assert lp(1, 64, 256, 40, 9, f16, 0, bwd) == 2         # W 9, kernel rank 40: passes of taps
        assert lp(1, 64, 256, 16, 17, bf, 0, bwd) == 2         # W 17-32 at kernel ranks <= 32: the forward in
        assert lp(4, 4096, 2048, 31, 32, f16, 1, bwd) == 2     # one or two passes, backward tap passes
        assert lp(1, 64, 256, 40, 17, bf, 0, bwd) == 2         # W 17, kernel rank 40: passes of taps
        assert lp(1, 64, 256, 64, 32, bf, 0, bwd) == 2         # W 32, kernel rank 64
        assert lp(1, 64, 256, 65, 4, bf, 0, bwd) == 2          # kernel rank 65: passes of ranks
        assert lp(1, 64, 256, 16, 33, bf, 0, bwd) == 0         # W 33-1024: generic kernels
        assert lp(1, 64, 256, 16, 1025, bf, 0, bwd) < 0        # W 1025: above DC_MAX_W
    for bwd in (0, 1):                                         # kernel ranks 65-256 as passes of ranks
        assert lp(4, 4096, 2048, 127, 4, bf, 1, bwd) == 2      # (forward 128 per pass up to W 4, 64 above; backward 32)
        assert lp(1, 64, 256, 255, 8, f16, 1, bwd) == 2        # kernel rank 256, W 8: 4 forward passes
        assert lp(1, 64, 256, 100, 16, bf, 0, bwd) == 2        # 2 x 2 forward passes
    assert lp(1, 64, 256, 127, 20, bf, 1, 0) == 0              # 2 x 3 forward passes (y rounded 6 times):
    assert lp(1, 64, 256, 127, 20, bf, 1, 1) == 2              # generic forward; backward on matrix cores
    assert lp(1, 64, 256, 255, 9, bf, 1, 0) == 0               # 4 x 2 forward passes: generic
    assert lp(1, 64, 256, 256, 4, bf, 1, 0) == E_UNSUP         # kernel rank 257: above DC_MAX_R
    for bwd in (0, 1):                                         # D a multiple of 8, not of 16
        assert lp(2, 100, 200, 16, 4, bf, 0, bwd) == 2
        assert lp(1, 50, 1000, 15, 3, f16, 1, bwd) == 2
        assert lp(2, 100, 20, 16, 4, bf, 0, bwd) == 0          # D % 8 != 0: generic
    assert hp(2, 8, 16, 3, 4, bf, 0, 0) == E_SHAPE
    assert lp(2, 8, 16, 0, 4, bf, 0, 0) == E_SHAPE
    assert lp(2, 8, 16, 4, 1025, bf, 0, 1) == E_UNSUP


def test_proj_in_validation(lib):
    """dc_proj_in_*: shape limits of the matrix-core kernels (G*R <= 128, K % 8 == 0, 16-bit types),
    pointers and workspace, before any device call."""
    no_dev = not torch.cuda.is_available()
    g3 = arr(P, P, P)
    fwd = lambda G=3, M=64, K=256, R=31, dt=0, pre=P, w=P, z=g3: lib.dc_proj_in_fwd(pre, w, z, G, M, K, R, dt, None)  # noqa: E731
    assert fwd(dt=7) == E_DTYPE
    assert fwd(dt=2) == E_UNSUP          # fp32: a library GEMM takes it
    assert fwd(R=43) == E_UNSUP          # G*R = 129 > 128
    assert fwd(K=100) == E_UNSUP         # K % 8 != 0
    assert fwd(G=5, z=arr(P, P, P, P, P)) == E_UNSUP
    assert fwd(M=0) == E_SHAPE
    assert fwd(pre=None) == E_NULL
    assert fwd(z=arr(P, None, P)) == E_NULL
    assert fwd(pre=P + 8) == E_ALIGN
    need = lib.dc_proj_in_bwd_ws_bytes(3, 64, 256, 31, 0)
    assert need > 0 and need % (3 * 31 * 256 * 4) == 0   # one fp32 dW_in partial per row run
    bwd = lambda ws=P, nws=need, dz=g3, dpre=P: lib.dc_proj_in_bwd(P, P, dz, dpre, P, ws, nws, 3, 64, 256, 31, 0, None)  # noqa: E731
    assert bwd(ws=None) == E_WS
    assert bwd(nws=need - 4) == E_WS
    assert bwd(dz=arr(P, P, None)) == E_NULL
    assert bwd(dpre=P + 2) == E_ALIGN
    if no_dev:
        assert fwd() == E_DEV
        assert fwd(G=1, z=arr(P), R=128) == E_DEV
        assert bwd() == E_DEV


def _plan_ranges(lib, B, T, D, R, W, dt, st, bwd):
    """(bytes, bound) pairs of dc_lowrank_plan_ranges for one shape."""
    import ctypes

    n = lib.dc_lowrank_plan_ranges(B, T, D, R, W, dt, st, bwd, None, 0)
    assert n >= 0, (B, T, D, R, W, dt, st, bwd, n)
    buf = (ctypes.c_int64 * (2 * max(n, 1)))()
    assert lib.dc_lowrank_plan_ranges(B, T, D, R, W, dt, st, bwd, buf, n) == n
    return [(buf[2 * i], buf[2 * i + 1]) for i in range(n)]


def test_plan_buffer_ranges(lib):
    """Every launch plan of the matrix-core and fp32 lowrank kernels, for every tap and rank pass split
    at W <= 32 and kernel rank <= 256 (bf16, fp16; fp32 up to its kernel rank 64), forward and backward:
    each buffer resource's byte count, as the kernels compute it before make_rsrc's clamp, lies in
    [0, bound], where bound keeps the kernel's out-of-range offsets (a lane's 1 << 30, a tile's 1 << 29
    less 15 rows of halo) out of range.  A negative count (a pass whose offsets run past its rows, as the
    static-rank-only fp32 pass once did) or one that reaches an out-of-range offset fails here, on the
    CPU, before any launch.  Host logic only: the audit launches nothing."""
    dts = {0: 256, 1: 256, 2: 64}  # dtype: largest kernel rank to enumerate
    n_pairs = n_plans = 0
    for dt, rk_max in dts.items():
        for W in range(1, 33):
            for rk in list(range(1, 67)) + [95, 96, 97, 127, 128, 129, 160, 200, 255, 256]:
                if rk > rk_max:
                    continue
                for st in (0, 1):
                    R = rk - st
                    if R < 1:
                        continue
                    for bwd in (0, 1):
                        for B, T, D in ((2, 100, 256), (1, 50, 72)):
                            pairs = _plan_ranges(lib, B, T, D, R, W, dt, st, bwd)
                            n_plans += 1
                            n_pairs += len(pairs)
                            for i, (v, bound) in enumerate(pairs):
                                assert 0 <= v <= bound, (dict(B=B, T=T, D=D, R=R, W=W, dtype=dt, static=st, bwd=bwd),
                                                         i, v, bound)
    assert n_plans > 10000 and n_pairs > 10 * n_plans


def test_plan_buffer_ranges_long_sequences(lib):
    """The per-run resources of sequences past 512 MiB of rows (capped runs) and the widest rows:
    every count within its bound, for the BASELINE shapes at long T and the rank / tap pass splits."""
    shapes = [(1, 131172, 2048, 15, 4, 1), (1, 131172, 2048, 16, 4, 0), (1, 1 << 20, 4096, 31, 8, 1),
              (1, 65600, 2048, 127, 4, 1), (1, 32800, 4096, 63, 20, 1), (2, 8192, 4096, 255, 8, 1),
              (1, 400000, 64, 31, 32, 1)]
    for B, T, D, R, W, st in shapes:
        for dt in (0, 1, 2):
            for bwd in (0, 1):
                for i, (v, bound) in enumerate(_plan_ranges(lib, B, T, D, R, W, dt, st, bwd)):
                    assert 0 <= v <= bound, ((B, T, D, R, W, dt, st, bwd), i, v, bound)


def test_plan_ranges_catch_a_negative_count(lib):
    """The audit reports the pre-clamp counts: a plan whose U range would be negative shows up as
    one.  Checked on the shared count function's arithmetic through a shape that has a static-rank-only
    pass of ranks at a later pass of taps (fp32 kernel rank 33, W 12: rank pass 2 holds the static rank
    alone, its tap passes start at kofs > 0) -- the count must be 0 there, not R * uld - kofs * D < 0."""
    pairs = _plan_ranges(lib, 1, 60, 64, 32, 12, 2, 1, 0)
    assert pairs and all(0 <= v <= b for v, b in pairs)
    assert any(v == 0 for v, _ in pairs)  # the empty U range of the static-rank-only pass
