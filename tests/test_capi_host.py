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

OK, E_NULL, E_SHAPE, E_DTYPE, E_UNSUP, E_WS, E_ALIGN, E_DEV, E_LAUNCH = 0, -1, -2, -3, -4, -5, -6, -7, -8
P = 0x10000  # a fake, 256-byte aligned "device pointer"; never dereferenced on these paths


@pytest.fixture(scope="module")
def lib():
    return _capi.load()


def header_functions():
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\*\s]+?\b(dc_\w+)\s*\(", txt, re.M)))


def test_exports_every_declared_symbol(lib):
    names = header_functions()
    assert len(names) == 12, names
    raw = ctypes.CDLL(_capi.LIB_PATH)
    for n in names:
        assert hasattr(raw, n), f"{n} declared in dynconv.h but not exported"
    assert set(names) == set(_capi.SIGNATURES), "ctypes signatures out of sync with the header"


def test_abi_version_and_strings(lib):
    assert lib.dc_abi_version() == 4
    for s in (OK, E_NULL, E_SHAPE, E_DTYPE, E_UNSUP, E_WS, E_ALIGN, E_DEV, E_LAUNCH):
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
    assert hw_fwd(lib, W=9) == E_UNSUP           # > DC_MAX_W
    assert hw_fwd(lib, T=1 << 31) == E_SHAPE     # int32 row indexing bound
    assert hw_fwd(lib, x=None) == E_NULL
    assert hw_fwd(lib, y=None) == E_NULL
    assert hw_fwd(lib, x=P + 1) == E_ALIGN       # bf16 needs 2-byte alignment
    assert hw_fwd(lib, x=P + 2, dt=2) == E_ALIGN  # fp32 needs 4
    if no_dev:
        assert hw_fwd(lib) == E_DEV
        assert hw_fwd(lib, sw=P, res=1, W=1) == E_DEV


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


def lr_fwd(lib, x=P, z=P, U=P, sw=None, zeff=None, B=2, T=8, D=16, R=4, W=4, dt=0):
    return lib.dc_lowrank_fwd(x, z, U, sw, P, zeff, B, T, D, R, W, dt, 0, None)


def test_lowrank_validation(lib):
    no_dev = not torch.cuda.is_available()
    assert lr_fwd(lib, dt=-1) == E_DTYPE
    assert lr_fwd(lib, R=0) == E_SHAPE
    assert lr_fwd(lib, R=64, sw=P) == E_UNSUP    # kernel rank 65 > DC_MAX_R
    assert lr_fwd(lib, R=65) == E_UNSUP
    assert lr_fwd(lib, W=0) == E_SHAPE
    assert lr_fwd(lib, z=None) == E_NULL
    assert lr_fwd(lib, U=P + 1) == E_ALIGN
    assert lr_fwd(lib, zeff=P + 8) == E_ALIGN      # the padded z copy: 16-byte aligned
    # the padded z copy the backward would build: none when z's own rows serve (R % 4 == 0,
    # or 32 dynamic ranks for two rank chunks), else B*T rows of 4*k (one chunk) or 32 ranks
    zb = lib.dc_lowrank_zeff_bytes
    assert zb(2, 8, 16, 4, 4, 0, 1) == 0
    assert zb(2, 8, 16, 3, 4, 0, 1) == 2 * 8 * 4 * 2
    assert zb(2, 8, 16, 15, 4, 1, 1) == 2 * 8 * 16 * 2
    assert zb(2, 8, 16, 31, 4, 0, 1) == 2 * 8 * 32 * 2
    assert zb(2, 8, 16, 32, 4, 0, 0) == 0
    assert zb(2, 8, 16, 28, 4, 0, 0) == 2 * 8 * 32 * 2
    assert zb(2, 8, 16, 3, 4, 2, 1) == 0              # fp32: the backward reads z itself
    assert zb(2, 8, 20, 3, 4, 0, 1) == 0              # D % 16 != 0: no matrix-core backward
    assert zb(2, 8, 16, 0, 4, 0, 1) == E_SHAPE
    need = lib.dc_lowrank_bwd_ws_bytes(2, 8, 16, 4, 4, 0, 1)
    assert need > 0
    assert lib.dc_lowrank_bwd_ws_bytes(2, 8, 16, 4, 9, 0, 1) == E_UNSUP
    st = lib.dc_lowrank_bwd(P, P, P, P, None, P, P, P, P, P, None, 0, 2, 8, 16, 4, 4, 0, 0, None)
    assert st == E_WS
    st = lib.dc_lowrank_bwd(P, P, P, P, None, P, P, P, P, P, P + 8, need, 2, 8, 16, 4, 4, 0, 0, None)
    assert st == E_WS  # workspace below 16-byte alignment
    st = lib.dc_lowrank_bwd(P, P, P, None, None, P, P, P, P, P, P, need, 2, 8, 16, 4, 4, 0, 0, None)
    assert st == E_NULL
    st = lib.dc_lowrank_bwd(P, P, P, P, P + 8, P, P, P, P, P, P, need, 2, 8, 16, 4, 4, 0, 0, None)
    assert st == E_ALIGN  # the padded z copy below 16-byte alignment
    if no_dev:
        assert lr_fwd(lib) == E_DEV
        assert lr_fwd(lib, R=3, sw=P, zeff=P) == E_DEV
        st = lib.dc_lowrank_bwd(P, P, P, P, None, P, P, P, P, P, P, need, 2, 8, 16, 4, 4, 0, 0, None)
        assert st == E_DEV
        st = lib.dc_lowrank_bwd(P, P, P, P, P, P, P, P, P, P, P, need, 2, 8, 16, 3, 4, 0, 0, None)
        assert st == E_DEV


def arr(*ptrs):
    """A host array of fake device pointers (a `const void* const*` argument)."""
    return (ctypes.c_void_p * len(ptrs))(*ptrs)


def lr_fwd_g(lib, G=3, x=P, x_ld=48, z="ok", U="ok", sw=None, y="ok", zeff=None, y_hd=0, B=2, T=8, D=16, R=4, W=4,
             dt=0):
    z = arr(*[P] * G) if z == "ok" else z
    U = arr(*[P] * G) if U == "ok" else U
    y = arr(*[P] * G) if y == "ok" else y
    return lib.dc_lowrank_fwd_grouped(G, x, x_ld, z, U, sw, y, zeff, y_hd, B, T, D, R, W, dt, 0, None)


def test_lowrank_grouped_fwd_validation(lib):
    no_dev = not torch.cuda.is_available()
    assert lr_fwd_g(lib, G=0) == E_UNSUP
    assert lr_fwd_g(lib, G=5, x_ld=80) == E_UNSUP          # > DC_MAX_GROUPS
    assert lr_fwd_g(lib, x_ld=47) == E_SHAPE               # rows narrower than G*D
    assert lr_fwd_g(lib, x_ld=1 << 31) == E_SHAPE
    assert lr_fwd_g(lib, dt=9) == E_DTYPE
    assert lr_fwd_g(lib, W=9) == E_UNSUP
    assert lr_fwd_g(lib, x=None) == E_NULL
    assert lr_fwd_g(lib, z=None) == E_NULL
    assert lr_fwd_g(lib, y=arr(P, None, P)) == E_NULL      # a NULL entry
    assert lr_fwd_g(lib, sw=arr(P, P, None)) == E_NULL      # static_w for every group or none
    assert lr_fwd_g(lib, U=arr(P, P + 1, P)) == E_ALIGN
    assert lr_fwd_g(lib, zeff=arr(P, None, P)) == E_NULL    # padded z copies for every group or none
    assert lr_fwd_g(lib, zeff=arr(P, P + 8, P)) == E_ALIGN
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

    def call(G=3, x_ld=48, dx_ld=48, sw=None, dsw=None, ws=P, nws=need, dz=g3, dy=g3, dy_hd=0, zeff=None):
        return lib.dc_lowrank_bwd_grouped(G, P, x_ld, g3, g3, sw, zeff, dy, dy_hd, P, dx_ld, dz, g3, dsw, ws, nws,
                                          2, 8, 16, 4, 4, 0, 0, None)

    assert call(G=5) == E_UNSUP
    assert call(dx_ld=40) == E_SHAPE
    assert call(x_ld=40) == E_SHAPE
    assert call(sw=g3, dsw=None) == E_NULL
    assert call(sw=None, dsw=g3) == E_NULL
    assert call(dz=arr(P, None, P)) == E_NULL
    assert call(dy=None) == E_NULL
    assert call(zeff=arr(P, P, None)) == E_NULL
    assert call(zeff=arr(P + 8, P, P)) == E_ALIGN
    assert call(sw=g3, dsw=g3, ws=None) == E_WS
    assert call(sw=g3, dsw=g3, nws=need - 256) == E_WS
    assert call(sw=g3, dsw=g3, ws=P + 16) == E_WS           # workspace shares start 256-byte aligned
    assert call(dy_hd=3) == E_SHAPE                         # D % dy_hd != 0
    assert call(dy_hd=-2) == E_SHAPE
    if no_dev:
        assert call(sw=g3, dsw=g3) == E_DEV
        assert call(sw=g3, dsw=g3, dy_hd=8) == E_DEV
