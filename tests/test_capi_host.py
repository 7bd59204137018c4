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
    assert len(names) == 8, names
    raw = ctypes.CDLL(_capi.LIB_PATH)
    for n in names:
        assert hasattr(raw, n), f"{n} declared in dynconv.h but not exported"
    assert set(names) == set(_capi.SIGNATURES), "ctypes signatures out of sync with the header"


def test_abi_version_and_strings(lib):
    assert lib.dc_abi_version() == 1
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
    if no_dev:
        assert hw_bwd(lib) == E_DEV
        assert hw_bwd(lib, sw=P, dsw=P, ws=P, nws=need) == E_DEV


def lr_fwd(lib, x=P, z=P, U=P, sw=None, B=2, T=8, D=16, R=4, W=4, dt=0):
    return lib.dc_lowrank_fwd(x, z, U, sw, P, B, T, D, R, W, dt, 0, None)


def test_lowrank_validation(lib):
    no_dev = not torch.cuda.is_available()
    assert lr_fwd(lib, dt=-1) == E_DTYPE
    assert lr_fwd(lib, R=0) == E_SHAPE
    assert lr_fwd(lib, R=64, sw=P) == E_UNSUP    # kernel rank 65 > DC_MAX_R
    assert lr_fwd(lib, R=65) == E_UNSUP
    assert lr_fwd(lib, W=0) == E_SHAPE
    assert lr_fwd(lib, z=None) == E_NULL
    assert lr_fwd(lib, U=P + 1) == E_ALIGN
    need = lib.dc_lowrank_bwd_ws_bytes(2, 8, 16, 4, 4, 0, 1)
    assert need > 0
    assert lib.dc_lowrank_bwd_ws_bytes(2, 8, 16, 4, 9, 0, 1) == E_UNSUP
    st = lib.dc_lowrank_bwd(P, P, P, P, P, P, P, P, P, None, 0, 2, 8, 16, 4, 4, 0, 0, None)
    assert st == E_WS
    st = lib.dc_lowrank_bwd(P, P, P, None, P, P, P, P, P, P, need, 2, 8, 16, 4, 4, 0, 0, None)
    assert st == E_NULL
    if no_dev:
        assert lr_fwd(lib) == E_DEV
        st = lib.dc_lowrank_bwd(P, P, P, P, P, P, P, P, P, P, need, 2, 8, 16, 4, 4, 0, 0, None)
        assert st == E_DEV
