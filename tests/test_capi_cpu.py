"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares, and its (host-only) QLinearConv dispatch agrees with the
oracle's restatement of QLinearConv::exec_simd_4d on a grid of shapes.
No GPU call is made here."""
import itertools
import os
import re

import numpy as np
import pytest

import nnr_amd
from nnr_amd import _lib
from oracle import pyoracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    txt = open(os.path.join(ROOT, "include", "nnr_hip.h")).read()
    return sorted(set(re.findall(r"\b(nnrh_[a-z0-9_]+)\s*\(", txt)))


def test_header_symbols_exported():
    L = _lib.lib()
    syms = header_symbols()
    assert len(syms) >= 30
    for s in syms:
        assert hasattr(L, s), s
    assert sorted(_lib.EXPORTS) == syms


def test_every_export_has_a_signature():
    """ctypes passes Python ints as 32-bit C ints when a function has no
    argtypes, which truncates device pointers: every exported entry point
    must have its argument types declared."""
    L = _lib.lib()
    for s in _lib.EXPORTS:
        assert getattr(L, s).argtypes is not None, s


def test_host_export_signatures():
    from nnr_amd import graph as G
    txt = open(os.path.join(ROOT, "include", "nnr_host.h")).read()
    L = G.host_lib()
    for s in sorted(set(re.findall(r"\b(nnr_[a-z0-9_]+)\s*\(", txt))):
        assert getattr(L, s).argtypes is not None, s


def test_host_header_symbols_exported():
    """Every nnr_ctx_* / nnr_* entry of include/nnr_host.h is exported by the
    host framework library."""
    import ctypes
    from nnr_amd import graph as G
    txt = open(os.path.join(ROOT, "include", "nnr_host.h")).read()
    syms = sorted(set(re.findall(r"\b(nnr_[a-z0-9_]+)\s*\(", txt)))
    assert len(syms) >= 15
    L = G.host_lib()
    for s in syms:
        assert hasattr(L, s), s
    assert isinstance(L, ctypes.CDLL)


def test_version_and_errors():
    L = _lib.lib()
    assert b"gfx950" in L.nnrh_version()
    br = __import__("ctypes").c_int()
    d, _keep = nnr_amd._conv_desc(1, 8, 8, 8, np.zeros((6, 4, 3, 3), np.int8), group=2)
    d.oH = 99                      # inconsistent output size must be rejected
    rc = L.nnrh_qconv_dispatch(__import__("ctypes").byref(d), __import__("ctypes").byref(br))
    assert rc == _lib.NNRH_ERR_INVALID
    assert b"output" in L.nnrh_last_error()


GRID = list(itertools.product(
    [1, 3, 4, 16, 64],            # C
    [1, 3, 7],                    # k
    [1, 2],                       # stride
    [0, 1],                       # x_nhwc
    [0, 1],                       # y_nhwc
    ["g1", "dw", "g2"],           # grouping
    [0, 1],                       # post_fn
))


@pytest.mark.parametrize("C,k,s,xn,yn,grp,post", GRID[::3])
def test_dispatch_matches_oracle(C, k, s, xn, yn, grp, post):
    OC = {"g1": 32, "dw": C, "g2": 2 * C}[grp]
    G = {"g1": 1, "dw": C, "g2": 2 if C % 2 == 0 else 1}[grp]
    if grp == "g2" and G == 1:
        OC = 32
    H = W = 9 if k == 7 else 12
    p = k // 2
    w = np.zeros((OC, C // G, k, k), np.int8)
    for act, wzp in [(np.uint8, ()), (np.int8, ()), (np.uint8, (3,))]:
        kw = dict(group=G, stride=(s, s), pads=(p, p, p, p), x_nhwc=xn, y_nhwc=yn,
                  post_fn=post, act_dtype=act, w_zp=wzp)
        br = nnr_amd.conv_dispatch(1, C, H, W, w, **kw)
        ocv = O.Conv(1, C, H, W, OC, k, k, **kw)
        assert br == ocv.dispatch(), (C, k, s, xn, yn, grp, post, act, wzp)


def test_group_create_errors():
    """nnr_group_create refuses a missing context list before touching a
    GPU; destroying a NULL group is a no-op."""
    import ctypes as C
    from nnr_amd import graph as G
    L = G.host_lib()
    g = C.c_void_p()
    assert L.nnr_group_create(None, 0, C.byref(g)) != 0
    assert b"no contexts" in L.nnr_last_error()
    assert g.value is None
    assert L.nnr_group_destroy(None) == 0
