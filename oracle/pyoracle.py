"""ctypes view of the CPU oracle (oracle/nnr_oracle.h).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
the cpu_baseline leg of bench.py, never by the product (nnr_amd/).
"""
from __future__ import annotations

import ctypes as ct
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "build", "liboracle.so")
U8, S8, I32, F32, F16 = range(5)
BR = {"DW": 1, "FIRST": 2, "DIRECT": 3, "PACKED": 4, "NR16": 5, "IM2COL_S1": 6,
      "IM2COL": 7, "FLOAT": 8}


class ConvParams(ct.Structure):
    _fields_ = [(n, ct.c_int) for n in (
        "N", "C", "H", "W", "OC", "kH", "kW", "group", "sH", "sW", "dH", "dW",
        "pad_t", "pad_l", "pad_b", "pad_r", "oH", "oW", "x_nhwc", "y_nhwc", "post_fn",
        "act_dtype")] + [
        ("x_scale", ct.c_float), ("x_zp", ct.c_int),
        ("w_scale", ct.POINTER(ct.c_float)), ("w_scale_count", ct.c_int),
        ("w_zp", ct.POINTER(ct.c_int8)), ("w_zp_count", ct.c_int),
        ("y_scale", ct.c_float), ("y_zp", ct.c_int),
        ("bias", ct.POINTER(ct.c_int32)), ("vnni", ct.c_int)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            import subprocess
            subprocess.run(["make", "-C", _HERE, "CC=gcc"], check=True,
                           stdout=subprocess.DEVNULL)
        L = ct.CDLL(LIB_PATH)
        i, f, vp, sz = ct.c_int, ct.c_float, ct.c_void_p, ct.c_size_t
        P = ct.POINTER
        sigs = {
            "orc_set_contract": (None, [i]),
            "orc_set_vnni": (None, [i]),
            "orc_get_vnni": (i, []),
            "orc_vnni_available": (i, []),
            "orc_set_host_threads": (None, [i, i]),
            "orc_int8_compute_threads": (i, [i, ct.c_longlong]),
            "orc_vnni_cache": (None, [i]),
            "orc_set_threads": (None, [i]),
            "orc_get_threads": (i, []),
            "orc_f32_to_f16": (ct.c_uint16, [f]),
            "orc_f16_to_f32": (f, [ct.c_uint16]),
            "orc_rq_a": (i, [ct.c_int32, f, f, f, i, i, i]),
            "orc_rq_a_tail": (i, [ct.c_int32, f, f, f, i, i, i]),
            "orc_rq_b": (i, [ct.c_int32, ct.c_int32, f, i, i, i]),
            "orc_rq_b_roundf": (i, [ct.c_int32, ct.c_int32, f, i, i, i]),
            "orc_rq_c": (i, [ct.c_int32, f, f, f, i, i, i]),
            "orc_rq_d": (i, [ct.c_int32, f, i, i, i]),
            "orc_quantize_linear": (None, [vp, sz, f, i, i, vp]),
            "orc_dequantize_linear": (None, [vp, i, sz, f, i, vp]),
            "orc_hardswish_f32": (None, [vp, vp, sz, i]),
            "orc_dynamic_quantize_linear": (None, [vp, sz, vp, vp, vp]),
            "orc_qlinear_matmul": (i, [i, i, i, i, vp, i, i, vp, vp, vp, i, i, vp, vp, vp, vp,
                                       i, vp, i]),
            "orc_qmatmul_combined_scale": (f, [vp, vp, vp, i]),
            "orc_matmul_integer": (i, [vp, i, vp, i, vp, i, vp, i, i, i, vp]),
            "orc_conv_out_dim": (i, [i, i, i, i, i, i]),
            "orc_conv_dispatch": (i, [P(ConvParams)]),
            "orc_conv_acc": (None, [P(ConvParams), vp, vp, vp]),
            "orc_qlinear_conv": (i, [P(ConvParams), vp, vp, vp]),
            "orc_qlinear_conv1d": (i, [P(ConvParams), vp, vp, vp]),
            "orc_qlinear_conv_from_acc": (i, [P(ConvParams), vp, vp]),
            "orc_qlinear_add": (None, [i, vp, vp, vp, sz, i, i, i, i, i, f, i, f, i, f, i]),
            "orc_maxpool_u8_nhwc": (None, [vp, vp] + [i] * 12),
            "orc_qlinear_global_avgpool": (None, [vp, vp, i, i, i, i, i, f, i, f, i]),
            "orc_qlinear_avgpool": (None, [vp, vp] + [i] * 14 + [f, i, f, i]),
            "orc_qlinear_concat": (None, [i, P(vp), P(ct.c_longlong), ct.c_longlong, i, P(f), P(i), f, i, vp]),
            "orc_qlinear_mul": (None, [i, vp, vp, vp, sz, i, i, i, i, i, f, i, f, i, f, i]),
            "orc_nchw_to_nhwc_u8": (None, [vp, vp, i, i, i]),
            "orc_fold_bn": (None, [i, vp, vp, vp, vp, f, i, f, i, f, i, vp, vp]),
            "orc_conv_integer": (None, [vp, i, vp, i, i, vp] + [i] * 16 + [vp]),
            "orc_batchnorm_u8": (None, [vp, i, vp, vp, vp, ct.c_longlong, i, ct.c_longlong, i]),
        }
        for n, (r, a) in sigs.items():
            fn = getattr(L, n)
            fn.restype = r
            fn.argtypes = a
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def dt_of(a):
    return {np.dtype(np.uint8): U8, np.dtype(np.int8): S8, np.dtype(np.int32): I32,
            np.dtype(np.float32): F32}[a.dtype]


def set_threads(n):
    lib().orc_set_threads(int(n))


def set_contract(on):
    lib().orc_set_contract(1 if on else 0)


# ---- element ops ---------------------------------------------------------------
def quantize_linear(x, scale, zp, dtype=np.uint8):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=dtype)
    lib().orc_quantize_linear(_p(x), x.size, float(scale), int(zp), dt_of(y), _p(y))
    return y


def dequantize_linear(x, scale, zp):
    x = np.ascontiguousarray(x)
    y = np.empty(x.shape, dtype=np.float32)
    lib().orc_dequantize_linear(_p(x), dt_of(x), x.size, float(scale), int(zp), _p(y))
    return y


def hardswish(x, post_op=False):
    """fp32 HardSwish with the reference's body / tail split over x's flat order."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.float32)
    lib().orc_hardswish_f32(_p(x), _p(y), x.size, 1 if post_op else 0)
    return y


def dynamic_quantize_linear(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint8)
    s = np.zeros(1, np.float32)
    z = np.zeros(1, np.uint8)
    lib().orc_dynamic_quantize_linear(_p(x), x.size, _p(y), _p(s), _p(z))
    return y, float(s[0]), int(z[0])


def qlinear_matmul(a, a_scale, a_zp, b, b_scale, b_zp, y_scale, y_zp, y_dtype=np.uint8,
                   scale_dtype=np.float32):
    """a: [batch?, m, k]; b: [batch?, k, n]; per-tensor params (scalars)."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    a3 = a.reshape((-1,) + a.shape[-2:])
    b3 = b.reshape((-1,) + b.shape[-2:])
    batch = max(a3.shape[0], b3.shape[0])
    m, k = a3.shape[1:]
    n = b3.shape[2]
    sd = F16 if scale_dtype == np.float16 else F32
    sc = lambda v: np.array([v], dtype=scale_dtype)
    a_s, b_s, y_s = sc(a_scale), sc(b_scale), sc(y_scale)
    a_z, b_z = np.array([a_zp], a.dtype), np.array([b_zp], b.dtype)
    y_z = np.array([y_zp], y_dtype)
    y = np.empty((batch, m, n), dtype=y_dtype)
    lib().orc_qlinear_matmul(batch, m, n, k, _p(a3), dt_of(a3), a3.shape[0], _p(a_s), _p(a_z),
                             _p(b3), dt_of(b3), b3.shape[0], _p(b_s), _p(b_z), _p(y_s), _p(y_z),
                             sd, _p(y), dt_of(y))
    lead = a.shape[:-2] if a3.shape[0] >= b3.shape[0] else b.shape[:-2]
    return y.reshape(lead + (m, n))


def qmatmul_combined_scale(a_s, b_s, y_s, scale_dtype=np.float32):
    sd = F16 if scale_dtype == np.float16 else F32
    arr = [np.array([v], dtype=scale_dtype) for v in (a_s, b_s, y_s)]
    return float(lib().orc_qmatmul_combined_scale(*[_p(x) for x in arr], sd))


def matmul_integer(a, b, a_zp=0, b_zp=0):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    ad = np.array(a.shape, np.int32)
    bd = np.array(b.shape, np.int32)
    a2 = list(a.shape) if a.ndim > 1 else [1, a.shape[0]]
    b2 = list(b.shape) if b.ndim > 1 else [b.shape[0], 1]
    nd = max(len(a2), len(b2))
    a2 = [1] * (nd - len(a2)) + a2
    b2 = [1] * (nd - len(b2)) + b2
    lead = [max(x, y) for x, y in zip(a2[:-2], b2[:-2])]
    y = np.empty(lead + [a2[-2], b2[-1]], np.int32)
    rc = lib().orc_matmul_integer(_p(ad), a.ndim, _p(a), dt_of(a), _p(bd), b.ndim, _p(b),
                                  dt_of(b), int(a_zp), int(b_zp), _p(y))
    assert rc == 0
    return y


def qlinear_add(kind, a, b, a_s, a_zp, b_s, b_zp, y_s, y_zp, C=0, HW=0, y_nhwc=0):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    full = a if a.size >= b.size else b
    y = np.empty(full.shape, a.dtype)
    N = full.size // (C * HW) if C and HW else 0
    lib().orc_qlinear_add(kind, _p(a), _p(b), _p(y), y.size, N, C, HW, y_nhwc, dt_of(a),
                          float(a_s), int(a_zp), float(b_s), int(b_zp), float(y_s), int(y_zp))
    return y


def qlinear_global_avgpool(x, x_s, x_zp, y_s, y_zp, nhwc=0):
    """x: [N, C, *spatial] (or [N, *spatial, C] with nhwc); y: [N, C]."""
    x = np.ascontiguousarray(x)
    N = x.shape[0]
    C = x.shape[-1] if nhwc else x.shape[1]
    sp = x.size // (N * C)
    y = np.empty((N, C), x.dtype)
    lib().orc_qlinear_global_avgpool(_p(x), _p(y), N, C, sp, nhwc, dt_of(x), float(x_s), int(x_zp),
                                     float(y_s), int(y_zp))
    return y


def qlinear_avgpool(x, k, stride, pads, oH, oW, x_s, x_zp, y_s, y_zp, nhwc=0):
    x = np.ascontiguousarray(x)
    if nhwc:
        N, H, W, Cc = x.shape
        y = np.empty((N, oH, oW, Cc), x.dtype)
    else:
        N, Cc, H, W = x.shape
        y = np.empty((N, Cc, oH, oW), x.dtype)
    lib().orc_qlinear_avgpool(_p(x), _p(y), N, Cc, H, W, oH, oW, k[0], k[1], stride[0], stride[1],
                              pads[0], pads[1], nhwc, dt_of(x), float(x_s), int(x_zp), float(y_s), int(y_zp))
    return y


def qlinear_concat(xs, counts, outer, scales, zps, y_s, y_zp):
    """xs: arrays of outer x counts[t] elements (flattened); y: outer x sum(counts)."""
    xs = [np.ascontiguousarray(x) for x in xs]
    n = len(xs)
    y = np.empty(outer * sum(counts), xs[0].dtype)
    ptrs = (ct.c_void_p * n)(*[x.ctypes.data for x in xs])
    cnt = (ct.c_longlong * n)(*counts)
    sc = (ct.c_float * n)(*scales)
    zp = (ct.c_int * n)(*zps)
    lib().orc_qlinear_concat(n, ptrs, cnt, outer, dt_of(xs[0]), sc, zp, float(y_s), int(y_zp), _p(y))
    return y


def qlinear_mul(kind, a, b, a_s, a_zp, b_s, b_zp, y_s, y_zp, C=0, HW=0, y_nhwc=0):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    full = a if a.size >= b.size else b
    y = np.empty(full.shape, a.dtype)
    N = full.size // (C * HW) if C and HW else 0
    lib().orc_qlinear_mul(kind, _p(a), _p(b), _p(y), y.size, N, C, HW, y_nhwc, dt_of(a),
                          float(a_s), int(a_zp), float(b_s), int(b_zp), float(y_s), int(y_zp))
    return y


def fold_bn(sc, bias, mean, var, eps, q_s, q_zp, dq=None):
    """fold_bn_qdq's (A, B) per channel; dq = (dq_scale, dq_zp) for DQ->BN->Q."""
    C = len(sc)
    f = lambda a: np.ascontiguousarray(a, np.float32)
    sc, bias, mean, var = f(sc), f(bias), f(mean), f(var)
    A = np.empty(C, np.float32)
    B = np.empty(C, np.float32)
    lib().orc_fold_bn(C, _p(sc), _p(bias), _p(mean), _p(var), float(eps), 1 if dq else 0,
                      float(dq[0]) if dq else 0.0, int(dq[1]) if dq else 0, float(q_s), int(q_zp), _p(A), _p(B))
    return A, B


def batchnorm_u8(x, A, B, nhwc=0):
    x = np.ascontiguousarray(x)
    N = x.shape[0]
    C = x.shape[-1] if nhwc else x.shape[1]
    HW = x.size // (N * C)
    y = np.empty(x.shape, np.uint8)
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    lib().orc_batchnorm_u8(_p(x), 1 if x.dtype == np.float32 else 0, _p(y), _p(A), _p(B), N, C, HW, nhwc)
    return y


def conv_integer(x, w, x_zp, w_zp, strides=(1, 1), pads=(0, 0), dilations=(1, 1), group=1, out_hw=None):
    """ConvInteger, 4-D NCHW: int32 y = sum (x - x_zp)(w - w_zp[oc]); w_zp a
    scalar or [OC]; pads = the begin pads; out_hw defaults to the explicit-pad
    extent with the end pads equal to the begin ones."""
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w)
    N, C, iH, iW = x.shape
    OC, _, kH, kW = w.shape
    if out_hw is None:
        out_hw = tuple((d + 2 * p_ - ((k - 1) * dl + 1)) // s + 1
                       for d, p_, k, dl, s in zip((iH, iW), pads, (kH, kW), dilations, strides))
    wzp = np.ascontiguousarray(np.broadcast_to(np.asarray(w_zp, np.int32).reshape(-1), (OC,)), np.int32)
    y = np.empty((N, OC, *out_hw), np.int32)
    lib().orc_conv_integer(_p(x), dt_of(x), _p(w), dt_of(w), int(x_zp), _p(wzp), N, C, iH, iW, OC, kH, kW,
                           strides[0], strides[1], pads[0], pads[1], dilations[0], dilations[1], out_hw[0],
                           out_hw[1], group, _p(y))
    return y


def maxpool_u8_nhwc(x, kH, kW, sH, sW, pH, pW, oH, oW):
    x = np.ascontiguousarray(x, np.uint8)
    N, H, W, Cc = x.shape
    y = np.empty((N, oH, oW, Cc), np.uint8)
    lib().orc_maxpool_u8_nhwc(_p(x), _p(y), N, Cc, H, W, oH, oW, kH, kW, sH, sW, pH, pW)
    return y


# ---- QLinearConv ---------------------------------------------------------------
class Conv:
    """Holds one QLinearConv configuration for the oracle."""

    def __init__(self, N, C, H, W, OC, kH, kW, group=1, stride=(1, 1), dil=(1, 1),
                 pads=(0, 0, 0, 0), x_nhwc=0, y_nhwc=0, post_fn=0, act_dtype=np.uint8,
                 x_scale=0.02, x_zp=128, w_scale=(0.01,), w_zp=(), y_scale=0.05, y_zp=0,
                 bias=None, vnni=1):
        self.w_scale = np.ascontiguousarray(w_scale, np.float32)
        self.w_zp = np.ascontiguousarray(w_zp, np.int8)
        self.bias = None if bias is None else np.ascontiguousarray(bias, np.int32)
        o = lib().orc_conv_out_dim
        oH = o(H, kH, dil[0], stride[0], pads[0], pads[2])
        oW = o(W, kW, dil[1], stride[1], pads[1], pads[3])
        self.p = ConvParams(
            N, C, H, W, OC, kH, kW, group, stride[0], stride[1], dil[0], dil[1],
            pads[0], pads[1], pads[2], pads[3], oH, oW, x_nhwc, y_nhwc, post_fn,
            U8 if act_dtype == np.uint8 else S8, float(x_scale), int(x_zp),
            self.w_scale.ctypes.data_as(ct.POINTER(ct.c_float)), self.w_scale.size,
            self.w_zp.ctypes.data_as(ct.POINTER(ct.c_int8)) if self.w_zp.size else None,
            self.w_zp.size, float(y_scale), int(y_zp),
            self.bias.ctypes.data_as(ct.POINTER(ct.c_int32)) if self.bias is not None else None,
            vnni)
        self.act_dtype = act_dtype

    @property
    def out_shape(self):
        p = self.p
        return (p.N, p.oH, p.oW, p.OC) if p.y_nhwc else (p.N, p.OC, p.oH, p.oW)

    def dispatch(self):
        return lib().orc_conv_dispatch(ct.byref(self.p))

    def acc(self, x, w):
        p = self.p
        x = np.ascontiguousarray(x)
        w = np.ascontiguousarray(w, np.int8)
        a = np.empty((p.N, p.OC, p.oH, p.oW), np.int32)
        lib().orc_conv_acc(ct.byref(p), _p(x), _p(w), _p(a))
        return a

    def run(self, x, w):
        x = np.ascontiguousarray(x)
        w = np.ascontiguousarray(w, np.int8)
        y = np.empty(self.out_shape, self.act_dtype)
        br = lib().orc_qlinear_conv(ct.byref(self.p), _p(x), _p(w), _p(y))
        return y, br

    def from_acc(self, acc):
        y = np.empty(self.out_shape, self.act_dtype)
        br = lib().orc_qlinear_conv_from_acc(ct.byref(self.p), _p(np.ascontiguousarray(acc)), _p(y))
        return y, br


class Conv1d:
    """QLinearConv on 3-D tensors: x [N][C][W], w [OC][C/group][kW]; the
    reference's exec_typed path (RQ-S)."""

    def __init__(self, N, C, W, OC, kW, group=1, stride=1, dil=1, pads=(0, 0), act_dtype=np.uint8,
                 x_scale=0.02, x_zp=128, w_scale=(0.01,), w_zp=(), y_scale=0.05, y_zp=0, bias=None):
        self.c = Conv(N, C, 1, W, OC, 1, kW, group=group, stride=(1, stride), dil=(1, dil),
                      pads=(0, pads[0], 0, pads[1]), act_dtype=act_dtype, x_scale=x_scale, x_zp=x_zp,
                      w_scale=w_scale, w_zp=w_zp, y_scale=y_scale, y_zp=y_zp, bias=bias)
        self.act_dtype = act_dtype

    @property
    def out_shape(self):
        p = self.c.p
        return (p.N, p.OC, p.oW)

    def run(self, x, w):
        x = np.ascontiguousarray(x)
        w = np.ascontiguousarray(w, np.int8)
        y = np.empty(self.out_shape, self.act_dtype)
        br = lib().orc_qlinear_conv1d(ct.byref(self.c.p), _p(x), _p(w), _p(y))
        return y, br


def set_vnni(on: bool) -> bool:
    """Route conv / matmul accumulators through the AVX-512 VNNI
    restatement (nnr_vnni.c); returns whether it is active (needs AVX-512
    VNNI on this host)."""
    lib().orc_set_vnni(1 if on else 0)
    return bool(lib().orc_get_vnni())


def vnni_available() -> bool:
    return bool(lib().orc_vnni_available())

