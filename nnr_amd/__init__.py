"""nnr_amd -- MI355X (gfx950) backend for NNR's int8 QDQ compute path.

The product is the C ABI in include/nnr_hip.h (nnr_amd/lib/libnnr_hip.so,
HIP kernels in nnr_amd/csrc) and the C++ operator layer in nnr_amd/host that
mirrors NNR's operator_t / registry_t interface. This Python module is a thin
convenience view of the same C ABI for tests and benchmarks: device memory is
torch tensors, every call goes straight to the HIP library, and a missing
library raises instead of falling back to anything.
"""
from __future__ import annotations

import ctypes as ct

import numpy as np

from ._lib import (BRANCH_NAMES, F16, F32, I32, NNRH_ERR_UNSUPPORTED, S8, U8, NnrHipError,  # noqa: F401
                   QConvDesc,
                   QMatMulDesc, check, cur_stream, lib, ptr)

__all__ = ["QLinearConv", "QLinearMatMul", "MatMulIntegerScaled", "MatMulInteger", "quantize_linear",
           "dequantize_linear", "dynamic_quantize_linear", "qlinear_add", "maxpool_u8_nhwc",
           "conv_dispatch", "NnrHipError", "lib"]


def _dt(np_dtype) -> int:
    return U8 if np.dtype(np_dtype) == np.uint8 else S8


def _conv_desc(N, C, H, W, w, *, group=1, stride=(1, 1), dil=(1, 1), pads=(0, 0, 0, 0),
               x_nhwc=0, y_nhwc=0, post_fn=0, act_dtype=np.uint8, x_scale=0.02, x_zp=128,
               w_scale=(0.01,), w_zp=(), y_scale=0.05, y_zp=0, bias=None, spatial_dims=2):
    w = np.ascontiguousarray(w, np.int8)
    if spatial_dims == 1 and w.ndim == 3:
        w = w[:, :, None, :]
    OC, _, kH, kW = w.shape
    keep = {
        "w": w,
        "w_scale": np.ascontiguousarray(w_scale, np.float32).reshape(-1),
        "w_zp": np.ascontiguousarray(np.asarray(w_zp).astype(np.int64).astype(np.uint8).view(np.int8)
                                     if len(np.atleast_1d(w_zp)) else np.zeros(0, np.int8)),
        "bias": None if bias is None else np.ascontiguousarray(bias, np.int32),
    }
    ek_h, ek_w = (kH - 1) * dil[0] + 1, (kW - 1) * dil[1] + 1
    oH = int(np.floor((H + pads[0] + pads[2] - ek_h) / stride[0] + 1))
    oW = int(np.floor((W + pads[1] + pads[3] - ek_w) / stride[1] + 1))
    P = ct.POINTER
    d = QConvDesc(N, C, H, W, OC, kH, kW, group, stride[0], stride[1], dil[0], dil[1],
                  pads[0], pads[1], pads[2], pads[3], oH, oW, int(x_nhwc), int(y_nhwc),
                  int(post_fn), _dt(act_dtype), float(x_scale), int(x_zp),
                  keep["w_scale"].ctypes.data_as(P(ct.c_float)), keep["w_scale"].size,
                  keep["w_zp"].ctypes.data_as(P(ct.c_int8)) if keep["w_zp"].size else None,
                  keep["w_zp"].size, float(y_scale), int(y_zp),
                  keep["w"].ctypes.data_as(P(ct.c_int8)),
                  keep["bias"].ctypes.data_as(P(ct.c_int32)) if keep["bias"] is not None else None,
                  int(spatial_dims))
    return d, keep


def conv_dispatch(N, C, H, W, w, **kw) -> int:
    """Kernel branch NNR's QLinearConv would take (pure host computation)."""
    d, _keep = _conv_desc(N, C, H, W, w, **kw)
    br = ct.c_int()
    check(lib().nnrh_qconv_dispatch(ct.byref(d), ct.byref(br)))
    return br.value


class QLinearConv:
    """QLinearConv on the GPU: create packs weights, __call__ launches."""

    def __init__(self, N, C, H, W, w, **kw):
        self.desc, keep = _conv_desc(N, C, H, W, w, **kw)
        self.act_dtype = np.dtype(kw.get("act_dtype", np.uint8))
        h = ct.c_void_p()
        check(lib().nnrh_qconv_create(ct.byref(h), ct.byref(self.desc)))
        self.h = h
        br = ct.c_int()
        check(lib().nnrh_qconv_branch(h, ct.byref(br)))
        self.branch = br.value
        d = self.desc
        self.out_shape = (d.N, d.oH, d.oW, d.OC) if d.y_nhwc else (d.N, d.OC, d.oH, d.oW)
        self.in_shape = (d.N, d.H, d.W, d.C) if d.x_nhwc else (d.N, d.C, d.H, d.W)
        if d.spatial_dims == 1:   # 3-D tensors [N][C][W]
            self.out_shape, self.in_shape = (d.N, d.OC, d.oW), (d.N, d.C, d.W)

    def __call__(self, x, y=None, stream=None):
        import torch
        if tuple(x.shape) != self.in_shape or not x.is_contiguous():
            raise ValueError(f"x shape {tuple(x.shape)} != {self.in_shape} or not contiguous")
        if y is None:
            y = torch.empty(self.out_shape, dtype=torch.uint8 if self.act_dtype == np.uint8
                            else torch.int8, device=x.device)
        check(lib().nnrh_qconv_run(self.h, ptr(x), ptr(y),
                                   cur_stream() if stream is None else stream))
        return y

    def fuse_add(self, conv_is_a, a_scale, a_zp, b_scale, b_zp, y_scale, y_zp):
        """Fuse a same-shape QLinearAdd of this conv's output into its kernel.
        Returns False (handle unchanged) when this conv's kernel cannot."""
        from ._lib import QAddFuseDesc
        d = QAddFuseDesc(int(bool(conv_is_a)), a_scale, a_zp, b_scale, b_zp, y_scale, y_zp)
        rc = lib().nnrh_qconv_fuse_add(self.h, ct.byref(d))
        if rc == 0:
            return True
        if rc == NNRH_ERR_UNSUPPORTED:
            return False
        check(rc)

    def run_add(self, x, other, y=None, stream=None):
        """Conv then QLinearAdd with `other` (same layout and shape as y)."""
        import torch
        if tuple(x.shape) != self.in_shape or not x.is_contiguous():
            raise ValueError(f"x shape {tuple(x.shape)} != {self.in_shape} or not contiguous")
        if tuple(other.shape) != self.out_shape or not other.is_contiguous():
            raise ValueError(f"other shape {tuple(other.shape)} != {self.out_shape}")
        if y is None:
            y = torch.empty(self.out_shape, dtype=other.dtype, device=x.device)
        check(lib().nnrh_qconv_run_add(self.h, ptr(x), ptr(other), ptr(y),
                                       cur_stream() if stream is None else stream))
        return y

    def fuse_quantize(self, scale, zero_point):
        """Run the QuantizeLinear producing this first-layer conv's input in the
        conv's layout kernel; afterwards call run_f32 with the fp32 input."""
        rc = lib().nnrh_qconv_fuse_quantize(self.h, float(scale), int(zero_point))
        if rc == NNRH_ERR_UNSUPPORTED:
            return False
        check(rc)
        return True

    def fuse_maxpool(self, k=(3, 3), s=(2, 2), pads=(1, 1, 1, 1)):
        """Run the MaxPool reading this first-layer conv's uint8 NHWC output in
        the conv's kernel; afterwards the output is the pooled tensor.
        Returns False (handle unchanged) when the kernel cannot."""
        rc = lib().nnrh_qconv_fuse_maxpool(self.h, int(k[0]), int(k[1]), int(s[0]), int(s[1]),
                                           *[int(p) for p in pads])
        if rc == NNRH_ERR_UNSUPPORTED:
            return False
        check(rc)
        d = self.desc
        self.out_shape = (d.N, (d.oH - 1) // 2 + 1, (d.oW - 1) // 2 + 1, d.OC)
        return True

    def run_f32(self, x, y=None, stream=None):
        import torch
        if tuple(x.shape) != self.in_shape or not x.is_contiguous() or x.dtype != torch.float32:
            raise ValueError(f"x must be contiguous float32 of shape {self.in_shape}")
        if y is None:
            y = torch.empty(self.out_shape, dtype=torch.uint8, device=x.device)
        check(lib().nnrh_qconv_run_f32(self.h, ptr(x), ptr(y), cur_stream() if stream is None else stream))
        return y

    def __del__(self):
        try:
            if getattr(self, "h", None):
                lib().nnrh_qconv_destroy(self.h)
                self.h = None
        except Exception:
            pass


class QLinearMatMul:
    """QLinearMatMul with constant B (prepacked at construction)."""

    def __init__(self, b, a_scale, a_zp, b_scale, b_zp, y_scale, y_zp, *, m, a_dtype=np.uint8,
                 y_dtype=np.uint8, scale_dtype=np.float32):
        b = np.ascontiguousarray(b)
        k, n = b.shape
        sd = np.float16 if scale_dtype == np.float16 else np.float32
        self._keep = dict(
            b=b, a_s=np.array([a_scale], sd), a_z=np.array([a_zp], a_dtype),
            b_s=np.array([b_scale], sd), b_z=np.array([b_zp], b.dtype),
            y_s=np.array([y_scale], sd), y_z=np.array([y_zp], y_dtype))
        kp = self._keep
        self.desc = QMatMulDesc(m, n, k, _dt(a_dtype), _dt(b.dtype), _dt(y_dtype),
                                F16 if sd == np.float16 else F32,
                                kp["a_s"].ctypes.data, kp["a_z"].ctypes.data,
                                kp["b_s"].ctypes.data, kp["b_z"].ctypes.data,
                                kp["y_s"].ctypes.data, kp["y_z"].ctypes.data, b.ctypes.data)
        h = ct.c_void_p()
        check(lib().nnrh_qmatmul_create(ct.byref(h), ct.byref(self.desc)))
        self.h = h
        self.m, self.n, self.k = m, n, k
        self.y_dtype = np.dtype(y_dtype)
        self._f32 = False

    def fuse_dq_bias(self, dq_scale, dq_zp, bias=None):
        """Then DequantizeLinear(y_zp, dq_scale) and + bias[n]: float32 output."""
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self._keep["dq_bias"] = b
        check(lib().nnrh_qmatmul_fuse_dq_bias(
            self.h, float(dq_scale), int(dq_zp),
            None if b is None else b.ctypes.data_as(ct.POINTER(ct.c_float))))
        self._f32 = True

    def fuse_gelu(self):
        check(lib().nnrh_qmatmul_fuse_gelu(self.h))

    def minmax_count(self, batch=1):
        n = ct.c_int()
        check(lib().nnrh_qmatmul_minmax_count(self.h, batch, ct.byref(n)))
        return n.value

    def set_minmax_out(self, parts):
        """parts: float32 device tensor of (min, max) pairs, or None."""
        check(lib().nnrh_qmatmul_set_minmax_out(self.h, ptr(parts),
                                                0 if parts is None else parts.numel() // 2))
        self._keep["parts"] = parts

    def set_codes_out(self, on=True):
        """After fuse_dq_bias (+ fuse_gelu) and set_minmax_out: runs write the
        uint8 QLinearMatMul bytes and the chain values' (min, max) pairs
        instead of the float32 values; dynamic_quantize_codes then gives the
        DynamicQuantizeLinear of those values."""
        check(lib().nnrh_qmatmul_set_codes_out(self.h, 1 if on else 0))
        self._codes = bool(on)

    def dq_params(self):
        """(zero point, scale, device bias pointer) of the fused chain, for a
        reader of its bytes (dq_codes)."""
        zp, sc, b = ct.c_int(), ct.c_float(), ct.c_void_p()
        check(lib().nnrh_qmatmul_dq_params(self.h, ct.byref(zp), ct.byref(sc), ct.byref(b)))
        return zp.value, sc.value, b.value

    def dynamic_quantize_codes(self, codes, stream=None):
        """(y, y_scale, y_zp) of DynamicQuantizeLinear over the chain values
        of a codes-mode run's output `codes` (its (min, max) pairs must be
        the last ones written)."""
        import torch
        batch = codes.numel() // (self.m * self.n)
        y = torch.empty(tuple(codes.shape), dtype=torch.uint8, device=codes.device)
        ys = torch.empty(1, dtype=torch.float32, device=codes.device)
        yz = torch.empty(1, dtype=torch.uint8, device=codes.device)
        check(lib().nnrh_qmatmul_dynamic_quantize_codes(self.h, ptr(codes), batch, ptr(y), ptr(ys), ptr(yz),
                                                        cur_stream() if stream is None else stream))
        return y, ys, yz

    def __call__(self, a, y=None, a_scale_dev=None, a_zp_dev=None, stream=None):
        import torch
        if a.shape[-1] != self.k or a.shape[-2] != self.m:
            raise ValueError("a shape mismatch")
        batch = int(np.prod(a.shape[:-2])) if a.dim() > 2 else 1
        if y is None:
            dt = torch.float32 if self._f32 and not getattr(self, "_codes", False) else (
                torch.uint8 if self.y_dtype == np.uint8 else torch.int8)
            y = torch.empty(tuple(a.shape[:-1]) + (self.n,), dtype=dt, device=a.device)
        check(lib().nnrh_qmatmul_run(self.h, ptr(a), self.m * self.k if batch > 1 else 0, ptr(y),
                                     batch, ptr(a_scale_dev), ptr(a_zp_dev),
                                     cur_stream() if stream is None else stream))
        return y

    def __del__(self):
        try:
            if getattr(self, "h", None):
                lib().nnrh_qmatmul_destroy(self.h)
                self.h = None
        except Exception:
            pass


class MatMulIntegerScaled(QLinearMatMul):
    """MatMulInteger with constant B followed by Cast -> Mul(fl(a_scale *
    w_scale[n])) -> Add(bias[n]) in one kernel (float32 output); runs like a
    fused-dequantize QLinearMatMul (Gelu, min / max pairs, groups)."""

    def __init__(self, b, w_scale, bias=None, *, m, a_scale=1.0, a_zp=0, a_dtype=np.uint8, b_zp=0):
        b = np.ascontiguousarray(b)
        k, n = b.shape
        ws = np.ascontiguousarray(w_scale, np.float32)
        bi = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self._keep = dict(b=b, ws=ws, bias=bi)
        from ._lib import MmiScaledDesc
        self.desc = MmiScaledDesc(m, n, k, _dt(a_dtype), _dt(b.dtype), b.ctypes.data, int(a_zp), int(b_zp),
                                  float(a_scale), ws.ctypes.data, None if bi is None else bi.ctypes.data)
        h = ct.c_void_p()
        check(lib().nnrh_matmul_integer_scaled_create(ct.byref(h), ct.byref(self.desc)))
        self.h = h
        self.m, self.n, self.k = m, n, k
        self.y_dtype = np.dtype(np.float32)
        self._f32 = True


class QLinearMatMulGroup:
    """2..4 fused-dequantize QLinearMatMuls reading the same A, one launch."""

    def __init__(self, members):
        self._members = list(members)   # keep the member handles alive
        arr = (ct.c_void_p * len(members))(*[m.h.value for m in members])
        h = ct.c_void_p()
        check(lib().nnrh_qmatmul_group_create(ct.byref(h), arr, len(members)))
        self.h = h
        self.n = members[0].n

    def set_codes_out(self, on=True):
        """The launch writes the members' uint8 QLinearMatMul bytes."""
        check(lib().nnrh_qmatmul_group_set_codes_out(self.h, 1 if on else 0))

    def __call__(self, a, ys, a_scale_dev=None, a_zp_dev=None, stream=None):
        rows = a.numel() // a.shape[-1]
        arr = (ct.c_void_p * len(ys))(*[y.data_ptr() for y in ys])
        check(lib().nnrh_qmatmul_group_run(self.h, ptr(a), rows, arr, ptr(a_scale_dev), ptr(a_zp_dev),
                                           cur_stream() if stream is None else stream))
        return ys

    def __del__(self):
        try:
            if getattr(self, "h", None):
                lib().nnrh_qmatmul_group_destroy(self.h)
                self.h = None
        except Exception:
            pass


class MatMulInteger:
    def __init__(self, m, n, k, a_dtype=np.uint8, b_dtype=np.int8, max_batch=1):
        h = ct.c_void_p()
        check(lib().nnrh_matmul_integer_create(ct.byref(h), m, n, k, _dt(a_dtype), _dt(b_dtype),
                                               max_batch))
        self.h, self.m, self.n, self.k = h, m, n, k

    def __call__(self, a, b, a_zp=0, b_zp=0, batch=1, a_bstride=None, b_bstride=None, y=None,
                 stream=None):
        import torch
        if y is None:
            y = torch.empty((batch, self.m, self.n) if batch > 1 else (self.m, self.n),
                            dtype=torch.int32, device=a.device)
        ab = (self.m * self.k if batch > 1 else 0) if a_bstride is None else a_bstride
        bb = (self.k * self.n if batch > 1 and b.dim() > 2 else 0) if b_bstride is None else b_bstride
        check(lib().nnrh_matmul_integer_run(self.h, ptr(a), ab, ptr(b), bb, int(a_zp), int(b_zp),
                                            ptr(y), batch,
                                            cur_stream() if stream is None else stream))
        return y

    def __del__(self):
        try:
            if getattr(self, "h", None):
                lib().nnrh_matmul_integer_destroy(self.h)
                self.h = None
        except Exception:
            pass


def quantize_linear(x, scale, zp, dtype=np.uint8, y=None):
    import torch
    if y is None:
        y = torch.empty(x.shape, dtype=torch.uint8 if np.dtype(dtype) == np.uint8 else torch.int8,
                        device=x.device)
    check(lib().nnrh_quantize_linear(ptr(x), x.numel(), float(scale), int(zp), _dt(dtype), ptr(y),
                                     cur_stream()))
    return y


def dequantize_linear(x, scale, zp, y=None):
    import torch
    if y is None:
        y = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    dt = {torch.uint8: U8, torch.int8: S8, torch.int32: I32}[x.dtype]
    check(lib().nnrh_dequantize_linear(ptr(x), dt, x.numel(), float(scale), int(zp), ptr(y),
                                       cur_stream()))
    return y


_dq_ws = {}


def dynamic_quantize_linear(x):
    import torch
    dev = x.device
    if dev not in _dq_ws:
        _dq_ws[dev] = torch.empty(int(lib().nnrh_dynamic_quantize_workspace()), dtype=torch.uint8,
                                  device=dev)
    y = torch.empty(x.shape, dtype=torch.uint8, device=dev)
    s = torch.empty(1, dtype=torch.float32, device=dev)
    z = torch.empty(1, dtype=torch.uint8, device=dev)
    check(lib().nnrh_dynamic_quantize_linear(ptr(x), x.numel(), ptr(y), ptr(s), ptr(z),
                                             ptr(_dq_ws[dev]), cur_stream()))
    return y, s, z


def dynamic_quantize_linear_parts(x, parts):
    """DynamicQuantizeLinear of x from producer-written (min, max) pairs."""
    import torch
    dev = x.device
    y = torch.empty(x.shape, dtype=torch.uint8, device=dev)
    s = torch.empty(1, dtype=torch.float32, device=dev)
    z = torch.empty(1, dtype=torch.uint8, device=dev)
    check(lib().nnrh_dynamic_quantize_linear_parts(ptr(x), x.numel(), ptr(parts), parts.numel() // 2,
                                                   ptr(y), ptr(s), ptr(z), cur_stream()))
    return y, s, z


def layernorm(x, gamma, beta=None, eps=1e-5, r=None, parts=None):
    """LayerNormalization over the last axis of x (of x + r when r is given);
    parts: optional float32 device tensor receiving one (min, max) per group
    of 4 rows."""
    import torch
    D = x.shape[-1]
    y = torch.empty_like(x)
    check(lib().nnrh_add_layernorm_f32(ptr(x), ptr(r), ptr(gamma), ptr(beta), ptr(y), x.numel() // D, D,
                                       float(eps), ptr(parts), cur_stream()))
    return y


def dq_codes(codes, op):
    """nnrh_dq_codes for the bytes `codes` of fused QLinearMatMul `op`'s chain."""
    from ._lib import DqCodes
    zp, sc, b = op.dq_params()
    return DqCodes(codes.data_ptr(), zp, sc, b)


def layernorm_codes(xc, gamma, beta=None, eps=1e-5, r=None, parts=None):
    """layernorm with x given as chain bytes: xc = (uint8 device tensor, the
    QLinearMatMul whose chain they belong to)."""
    import torch
    codes, op = xc
    D = codes.shape[-1]
    y = torch.empty(tuple(codes.shape), dtype=torch.float32, device=codes.device)
    d = dq_codes(codes, op)
    check(lib().nnrh_add_layernorm_codes_f32(ct.byref(d), ptr(r), ptr(gamma), ptr(beta), ptr(y), codes.numel() // D,
                                             D, float(eps), ptr(parts), cur_stream()))
    return y


def multihead_attention_codes(qc, kc, vc, num_heads, scale, parts=None):
    """The fused attention on q, k, v given as chain bytes ((tensor, op)
    pairs); y fp32 of the same [B][S][hidden] shape."""
    import torch
    codes = qc[0]
    B, S, Hd = codes.shape
    y = torch.empty((B, S, Hd), dtype=torch.float32, device=codes.device)
    dq = [dq_codes(c, o) for c, o in (qc, kc, vc)]
    check(lib().nnrh_multihead_attention_codes_f32(ct.byref(dq[0]), ct.byref(dq[1]), ct.byref(dq[2]), ptr(y), B, S,
                                                   Hd, num_heads, float(scale), ptr(parts), cur_stream()))
    return y


def qlinear_add(kind, a, b, a_s, a_zp, b_s, b_zp, y_s, y_zp, C=0, HW=0, y_nhwc=0, y=None):
    import torch
    full = a if a.numel() >= b.numel() else b
    if y is None:
        y = torch.empty(full.shape, dtype=full.dtype, device=full.device)
    dt = U8 if a.dtype == torch.uint8 else S8
    check(lib().nnrh_qlinear_add(kind, ptr(a), ptr(b), ptr(y), y.numel(), C, HW, y_nhwc, dt,
                                 float(a_s), int(a_zp), float(b_s), int(b_zp), float(y_s),
                                 int(y_zp), cur_stream()))
    return y


def qlinear_mul(kind, a, b, a_s, a_zp, b_s, b_zp, y_s, y_zp, C=0, HW=0, y_nhwc=0, y=None):
    import torch
    full = a if a.numel() >= b.numel() else b
    if y is None:
        y = torch.empty(full.shape, dtype=full.dtype, device=full.device)
    dt = U8 if a.dtype == torch.uint8 else S8
    check(lib().nnrh_qlinear_mul(kind, ptr(a), ptr(b), ptr(y), y.numel(), C, HW, y_nhwc, dt,
                                 float(a_s), int(a_zp), float(b_s), int(b_zp), float(y_s),
                                 int(y_zp), cur_stream()))
    return y


def qlinear_global_avgpool(x, x_s, x_zp, y_s, y_zp, nhwc=0):
    """x [N, C, *spatial] (or [N, *spatial, C] with nhwc) -> y [N, C]."""
    import torch
    N = x.shape[0]
    C = x.shape[-1] if nhwc else x.shape[1]
    sp = x.numel() // (N * C)
    y = torch.empty((N, C), dtype=x.dtype, device=x.device)
    dt = U8 if x.dtype == torch.uint8 else S8
    check(lib().nnrh_qlinear_global_avgpool(ptr(x), ptr(y), N, C, sp, nhwc, dt, float(x_s), int(x_zp),
                                            float(y_s), int(y_zp), cur_stream()))
    return y


def qlinear_avgpool(x, k, stride, pads, oH, oW, x_s, x_zp, y_s, y_zp, nhwc=0):
    import torch
    if nhwc:
        N, H, W, Cc = x.shape
        y = torch.empty((N, oH, oW, Cc), dtype=x.dtype, device=x.device)
    else:
        N, Cc, H, W = x.shape
        y = torch.empty((N, Cc, oH, oW), dtype=x.dtype, device=x.device)
    dt = U8 if x.dtype == torch.uint8 else S8
    check(lib().nnrh_qlinear_avgpool(ptr(x), ptr(y), N, Cc, H, W, oH, oW, k[0], k[1], stride[0], stride[1],
                                     pads[0], pads[1], nhwc, dt, float(x_s), int(x_zp), float(y_s), int(y_zp),
                                     cur_stream()))
    return y


def qlinear_concat(xs, counts, outer, scales, zps, y_s, y_zp):
    """xs: device tensors of outer x counts[t] elements; y: outer x sum(counts)."""
    import torch
    row = sum(counts)
    y = torch.empty(outer * row, dtype=xs[0].dtype, device=xs[0].device)
    dt = U8 if xs[0].dtype == torch.uint8 else S8
    n = len(xs)
    P = (ct.c_void_p * n)(*[ptr(x) for x in xs])
    check(lib().nnrh_qlinear_concat(n, P, (ct.c_longlong * n)(*counts), (ct.c_float * n)(*map(float, scales)),
                                    (ct.c_int * n)(*map(int, zps)), outer, dt, float(y_s), int(y_zp), ptr(y),
                                    cur_stream()))
    return y


def conv_integer(x, w, x_zp, w_zp, strides=(1, 1), pads=(0, 0), dilations=(1, 1), group=1, out_hw=None):
    """ConvInteger on the device (nnrh_conv_integer_*): x, w device uint8 /
    int8 NCHW tensors; w_zp a scalar or a sequence of OC values; int32 y."""
    import numpy as np
    import torch
    N, C, iH, iW = x.shape
    OC, _, kH, kW = w.shape
    if out_hw is None:
        out_hw = tuple((d + 2 * p_ - ((k - 1) * dl + 1)) // s + 1
                       for d, p_, k, dl, s in zip((iH, iW), pads, (kH, kW), dilations, strides))
    dt = lambda t: U8 if t.dtype == torch.uint8 else S8
    h = ct.c_void_p()
    check(lib().nnrh_conv_integer_create(ct.byref(h), N, C, iH, iW, OC, kH, kW, strides[0], strides[1], pads[0],
                                         pads[1], dilations[0], dilations[1], out_hw[0], out_hw[1], group, dt(x), dt(w)))
    y = torch.empty((N, OC, *out_hw), dtype=torch.int32, device=x.device)
    wz = np.asarray(w_zp, np.int32).reshape(-1)
    wz_dev = torch.from_numpy(wz).to(x.device) if wz.size > 1 else None
    try:
        check(lib().nnrh_conv_integer_run(h, ptr(x), ptr(w), int(x_zp), int(wz[0]) if wz_dev is None else 0,
                                          ptr(wz_dev) if wz_dev is not None else None, ptr(y), cur_stream()))
        check(lib().nnrh_stream_synchronize(cur_stream()))
    finally:
        lib().nnrh_conv_integer_destroy(h)
    return y


def batchnorm_u8(x, a, b, nhwc=0):
    """Folded BatchNormalization: y = uint8(A[c] * x + B[c]). x: device uint8 or
    float32 [N, C, ...] (with nhwc, [N, H, W, C]); a, b: device float32 [C]."""
    import torch
    N = x.shape[0]
    C = x.shape[-1] if nhwc else x.shape[1]
    HW = x.numel() // (N * C)
    y = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    check(lib().nnrh_batchnorm_u8(ptr(x), 1 if x.dtype == torch.float32 else 0, ptr(y), ptr(a), ptr(b), N, C, HW,
                                  nhwc, cur_stream()))
    return y


def maxpool_u8_nhwc(x, kH, kW, sH, sW, pH, pW, oH, oW):
    import torch
    N, H, W, C = x.shape
    y = torch.empty((N, oH, oW, C), dtype=torch.uint8, device=x.device)
    check(lib().nnrh_maxpool_u8_nhwc(ptr(x), ptr(y), N, C, H, W, oH, oW, kH, kW, sH, sW, pH, pW,
                                     cur_stream()))
    return y
