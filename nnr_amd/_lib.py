"""ctypes binding of the C ABI in include/nnr_hip.h.

This is the Python view of the same boundary the C++ host operators use. It
loads nnr_amd/lib/libnnr_hip.so and fails loudly when the library is missing:
there is no CPU fallback anywhere in the product path.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libnnr_hip.so")

NNRH_OK, NNRH_ERR_INVALID, NNRH_ERR_UNSUPPORTED, NNRH_ERR_HIP, NNRH_ERR_NOMEM = range(5)
U8, S8, I32, F32, F16 = range(5)
BRANCH_NAMES = {1: "DW", 2: "FIRST", 3: "DIRECT", 4: "PACKED", 5: "NR16",
                6: "IM2COL_S1", 7: "IM2COL", 8: "FLOAT", 9: "TYPED"}

# every symbol the header declares (checked by the CPU test suite)
EXPORTS = [
    "nnrh_last_error", "nnrh_version", "nnrh_device_count", "nnrh_set_device",
    "nnrh_malloc", "nnrh_free", "nnrh_memcpy", "nnrh_fill_u8", "nnrh_stream_create",
    "nnrh_stream_destroy", "nnrh_stream_synchronize", "nnrh_device_synchronize",
    "nnrh_event_create", "nnrh_event_destroy", "nnrh_event_record", "nnrh_event_elapsed_ms",
    "nnrh_stream_wait_event",
    "nnrh_profile_enable", "nnrh_profile_reset", "nnrh_profile_count", "nnrh_profile_get",
    "nnrh_profile_enabled", "nnrh_graph_begin_capture", "nnrh_graph_end_capture", "nnrh_graph_launch",
    "nnrh_graph_destroy",
    "nnrh_qconv_dispatch", "nnrh_qconv_create", "nnrh_qconv_branch", "nnrh_qconv_run",
    "nnrh_qconv_destroy", "nnrh_qconv_fuse_add", "nnrh_qconv_run_add",
    "nnrh_qconv_fuse_quantize", "nnrh_qconv_run_f32", "nnrh_qconv_fuse_maxpool", "nnrh_global_avgpool_dequant",
    "nnrh_multihead_attention_workspace", "nnrh_multihead_attention_f32", "nnrh_multihead_attention_minmax_count", "nnrh_qmatmul_create", "nnrh_qmatmul_run", "nnrh_qmatmul_destroy",
    "nnrh_qmatmul_fuse_dq_bias", "nnrh_qmatmul_fuse_gelu", "nnrh_qmatmul_minmax_count",
    "nnrh_qmatmul_set_minmax_out", "nnrh_qmatmul_set_codes_out", "nnrh_qmatmul_dynamic_quantize_codes",
    "nnrh_qmatmul_dq_params", "nnrh_qmatmul_group_set_codes_out", "nnrh_add_layernorm_codes_f32",
    "nnrh_multihead_attention_codes_f32",
    "nnrh_dynamic_quantize_linear_parts", "nnrh_add_layernorm_f32",
    "nnrh_qmatmul_group_create", "nnrh_qmatmul_group_run", "nnrh_qmatmul_group_destroy",
    "nnrh_qlinear_mul", "nnrh_qlinear_global_avgpool", "nnrh_qlinear_avgpool", "nnrh_qlinear_concat_part",
    "nnrh_batchnorm_u8", "nnrh_batchnorm_f32", "nnrh_qlinear_concat",
    "nnrh_conv_integer_create", "nnrh_conv_integer_run", "nnrh_conv_integer_destroy",
    "nnrh_matmul_integer_create", "nnrh_matmul_integer_run", "nnrh_matmul_integer_destroy",
    "nnrh_matmul_integer_scaled_create", "nnrh_matmul_integer_run_dev_zp", "nnrh_cast_to_f32",
    "nnrh_quantize_linear", "nnrh_dequantize_linear", "nnrh_dynamic_quantize_workspace",
    "nnrh_dynamic_quantize_linear", "nnrh_dynamic_quantize_linear_noalloc", "nnrh_qlinear_add", "nnrh_maxpool_u8_nhwc",
    "nnrh_nchw_to_nhwc_u8", "nnrh_global_avgpool_f32", "nnrh_gemm_f32", "nnrh_clip_f32",
    "nnrh_gemm_f32_batched", "nnrh_binary_f32", "nnrh_softmax_f32", "nnrh_layernorm_f32",
    "nnrh_gelu_f32", "nnrh_hardswish_f32", "nnrh_transpose_f32",
]


class NnrHipError(RuntimeError):
    def __init__(self, rc: int, msg: str):
        super().__init__(f"nnrh error {rc}: {msg}")
        self.rc = rc


class QAddFuseDesc(C.Structure):
    _fields_ = [("conv_is_a", C.c_int), ("a_scale", C.c_float), ("a_zp", C.c_int),
                ("b_scale", C.c_float), ("b_zp", C.c_int), ("y_scale", C.c_float),
                ("y_zp", C.c_int)]


class QConvDesc(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "N", "C", "H", "W", "OC", "kH", "kW", "group", "sH", "sW", "dH", "dW",
        "pad_t", "pad_l", "pad_b", "pad_r", "oH", "oW", "x_nhwc", "y_nhwc",
        "post_fn", "act_dtype")] + [
        ("x_scale", C.c_float), ("x_zp", C.c_int),
        ("w_scale_host", C.POINTER(C.c_float)), ("w_scale_count", C.c_int),
        ("w_zp_host", C.POINTER(C.c_int8)), ("w_zp_count", C.c_int),
        ("y_scale", C.c_float), ("y_zp", C.c_int),
        ("w_host", C.POINTER(C.c_int8)), ("bias_host", C.POINTER(C.c_int32)),
        ("spatial_dims", C.c_int),
    ]


class QMatMulDesc(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("m", "n", "k", "a_dtype", "b_dtype", "y_dtype",
                                        "scale_dtype")] + [
        (n, C.c_void_p) for n in ("a_scale_host", "a_zp_host", "b_scale_host", "b_zp_host",
                                  "y_scale_host", "y_zp_host", "b_host")]


class MmiScaledDesc(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("m", "n", "k", "a_dtype", "b_dtype")] + [
        ("b_host", C.c_void_p), ("a_zp", C.c_int), ("b_zp", C.c_int), ("a_scale", C.c_float),
        ("w_scale_host", C.c_void_p), ("bias_host", C.c_void_p)]


class DqCodes(C.Structure):
    _fields_ = [("codes_dev", C.c_void_p), ("zp", C.c_int), ("scale", C.c_float), ("bias_dev", C.c_void_p)]


_lib = None


def lib():
    """Load the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: run __graft_entry__.build() "
                          "(hipcc --offload-arch=gfx950) first")
    L = C.CDLL(LIB_PATH)
    vp, i, sz, f, ll = C.c_void_p, C.c_int, C.c_size_t, C.c_float, C.c_longlong
    P = C.POINTER
    sig = {
        "nnrh_last_error": (C.c_char_p, []),
        "nnrh_version": (C.c_char_p, []),
        "nnrh_device_count": (i, [P(i)]),
        "nnrh_set_device": (i, [i]),
        "nnrh_malloc": (i, [P(vp), sz]),
        "nnrh_free": (i, [vp]),
        "nnrh_memcpy": (i, [vp, vp, sz, i, vp]),
        "nnrh_fill_u8": (i, [vp, C.c_uint8, sz, vp]),
        "nnrh_stream_create": (i, [P(vp)]),
        "nnrh_stream_destroy": (i, [vp]),
        "nnrh_stream_synchronize": (i, [vp]),
        "nnrh_device_synchronize": (i, []),
        "nnrh_event_create": (i, [P(vp)]),
        "nnrh_event_destroy": (i, [vp]),
        "nnrh_event_record": (i, [vp, vp]),
        "nnrh_stream_wait_event": (i, [vp, vp]),
        "nnrh_event_elapsed_ms": (i, [P(f), vp, vp]),
        "nnrh_profile_enable": (i, [i]),
        "nnrh_profile_enabled": (i, []),
        "nnrh_graph_begin_capture": (i, [vp]),
        "nnrh_graph_end_capture": (i, [vp, P(vp)]),
        "nnrh_graph_launch": (i, [vp, vp]),
        "nnrh_graph_destroy": (i, [vp]),
        "nnrh_profile_reset": (i, []),
        "nnrh_profile_count": (i, [P(i)]),
        "nnrh_profile_get": (i, [i, P(C.c_char_p), P(i), P(C.c_double)]),
        "nnrh_qconv_dispatch": (i, [P(QConvDesc), P(i)]),
        "nnrh_qconv_create": (i, [P(vp), P(QConvDesc)]),
        "nnrh_qconv_branch": (i, [vp, P(i)]),
        "nnrh_qconv_run": (i, [vp, vp, vp, vp]),
        "nnrh_qconv_destroy": (i, [vp]),
        "nnrh_qconv_fuse_add": (i, [vp, P(QAddFuseDesc)]),
        "nnrh_qconv_run_add": (i, [vp, vp, vp, vp, vp]),
        "nnrh_qconv_fuse_quantize": (i, [vp, f, i]),
        "nnrh_qconv_run_f32": (i, [vp, vp, vp, vp]),
        "nnrh_qconv_fuse_maxpool": (i, [vp, i, i, i, i, i, i, i, i]),
        "nnrh_global_avgpool_dequant": (i, [vp, vp, i, i, i, i, i, f, i, vp]),
        "nnrh_multihead_attention_workspace": (i, [i, i, i, i, P(sz)]),
        "nnrh_multihead_attention_f32": (i, [vp, vp, vp, vp, i, i, i, i, f, vp, vp, vp]),
        "nnrh_multihead_attention_minmax_count": (i, [i, i, i, i, P(i)]),
        "nnrh_qmatmul_create": (i, [P(vp), P(QMatMulDesc)]),
        "nnrh_qmatmul_run": (i, [vp, vp, ll, vp, i, vp, vp, vp]),
        "nnrh_qmatmul_destroy": (i, [vp]),
        "nnrh_qmatmul_fuse_dq_bias": (i, [vp, f, i, P(f)]),
        "nnrh_qmatmul_fuse_gelu": (i, [vp]),
        "nnrh_qmatmul_minmax_count": (i, [vp, i, P(i)]),
        "nnrh_qmatmul_set_minmax_out": (i, [vp, vp, i]),
        "nnrh_qmatmul_set_codes_out": (i, [vp, i]),
        "nnrh_qmatmul_dq_params": (i, [vp, P(i), P(f), P(vp)]),
        "nnrh_qmatmul_group_set_codes_out": (i, [vp, i]),
        "nnrh_add_layernorm_codes_f32": (i, [P(DqCodes), vp, vp, vp, vp, sz, i, f, vp, vp]),
        "nnrh_multihead_attention_codes_f32": (i, [P(DqCodes), P(DqCodes), P(DqCodes), vp, i, i, i, i, f, vp, vp]),
        "nnrh_qmatmul_dynamic_quantize_codes": (i, [vp, vp, i, vp, vp, vp, vp]),
        "nnrh_qmatmul_group_create": (i, [P(vp), P(vp), i]),
        "nnrh_qmatmul_group_run": (i, [vp, vp, i, P(vp), vp, vp, vp]),
        "nnrh_qmatmul_group_destroy": (i, [vp]),
        "nnrh_dynamic_quantize_linear_parts": (i, [vp, sz, vp, i, vp, vp, vp, vp]),
        "nnrh_add_layernorm_f32": (i, [vp, vp, vp, vp, vp, sz, i, f, vp, vp]),
        "nnrh_matmul_integer_create": (i, [P(vp), i, i, i, i, i, i]),
        "nnrh_matmul_integer_run": (i, [vp, vp, ll, vp, ll, i, i, vp, i, vp]),
        "nnrh_matmul_integer_destroy": (i, [vp]),
        "nnrh_matmul_integer_scaled_create": (i, [P(vp), P(MmiScaledDesc)]),
        "nnrh_matmul_integer_run_dev_zp": (i, [vp, vp, ll, vp, ll, vp, i, vp, i, vp]),
        "nnrh_cast_to_f32": (i, [vp, i, vp, sz, vp]),
        "nnrh_quantize_linear": (i, [vp, sz, f, i, i, vp, vp]),
        "nnrh_dequantize_linear": (i, [vp, i, sz, f, i, vp, vp]),
        "nnrh_dynamic_quantize_workspace": (sz, []),
        "nnrh_dynamic_quantize_linear": (i, [vp, sz, vp, vp, vp, vp, vp]),
        "nnrh_dynamic_quantize_linear_noalloc": (i, [vp, sz, vp, vp, vp, vp]),
        "nnrh_qlinear_add": (i, [i, vp, vp, vp, sz, i, i, i, i, f, i, f, i, f, i, vp]),
        "nnrh_qlinear_mul": (i, [i, vp, vp, vp, sz, i, i, i, i, f, i, f, i, f, i, vp]),
        "nnrh_qlinear_global_avgpool": (i, [vp, vp, i, i, i, i, i, f, i, f, i, vp]),
        "nnrh_qlinear_avgpool": (i, [vp, vp] + [i] * 14 + [f, i, f, i, vp]),
        "nnrh_qlinear_concat_part": (i, [vp, vp, ll, ll, ll, ll, i, f, i, f, i, vp]),
        "nnrh_batchnorm_u8": (i, [vp, i, vp, vp, vp, ll, i, ll, i, vp]),
        "nnrh_qlinear_concat": (i, [i, vp, vp, vp, vp, ll, i, f, i, vp, vp]),
        "nnrh_conv_integer_create": (i, [C.POINTER(vp)] + [i] * 18),
        "nnrh_conv_integer_run": (i, [vp, vp, vp, i, i, vp, vp, vp]),
        "nnrh_conv_integer_destroy": (i, [vp]),
        "nnrh_batchnorm_f32": (i, [vp, vp, vp, vp, ll, i, ll, i, vp]),
        "nnrh_maxpool_u8_nhwc": (i, [vp, vp] + [i] * 12 + [vp]),
        "nnrh_nchw_to_nhwc_u8": (i, [vp, vp, i, i, i, vp]),
        "nnrh_global_avgpool_f32": (i, [vp, vp, i, i, i, i, vp]),
        "nnrh_gemm_f32": (i, [vp, vp, vp, vp, i, i, i, i, i, f, f, i, vp]),
        "nnrh_clip_f32": (i, [vp, vp, sz, f, f, vp]),
        "nnrh_gemm_f32_batched": (i, [vp, vp, vp, vp, i, i, i, i, i, f, f, i, i, ll, ll, ll, vp]),
        "nnrh_binary_f32": (i, [i, vp, vp, vp, sz, i, i, i, vp]),
        "nnrh_softmax_f32": (i, [vp, vp, sz, i, vp]),
        "nnrh_layernorm_f32": (i, [vp, vp, vp, vp, sz, i, f, vp]),
        "nnrh_gelu_f32": (i, [vp, vp, sz, vp]),
        "nnrh_hardswish_f32": (i, [vp, vp, sz, i, vp]),
        "nnrh_transpose_f32": (i, [vp, vp, i, P(i), P(i), vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != NNRH_OK:
        raise NnrHipError(rc, lib().nnrh_last_error().decode())


def ptr(t) -> int:
    """Device (or host) address of a torch tensor / numpy array / int."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    if hasattr(t, "ctypes"):
        return t.ctypes.data
    raise TypeError(type(t))


def profile_enable(on: bool = True) -> None:
    check(lib().nnrh_profile_enable(1 if on else 0))


def profile_reset() -> None:
    check(lib().nnrh_profile_reset())


def profile_read(variants: bool = False) -> dict:
    """{kernel name: (launches, total_ms)} accumulated since the last reset.
    With variants=True only the "variant:..." entries: launches of each
    GEMM kernel instantiation (tile, stages, producer, epilogue), no time."""
    L = lib()
    n = C.c_int()
    check(L.nnrh_profile_count(C.byref(n)))
    out = {}
    for i in range(n.value):
        name, cnt, ms = C.c_char_p(), C.c_int(), C.c_double()
        check(L.nnrh_profile_get(i, C.byref(name), C.byref(cnt), C.byref(ms)))
        nm = name.value.decode()
        if nm.startswith("variant:") == variants:
            out[nm] = (cnt.value, ms.value)
    return out


def cur_stream() -> int:
    import torch
    return torch.cuda.current_stream().cuda_stream
