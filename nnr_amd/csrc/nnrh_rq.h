// nnrh_rq.h -- bit-level requantize formulas of NNR's int8 path, as device
// functions. Every file that includes this is compiled with
// -ffp-contract=off: a*b + c stays two roundings; explicit __builtin_fmaf sits
// where the reference uses _mm512_fmadd_ps.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nnrh {

// _mm512_max_ps(_mm512_min_ps(v, hi), lo)
__device__ __forceinline__ float clamp_minmax(float v, float lo, float hi) {
    v = v < hi ? v : hi;
    return v > lo ? v : lo;
}
__device__ __forceinline__ int clampi(int v, int lo, int hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}
// (int32_t) of a float on x86 (cvttss2si / cvtss2si): out-of-range and NaN
// give INT32_MIN. The GPU conversion saturates instead, so mirror x86.
__device__ __forceinline__ int x86_f2i(float r) {
    return (r >= -2147483648.0f && r < 2147483648.0f) ? (int)r : (int)0x80000000;
}
__device__ __forceinline__ int32_t wrap_add(int32_t a, int32_t b) {
    return (int32_t)((uint32_t)a + (uint32_t)b);
}
__device__ __forceinline__ int32_t wrap_mul(int32_t a, int32_t b) {
    return (int32_t)((uint32_t)a * (uint32_t)b);
}
// Gelu, erf form (approximate = "none"): 0.5 x (1 + erf(x / sqrt 2)). The
// standalone kernel and every fused epilogue call this one expression, so
// fused and unfused results are the same bits.
__device__ __forceinline__ float gelu_erf(float v) {
    return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
}

// RQ-A: SIMD epilogue of the depthwise / direct / im2col paths
// (QLinearConv.cpp:630-638, depthwise_int8_avx512.h:249-255).
__device__ __forceinline__ int rq_a(int32_t acc, float cs, float bf, float inv_y,
                                    int y_zp, int L, int hi) {
    float f = __builtin_fmaf((float)acc, cs, bf);
    float q = f * inv_y;
    q = __builtin_rintf(q);
    q = q + (float)y_zp;
    q = clamp_minmax(q, (float)L, (float)hi);
    return (int)q;
}

// RQ-A': scalar-tail expression (QLinearConv.cpp:640-645), no contraction.
__device__ __forceinline__ int rq_a_tail(int32_t acc, float cs, float bf,
                                         float inv_y, int y_zp, int L, int hi) {
    float t = (float)acc * cs;
    float val = t + bf;
    float q = val * inv_y;
    int r = wrap_add(x86_f2i(__builtin_rintf(q)), y_zp);
    return clampi(r, L, hi);
}

// RQ-B: JIT NR48/NR16 epilogue (jit_conv_int8_ukernel.cpp:950-964).
__device__ __forceinline__ int rq_b(int32_t v, float os, int y_zp, int lo, int hi) {
    float f = (float)v * os;
    float qlo = (float)lo - (float)y_zp, qhi = (float)hi - (float)y_zp;
    f = f > qlo ? f : qlo;
    f = f < qhi ? f : qhi;
    return (int)__builtin_rintf(f) + y_zp;
}

// RQ-B': scalar third sub-panel of NR48 (gemm_int8_avx512.h:1487-1509).
__device__ __forceinline__ int rq_b_roundf(int32_t v, float os, int y_zp, int lo,
                                           int hi) {
    float f = (float)v * os;
    float qlo = (float)lo - (float)y_zp, qhi = (float)hi - (float)y_zp;
    f = f > qlo ? f : qlo;
    f = f < qhi ? f : qhi;
    int r = (int)__builtin_roundf(f) + y_zp;
    return clampi(r, 0, 255);
}

// RQ-C: first-layer epilogue (conv_first_layer_int8_avx512.h:262-273).
__device__ __forceinline__ int rq_c(int32_t acc, float cs, float bf, float inv_y,
                                    int y_zp, int qmin, int qmax) {
    float t = __builtin_fmaf((float)acc, cs, bf);
    float f = __builtin_fmaf(t, inv_y, (float)y_zp);
    f = clamp_minmax(f, (float)qmin, (float)qmax);
    return (int)__builtin_rintf(f);
}

// RQ-D: QLinearMatMul (QLinearMatMul.cpp:188-198), y_zp added before rounding.
__device__ __forceinline__ int rq_d(int32_t acc, float cm, int y_zp, int lo, int hi) {
    float t = (float)acc * cm;
    float val = t + (float)y_zp;
    return clampi(x86_f2i(__builtin_rintf(val)), lo, hi);
}

// ---------------------------------------------------------------------------
// Fast forms of the same formulas for the GEMM epilogue. Exactness:
//  * clamp(max then min) == v_med3 for qlo <= qhi and non-NaN input;
//  * for |x| < 2^22, fl(x + 1.5*2^23) lies in [2^23, 2^24] where the ulp is
//    1, so it is x rounded to an integer with ties to even (1.5*2^23 is even),
//    and its bit pattern is 0x4B400000 + rne(x);
//  * 0x4B400000 has a zero low byte, so the low byte of bits + zp is the
//    output byte of rne(x) + zp.
// Inputs that could exceed the window are first clamped to +-2^21, which
// never changes a result that saturates to an 8-bit range.
constexpr float RNE_MAGIC = 12582912.0f;   // 1.5 * 2^23
constexpr int RNE_MAGIC_BITS = 0x4B400000;

__device__ __forceinline__ int rne_bits(float x) { return __float_as_int(x + RNE_MAGIC); }
__device__ __forceinline__ float med3f(float x, float lo, float hi) {
    return __builtin_amdgcn_fmed3f(x, lo, hi);
}
__device__ __forceinline__ int med3i(int x, int lo, int hi) {
    return x < lo ? lo : (x > hi ? hi : x);
}

// RQ-B: f = clamp(float(v) * os, lo - zp, hi - zp); byte(rne(f) + zp)
__device__ __forceinline__ uint32_t rqb_fast(int32_t v, float os, int y_zp, int lo, int hi) {
    float f = (float)v * os;
    f = med3f(f, (float)lo - (float)y_zp, (float)hi - (float)y_zp);
    return (uint32_t)(rne_bits(f) + y_zp);
}
// RQ-A: clamp(rne(fma(v,cs,bf) * inv_y) + zp, L, hi)
__device__ __forceinline__ uint32_t rqa_fast(int32_t v, float cs, float bf, float inv_y, int y_zp,
                                             int L, int hi) {
    float f = __builtin_fmaf((float)v, cs, bf);
    float q = med3f(f * inv_y, -2097152.0f, 2097152.0f);
    return (uint32_t)med3i(rne_bits(q) - RNE_MAGIC_BITS + y_zp, L, hi);
}
// RQ-C: rne(clamp(fma(fma(v,cs,bf), inv_y, zp), qmin, qmax))
__device__ __forceinline__ uint32_t rqc_fast(int32_t v, float cs, float bf, float inv_y, int y_zp,
                                             int qmin, int qmax) {
    float t = __builtin_fmaf((float)v, cs, bf);
    float f = __builtin_fmaf(t, inv_y, (float)y_zp);
    f = med3f(f, (float)qmin, (float)qmax);
    return (uint32_t)rne_bits(f);
}
// RQ-D: clamp(nearbyint(v*cm + zp), lo, hi); |val| >= 2^31 converts to
// INT32_MIN on x86 and so clamps to lo
__device__ __forceinline__ uint32_t rqd_fast(int32_t v, float cm, int y_zp, int lo, int hi) {
    float t = (float)v * cm;
    float val = t + (float)y_zp;
    if (!(val < 2147483648.0f && val >= -2147483648.0f)) return (uint32_t)lo;
    float q = med3f(val, -2097152.0f, 2097152.0f);
    return (uint32_t)med3i(rne_bits(q) - RNE_MAGIC_BITS, lo, hi);
}

}  // namespace nnrh
