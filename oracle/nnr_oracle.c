/*
 * nnr_oracle.c -- CPU restatement of NNR's int8 QDQ compute path.
 *
 * TEST INFRASTRUCTURE ONLY (see nnr_oracle.h). Not part of the product.
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off -fopenmp).
 *
 * Citations are path:line into the reference tree (beru/nnr).
 */
#include "nnr_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_contract = 0;
static int g_threads = 0;
static int g_vnni = 0;   /* 1: accumulators through the AVX-512 VNNI restatement */

void orc_set_vnni(int on) { g_vnni = on && orc_vnni_available(); }
int orc_get_vnni(void) { return g_vnni; }

void orc_set_contract(int on) { g_contract = on ? 1 : 0; }
int orc_get_contract(void) { return g_contract; }
void orc_set_threads(int n) { g_threads = n; }
int orc_get_threads(void) {
#ifdef _OPENMP
    return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
    return 1;
#endif
}

/* a*b + c as a C++ expression in the reference: two roundings unless the
 * compiler contracts it (see header). */
static inline float mul_add_expr(float a, float b, float c) {
    if (g_contract) return fmaf(a, b, c);
    float t = a * b;
    return t + c;
}

/* (int32_t)float on x86 (cvttss2si): out of range or NaN -> INT32_MIN */
static inline int x86_f2i(float r) {
    return (r >= -2147483648.0f && r < 2147483648.0f) ? (int)r : (int)0x80000000;
}
static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
/* _mm512_max_ps(_mm512_min_ps(v, hi), lo) */
static inline float clampf_minmax(float v, float lo, float hi) {
    v = v < hi ? v : hi;
    return v > lo ? v : lo;
}

/* ---- fp16: src/nnrconf.h:147-199 ----------------------------------- */
uint16_t orc_f32_to_f16(float v) {
    uint32_t u; memcpy(&u, &v, 4);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    int e = (int)((u >> 23) & 0xffu) - 127;
    uint32_t mant = u & 0x7fffffu;
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    if (e >= -14) {
        uint32_t rb = mant & 0x1fffu;
        uint16_t y = (uint16_t)(sign | ((uint16_t)(e + 15) << 10) | (uint16_t)(mant >> 13));
        if (rb > 0x1000u || (rb == 0x1000u && (y & 1u))) y++;
        return y;
    }
    if (e >= -24) {
        mant |= 0x800000u;
        int sh = -e - 14 + 13;
        uint32_t rb = mant & ((1u << sh) - 1u);
        uint32_t half = 1u << (sh - 1);
        uint16_t y = (uint16_t)(sign | (uint16_t)(mant >> sh));
        if (rb > half || (rb == half && (y & 1u))) y++;
        return y;
    }
    return sign;
}

float orc_f16_to_f32(uint16_t v) {
    uint32_t sign = (uint32_t)(v & 0x8000u) << 16;
    uint32_t e = (v >> 10) & 0x1fu, mant = v & 0x3ffu, u;
    if (e == 0) {
        if (mant == 0) { u = sign; }
        else {
            int ee = 0;
            while (!(mant & 0x400u)) { mant <<= 1; ee--; }
            mant &= 0x3ffu; ee++;
            u = sign | ((uint32_t)(ee + 127 - 15) << 23) | (mant << 13);
        }
    } else if (e == 31) {
        u = sign | 0x7f800000u | (mant << 13);
    } else {
        u = sign | ((e + 127 - 15) << 23) | (mant << 13);
    }
    float f; memcpy(&f, &u, 4);
    return f;
}

/* ---- requantize primitives ------------------------------------------ */

/* RQ-A. SIMD epilogue of the direct / depthwise / im2col paths:
 * src/backend/cpu/QLinearConv.cpp:630-638 (direct),
 * src/backend/x64/depthwise_int8_avx512.h:249-255,
 * src/backend/x64/gemm_int8_avx512.h:727-736 (fused im2col). */
int orc_rq_a(int32_t acc, float cs, float bf, float inv_y, int y_zp, int L, int hi) {
    float f = fmaf((float)acc, cs, bf);
    float q = f * inv_y;
    q = rintf(q);
    q = q + (float)y_zp;
    q = clampf_minmax(q, (float)L, (float)hi);
    return (int)q;
}

/* RQ-A'. Scalar tails: QLinearConv.cpp:640-645, :1181-1185;
 * conv_first_layer_int8_avx512.h:305-313. */
int orc_rq_a_tail(int32_t acc, float cs, float bf, float inv_y, int y_zp, int L, int hi) {
    float val = mul_add_expr((float)acc, cs, bf);
    float t = val * inv_y;
    int q = (int)((uint32_t)x86_f2i(nearbyintf(t)) + (uint32_t)y_zp);
    return clampi(q, L, hi);
}

/* RQ-B. JIT packed NR48 / NHWC-direct NR16 epilogue:
 * src/backend/x64/jit_conv_int8_ukernel.cpp:950-964 and :1900-1918,
 * parameters from src/backend/cpu/QLinearConv_reshape.h:323-335. */
int orc_rq_b(int32_t acc, int32_t bias, float os, int y_zp, int lo, int hi) {
    int32_t v = (int32_t)((uint32_t)acc + (uint32_t)bias);
    float f = (float)v * os;
    f = f > (float)lo - (float)y_zp ? f : (float)lo - (float)y_zp;   /* vmaxps */
    f = f < (float)hi - (float)y_zp ? f : (float)hi - (float)y_zp;   /* vminps */
    int r = (int)rintf(f) + y_zp;                                   /* cvtps2dq */
    /* vpmovusdb: unsigned saturation (r is already inside [lo,hi]) */
    return r;
}

/* RQ-B'. Scalar fallback for the third NR48 sub-panel:
 * src/backend/x64/gemm_int8_avx512.h:1487-1509. */
int orc_rq_b_roundf(int32_t acc, int32_t bias, float os, int y_zp, int lo, int hi) {
    int32_t v = (int32_t)((uint32_t)acc + (uint32_t)bias);
    float f = (float)v * os;
    float qmin = (float)lo - (float)y_zp, qmax = (float)hi - (float)y_zp;
    f = f > qmin ? f : qmin;
    f = f < qmax ? f : qmax;
    int r = (int)roundf(f) + y_zp;
    return clampi(r, 0, 255);
}

/* RQ-C. First-layer epilogue: conv_first_layer_int8_avx512.h:262-273 and
 * :289-302. */
int orc_rq_c(int32_t acc, float cs, float bf, float inv_y, int y_zp, int qmin, int qmax) {
    float t = fmaf((float)acc, cs, bf);
    float f = fmaf(t, inv_y, (float)y_zp);
    f = clampf_minmax(f, (float)qmin, (float)qmax);
    return (int)rintf(f);
}

/* RQ-D. QLinearMatMul: src/backend/cpu/QLinearMatMul.cpp:188-198. */
int orc_rq_d(int32_t acc, float cm, int y_zp, int lo, int hi) {
    float val = mul_add_expr((float)acc, cm, (float)y_zp);
    int iv = x86_f2i(nearbyintf(val));
    return clampi(iv, lo, hi);
}

/* ---- element access -------------------------------------------------- */
static inline int32_t ld_q(const void* p, int dtype, size_t i) {
    switch (dtype) {
    case ORC_U8: return ((const uint8_t*)p)[i];
    case ORC_S8: return ((const int8_t*)p)[i];
    case ORC_I32: return ((const int32_t*)p)[i];
    default: return 0;
    }
}
static inline void st_q(void* p, int dtype, size_t i, int v) {
    if (dtype == ORC_U8) ((uint8_t*)p)[i] = (uint8_t)v;
    else if (dtype == ORC_S8) ((int8_t*)p)[i] = (int8_t)v;
    else ((int32_t*)p)[i] = v;
}
static inline void dtype_range(int dtype, int* lo, int* hi) {
    if (dtype == ORC_U8) { *lo = 0; *hi = 255; } else { *lo = -128; *hi = 127; }
}

/* ---- QuantizeLinear: src/backend/cpu/QuantizeLinear.cpp:128-194 -------
 * total >= 64: 4096-element blocks, 16-wide SIMD body multiplies by
 * fl(1/s); the last (end-i)<16 elements of each block divide by s.
 * total < 64: scalar divide everywhere. */
void orc_quantize_linear(const float* x, size_t n, float scale, int zp,
                         int y_dtype, void* y) {
    int lo, hi; dtype_range(y_dtype, &lo, &hi);
    if (n >= 64) {
        float inv = 1.0f / scale;
        const size_t BLOCK = 4096;
        #pragma omp parallel for schedule(static) num_threads(orc_get_threads())
        for (long long blk = 0; blk < (long long)((n + BLOCK - 1) / BLOCK); blk++) {
            size_t base = (size_t)blk * BLOCK;
            size_t end = base + BLOCK < n ? base + BLOCK : n;
            size_t body_end = end - (end - base) % 16;
            for (size_t i = base; i < body_end; i++) {
                float v = x[i] * inv;
                v = rintf(v) + (float)zp;
                v = clampf_minmax(v, (float)lo, (float)hi);
                st_q(y, y_dtype, i, (int)v);
            }
            for (size_t i = body_end; i < end; i++)
                st_q(y, y_dtype, i, clampi((int)nearbyintf(x[i] / scale) + zp, lo, hi));
        }
    } else {
        for (size_t i = 0; i < n; i++)
            st_q(y, y_dtype, i, clampi((int)nearbyintf(x[i] / scale) + zp, lo, hi));
    }
}

/* ---- DequantizeLinear: src/backend/cpu/DequantizeLinear.cpp:100-152 ---- */
void orc_dequantize_linear(const void* x, int x_dtype, size_t n, float scale,
                           int zp, float* y) {
    for (size_t i = 0; i < n; i++)
        y[i] = ((float)ld_q(x, x_dtype, i) - (float)zp) * scale;
}

/* ---- HardSwish, fp32: src/backend/cpu/HardSwish.cpp:18-50 --------------
 * exec(): avx512::hardswish over the whole tensor (vec_ops_avx512.h:96-117):
 * 16-wide body t = min_ps(max_ps(fl(fl(x * fl(1/6)) + 0.5), 0), 1) -- the
 * AVX-512 max / min return the second operand unless the first compares
 * greater / smaller --, scalar tail t = std::max(0, std::min(1, fl(fl(x / 6)
 * + 0.5))), y = fl(x * t). post_op: the fused form (apply_inplace with no
 * bias -> bias_hardswish(row, n, 0), vec_ops_avx512.h:74-94), which adds the
 * zero bias first. */
void orc_hardswish_f32(const float* x, float* y, size_t n, int post_op) {
    const size_t body = n - n % 16;
    for (size_t i = 0; i < n; i++) {
        float v = x[i];
        if (post_op) v = v + 0.0f;
        float t;
        if (i < body) {
            float u = v * (1.0f / 6.0f);
            u = u + 0.5f;
            float m = u > 0.0f ? u : 0.0f;
            t = m < 1.0f ? m : 1.0f;
        } else {
            float w = v / 6.0f;
            w = w + 0.5f;
            float m = (w < 1.0f) ? w : 1.0f;   /* std::min(1.0f, w) */
            t = (0.0f < m) ? m : 0.0f;         /* std::max(0.0f, m) */
        }
        y[i] = v * t;
    }
}

/* ---- DynamicQuantizeLinear: DynamicQuantizeLinear.cpp:27-58 ------------ */
void orc_dynamic_quantize_linear(const float* x, size_t n, uint8_t* y,
                                 float* y_scale, uint8_t* y_zp) {
    float mn = 0.0f, mx = 0.0f;
    for (size_t i = 0; i < n; i++) {
        mn = x[i] < mn ? x[i] : mn;     /* std::min(x_min, px[i]) */
        mx = mx < x[i] ? x[i] : mx;     /* std::max(x_max, px[i]) */
    }
    mn = mn < 0.0f ? mn : 0.0f;
    mx = mx > 0.0f ? mx : 0.0f;
    float s = (mx - mn) / 255.0f;
    if (s == 0.0f) s = 1.0f;
    int zp = clampi((int)nearbyintf(-mn / s), 0, 255);
    *y_scale = s;
    *y_zp = (uint8_t)zp;
    for (size_t i = 0; i < n; i++)
        y[i] = (uint8_t)clampi((int)nearbyintf(x[i] / s) + zp, 0, 255);
}

/* ---- QLinearMatMul: src/backend/cpu/QLinearMatMul.cpp:111-232 ----------- */
static float ld_scale(const void* p, int sd) {
    if (sd == ORC_F16) return orc_f16_to_f32(*(const uint16_t*)p);
    return *(const float*)p;
}

float orc_qmatmul_combined_scale(const void* a_s, const void* b_s,
                                 const void* y_s, int sd) {
    if (sd == ORC_F16) {
        /* float16_t *= and /= : compute in float, round to half (float16.h) */
        float fa = orc_f16_to_f32(*(const uint16_t*)a_s);
        float fb = orc_f16_to_f32(*(const uint16_t*)b_s);
        float fy = orc_f16_to_f32(*(const uint16_t*)y_s);
        uint16_t h = orc_f32_to_f16(fa * fb);
        h = orc_f32_to_f16(orc_f16_to_f32(h) / fy);
        return orc_f16_to_f32(h);
    }
    float as = *(const float*)a_s, bs = *(const float*)b_s, ys = *(const float*)y_s;
    float t = as * bs;
    return t / ys;
}

int orc_qlinear_matmul(int batch, int m, int n, int k,
                       const void* a, int a_dtype, int batch_a,
                       const void* a_scale, const void* a_zp,
                       const void* b, int b_dtype, int batch_b,
                       const void* b_scale, const void* b_zp,
                       const void* y_scale, const void* y_zp,
                       int sd, void* y, int y_dtype) {
    (void)b_scale;
    int azp = ld_q(a_zp, a_dtype, 0);
    int bzp = ld_q(b_zp, b_dtype, 0);            /* b_zp[0] only (:118-119) */
    int yzp = ld_q(y_zp, y_dtype, 0);
    float cm = orc_qmatmul_combined_scale(a_scale, b_scale, y_scale, sd);
    (void)ld_scale;
    int lo, hi; dtype_range(y_dtype, &lo, &hi);
    if (g_vnni && batch_b <= 1) {
        /* the packed VNNI GEMM's exact accumulators, then RQ-D */
        int32_t* acc = (int32_t*)malloc(sizeof(int32_t) * (size_t)batch * m * n);
        const int rc = orc_vnni_matmul_integer(batch, m, n, k, a, a_dtype,
                                               batch_a <= 1 ? 0 : (long long)m * k, b, b_dtype, azp, bzp, acc);
        if (rc == 0) {
            #pragma omp parallel for schedule(static) num_threads(orc_get_threads())
            for (long long i = 0; i < (long long)batch * m * n; i++)
                st_q(y, y_dtype, (size_t)i, orc_rq_d(acc[i], cm, yzp, lo, hi));
            free(acc);
            return 0;
        }
        free(acc);
    }
    for (int bi = 0; bi < batch; bi++) {
        size_t aoff = batch_a <= 1 ? 0 : (size_t)bi * m * k;
        size_t boff = batch_b <= 1 ? 0 : (size_t)bi * k * n;
        size_t yoff = (size_t)bi * m * n;
        #pragma omp parallel for schedule(static) num_threads(orc_get_threads())
        for (int u = 0; u < m; u++) {
            int32_t* row = (int32_t*)calloc((size_t)n, sizeof(int32_t));
            for (int w = 0; w < k; w++) {
                int32_t av = ld_q(a, a_dtype, aoff + (size_t)u * k + w) - azp;
                for (int v = 0; v < n; v++) {
                    int32_t bv = ld_q(b, b_dtype, boff + (size_t)w * n + v) - bzp;
                    row[v] = (int32_t)((uint32_t)row[v] + (uint32_t)(av * bv));
                }
            }
            for (int v = 0; v < n; v++)
                st_q(y, y_dtype, yoff + (size_t)u * n + v, orc_rq_d(row[v], cm, yzp, lo, hi));
            free(row);
        }
    }
    return 0;
}

/* ---- MatMulInteger: src/backend/cpu/MatMulInteger.cpp:11-150 -----------
 * y = sum (a - a_zp)(b - b_zp) with numpy broadcasting of leading dims. */
int orc_matmul_integer(const int* a_dims, int a_nd, const void* a, int a_dtype,
                       const int* b_dims, int b_nd, const void* b, int b_dtype,
                       int a_zp, int b_zp, int32_t* y) {
    int ad[8], bd[8], yd[8], nd;
    int an = a_nd, bn = b_nd;
    if (an < 1 || bn < 1 || an > 6 || bn > 6) return -1;
    /* promote 1-D operands (MatMulInteger.cpp:29-38) */
    int ta[8], tb[8];
    if (an == 1) { ta[0] = 1; ta[1] = a_dims[0]; an = 2; } else memcpy(ta, a_dims, sizeof(int) * an);
    if (bn == 1) { tb[0] = b_dims[0]; tb[1] = 1; bn = 2; } else memcpy(tb, b_dims, sizeof(int) * bn);
    nd = an > bn ? an : bn;
    for (int i = 0; i < nd; i++) {
        int ia = i - (nd - an), ib = i - (nd - bn);
        ad[i] = ia >= 0 ? ta[ia] : 1;
        bd[i] = ib >= 0 ? tb[ib] : 1;
    }
    int m = ad[nd - 2], k = ad[nd - 1], n = bd[nd - 1];
    if (bd[nd - 2] != k) return -1;
    if (g_vnni) {
        /* B shared by every batch: the packed VNNI GEMM */
        int bshared = 1;
        long long nbat = 1;
        for (int i = 0; i < nd - 2; i++) {
            if (bd[i] != 1) bshared = 0;
            nbat *= ad[i];
        }
        if (bshared && nbat < 0x7fffffff &&
            orc_vnni_matmul_integer((int)nbat, m, n, k, a, a_dtype, (long long)m * k, b, b_dtype, a_zp, b_zp,
                                    y) == 0)
            return 0;
    }
    size_t nb = 1;
    for (int i = 0; i < nd - 2; i++) {
        if (ad[i] != bd[i] && ad[i] > 1 && bd[i] > 1) return -1;
        yd[i] = ad[i] > bd[i] ? ad[i] : bd[i];
        nb *= (size_t)yd[i];
    }
    for (size_t bi = 0; bi < nb; bi++) {
        size_t rem = bi, aoff = 0, boff = 0, astr = 1, bstr = 1;
        for (int i = nd - 3; i >= 0; i--) {
            size_t idx = rem % (size_t)yd[i]; rem /= (size_t)yd[i];
            aoff += (ad[i] > 1 ? idx : 0) * astr;
            boff += (bd[i] > 1 ? idx : 0) * bstr;
            astr *= (size_t)ad[i]; bstr *= (size_t)bd[i];
        }
        aoff *= (size_t)m * k; boff *= (size_t)k * n;
        int32_t* yb = y + bi * (size_t)m * n;
        for (int u = 0; u < m; u++)
            for (int v = 0; v < n; v++) {
                uint32_t s = 0;
                for (int w = 0; w < k; w++)
                    s += (uint32_t)((ld_q(a, a_dtype, aoff + (size_t)u * k + w) - a_zp) *
                                    (ld_q(b, b_dtype, boff + (size_t)w * n + v) - b_zp));
                yb[(size_t)u * n + v] = (int32_t)s;
            }
    }
    return 0;
}

/* ---- QLinearConv ------------------------------------------------------ */

/* conv_shape.h:21-81, auto_pad NOTSET */
int orc_conv_out_dim(int in, int k, int d, int s, int pb, int pe) {
    int ek = (k - 1) * d + 1;
    return (int)floorf((float)(in + pb + pe - ek) / (float)s + 1.0f);
}

static int conv_per_channel_zp(const orc_conv_params* p) {
    /* QLinearConv.cpp:136-153: collapse all-equal per-channel zp */
    if (p->w_zp_count <= 1) return 0;
    for (int i = 1; i < p->w_zp_count; i++)
        if (p->w_zp[i] != p->w_zp[0]) return 1;
    return 0;
}

/* First-match dispatch of QLinearConv::exec_simd_4d (QLinearConv.cpp:1337-1351)
 * with the prepack preconditions of QLinearConv_reshape.h:36-284. */
int orc_conv_dispatch(const orc_conv_params* p) {
    const int u8 = p->act_dtype == ORC_U8;
    const int pcz = conv_per_channel_zp(p);
    const int wzp0 = p->w_zp_count > 0 ? p->w_zp[0] : 0;
    const int Cg = p->C / p->group;
    const int is_dw = (p->group == p->OC && Cg == 1);
    const int vnni_ok = p->vnni && u8 && !pcz;
    const int dil1 = (p->dH == 1 && p->dW == 1);
    /* (1) exec_dw_int8_nhwc: QLinearConv.cpp:467-526 */
    if (vnni_ok && is_dw && p->y_nhwc) return ORC_BR_DW;
    /* (2) exec_first_layer_int8: QLinearConv.cpp:665-700; prepack
     *     QLinearConv_reshape.h:211-256 (group 1, dil 1, IC<=4, kH>=3, OC>=16, w_zp 0) */
    if (vnni_ok && p->group == 1 && dil1 && Cg <= 4 && p->kH >= 3 && p->OC >= 16 &&
        wzp0 == 0 && p->C <= 4 && p->pad_t == p->pad_b && p->pad_l == p->pad_r &&
        !p->x_nhwc)
        return ORC_BR_FIRST;
    /* (3) exec_direct_int8: QLinearConv.cpp:579-652 */
    if (vnni_ok && p->group == 1 && dil1 && wzp0 == 0 && p->oH * p->oW <= 256 && !p->y_nhwc)
        return ORC_BR_DIRECT;
    /* (4) exec_packed_nr48: QLinearConv.cpp:706-848, NR16 predicate :750-759 */
    if (vnni_ok && p->group == 1) {
        if (p->kH == 3 && p->kW == 3 && p->sH == 1 && p->sW == 1 && dil1 &&
            p->pad_t == 1 && p->pad_l == 1 && p->C >= 64 && p->OC >= 64 &&
            (p->OC % 16) == 0 && wzp0 == 0 && p->y_nhwc)
            return ORC_BR_NR16;
        return ORC_BR_PACKED;
    }
    /* (6) exec_vnni_im2col: QLinearConv.cpp:1010-1196 */
    if (vnni_ok) return (p->sH == 1 && p->sW == 1) ? ORC_BR_IM2COL_S1 : ORC_BR_IM2COL;
    /* (7) exec_float_fallback: QLinearConv.cpp:1205-1335 */
    return ORC_BR_FLOAT;
}

void orc_conv_acc(const orc_conv_params* p, const void* x, const int8_t* w,
                  int32_t* acc) {
    if (g_vnni) {
        /* the same exact accumulators from the AVX-512 VNNI restatement */
        if (p->group == p->C && p->OC == p->C && p->C > 1 && orc_vnni_depthwise_acc(p, x, w, acc) == 0) return;
        if (p->group == 1 && orc_vnni_conv_acc(p, x, w, acc) == 0) return;
    }
    const int N = p->N, C = p->C, H = p->H, W = p->W;
    const int OC = p->OC, kH = p->kH, kW = p->kW, G = p->group;
    const int Cg = C / G, OCg = OC / G, oH = p->oH, oW = p->oW;
    const int pcz = conv_per_channel_zp(p);
    const int u8 = p->act_dtype == ORC_U8;
    /* xs: (x - x_zp) as int16, NHWC */
    int16_t* xs = (int16_t*)malloc(sizeof(int16_t) * (size_t)N * H * W * C);
    #pragma omp parallel for schedule(static) num_threads(orc_get_threads())
    for (long long i = 0; i < (long long)N * H * W; i++) {
        long long n = i / ((long long)H * W), hw = i % ((long long)H * W);
        for (int c = 0; c < C; c++) {
            size_t src = p->x_nhwc ? (size_t)i * C + c : ((size_t)(n * C + c) * H * W + hw);
            int v = u8 ? ((const uint8_t*)x)[src] : ((const int8_t*)x)[src];
            xs[(size_t)i * C + c] = (int16_t)(v - p->x_zp);
        }
    }
    /* ws: (w - w_zp) as int16, [OC][kH][kW][Cg] */
    int16_t* ws = (int16_t*)malloc(sizeof(int16_t) * (size_t)OC * kH * kW * Cg);
    /* The VNNI branches read w_zp through the activation type T
     * (QLinearConv.cpp:386, `(T*)inputs[5]->data`); the float fallback packs
     * with the weight type, int8 (QLinearConv_reshape.h:72-78). */
    const int zp_as_u8 = u8 && orc_conv_dispatch(p) != ORC_BR_FLOAT;
    for (int oc = 0; oc < OC; oc++) {
        int8_t zb = pcz ? p->w_zp[oc] : (p->w_zp_count > 0 ? p->w_zp[0] : 0);
        int zp = zp_as_u8 ? (int)(uint8_t)zb : (int)zb;
        for (int c = 0; c < Cg; c++)
            for (int a = 0; a < kH; a++)
                for (int b = 0; b < kW; b++)
                    ws[(((size_t)oc * kH + a) * kW + b) * Cg + c] =
                        (int16_t)(w[(((size_t)oc * Cg + c) * kH + a) * kW + b] - zp);
    }
    #pragma omp parallel for schedule(dynamic) num_threads(orc_get_threads())
    for (long long r = 0; r < (long long)N * oH; r++) {
        int n = (int)(r / oH), oh = (int)(r % oH);
        for (int ow = 0; ow < oW; ow++) {
            for (int oc = 0; oc < OC; oc++) {
                int g = oc / OCg;
                int32_t s = 0;
                for (int a = 0; a < kH; a++) {
                    int ih = oh * p->sH - p->pad_t + a * p->dH;
                    if (ih < 0 || ih >= H) continue;
                    for (int b = 0; b < kW; b++) {
                        int iw = ow * p->sW - p->pad_l + b * p->dW;
                        if (iw < 0 || iw >= W) continue;
                        const int16_t* xp = xs + (((size_t)n * H + ih) * W + iw) * C + (size_t)g * Cg;
                        const int16_t* wp = ws + (((size_t)oc * kH + a) * kW + b) * Cg;
                        int32_t t = 0;
                        for (int c = 0; c < Cg; c++) t += (int32_t)xp[c] * (int32_t)wp[c];
                        s = (int32_t)((uint32_t)s + (uint32_t)t);
                    }
                }
                acc[(((size_t)n * OC + oc) * oH + oh) * oW + ow] = s;
            }
        }
    }
    free(xs);
    free(ws);
}

/* acc_nhwc: accumulators laid out [N][oH][oW][OC] instead of [N][OC][oH][oW]
 * (the VNNI restatement's row-major output); the loop then walks pixels */
static int conv_epilogue(const orc_conv_params* p, const int32_t* acc, void* y, int acc_nhwc);

int orc_qlinear_conv_from_acc(const orc_conv_params* p, const int32_t* acc, void* y) {
    return conv_epilogue(p, acc, y, 0);
}

static int conv_epilogue(const orc_conv_params* p, const int32_t* acc, void* y, int acc_nhwc) {
    const int br = orc_conv_dispatch(p);
    const int N = p->N, OC = p->OC, oH = p->oH, oW = p->oW, sp = oH * oW;
    int lo, hi; dtype_range(p->act_dtype, &lo, &hi);
    const int qmin = p->post_fn ? (lo > p->y_zp ? lo : p->y_zp) : lo;   /* QLinearConv.cpp:419 */
    const float inv_y = 1.0f / p->y_scale;
    float* cs = (float*)malloc(sizeof(float) * OC);
    float* bf = (float*)malloc(sizeof(float) * OC);
    float* os = (float*)malloc(sizeof(float) * OC);
    /* QLinearConv_reshape.h:288-321 */
    for (int oc = 0; oc < OC; oc++) {
        float wsc = p->w_scale_count > 1 ? p->w_scale[oc] : p->w_scale[0];
        cs[oc] = p->x_scale * wsc;
        os[oc] = cs[oc] * inv_y;
        bf[oc] = p->bias ? (float)p->bias[oc] * cs[oc] : 0.0f;
    }
    /* RQ-B' columns: third NR48 sub-panel of the last block (gemm_int8_avx512.h:1465-1510) */
    const int b_prime_from = (OC % 48 > 32) ? OC - OC % 48 + 32 : OC;
    /* tiled im2col (QLinearConv.cpp:1082-1090) */
    int tile_h = oH;
    {
        const size_t TILE_BYTES = 256 * 1024;
        size_t CHW = (size_t)(p->C / p->group) * p->kH * p->kW;
        if (CHW * (size_t)sp > TILE_BYTES) {
            long th = (long)(TILE_BYTES / (CHW * (size_t)oW));
            tile_h = (int)(th < 1 ? 1 : th);
            if (tile_h > oH) tile_h = oH;
        }
    }
    /* the same per-element work in either order: (n, oc) planes for
     * [N][OC][..] accumulators, (n, pixel) rows for [N][..][OC] ones */
    const long long outer = acc_nhwc ? (long long)N * sp : (long long)N * OC;
    const int inner = acc_nhwc ? OC : sp;
    #pragma omp parallel for schedule(static) num_threads(orc_get_threads())
    for (long long oi = 0; oi < outer; oi++) {
        for (int ii = 0; ii < inner; ii++) {
                const int n = (int)(acc_nhwc ? oi / sp : oi / OC);
                const int oc = acc_nhwc ? ii : (int)(oi % OC);
                const int s = acc_nhwc ? (int)(oi % sp) : ii;
                const int oh = s / oW, ow = s % oW;
                int32_t a = acc_nhwc ? acc[((size_t)n * sp + s) * OC + oc] : acc[((size_t)n * OC + oc) * sp + s];
                int q;
                int32_t b32 = p->bias ? p->bias[oc] : 0;
                switch (br) {
                case ORC_BR_DW:
                case ORC_BR_IM2COL_S1:
                    q = orc_rq_a(a, cs[oc], bf[oc], inv_y, p->y_zp, lo, hi);
                    break;
                case ORC_BR_FIRST:
                    if (p->y_nhwc || ow < oW - oW % 16)
                        q = orc_rq_c(a, cs[oc], bf[oc], inv_y, p->y_zp, qmin, hi);
                    else
                        q = orc_rq_a_tail(a, cs[oc], bf[oc], inv_y, p->y_zp, qmin, hi);
                    break;
                case ORC_BR_DIRECT:
                case ORC_BR_FLOAT:
                    if (s < sp - sp % 16)
                        q = orc_rq_a(a, cs[oc], bf[oc], inv_y, p->y_zp, qmin, hi);
                    else
                        q = orc_rq_a_tail(a, cs[oc], bf[oc], inv_y, p->y_zp, qmin, hi);
                    break;
                case ORC_BR_IM2COL: {
                    int oh0 = (oh / tile_h) * tile_h;
                    int th = oH - oh0 < tile_h ? oH - oh0 : tile_h;
                    int tsp = th * oW, ts = (oh - oh0) * oW + ow;
                    if (ts < tsp - tsp % 16)
                        q = orc_rq_a(a, cs[oc], bf[oc], inv_y, p->y_zp, qmin, hi);
                    else
                        q = orc_rq_a_tail(a, cs[oc], bf[oc], inv_y, p->y_zp, qmin, hi);
                    break;
                }
                case ORC_BR_PACKED:
                    if (oc >= b_prime_from)
                        q = orc_rq_b_roundf(a, b32, os[oc], p->y_zp, lo, hi);
                    else
                        q = orc_rq_b(a, b32, os[oc], p->y_zp, lo, hi);
                    break;
                case ORC_BR_NR16:
                default:
                    q = orc_rq_b(a, b32, os[oc], p->y_zp, lo, hi);
                    break;
                }
                size_t di = p->y_nhwc ? (((size_t)n * sp + s) * OC + oc)
                                      : (((size_t)n * OC + oc) * sp + s);
                st_q(y, p->act_dtype, di, q);
            }
    }
    free(cs); free(bf); free(os);
    return br;
}

int orc_qlinear_conv(const orc_conv_params* p, const void* x, const int8_t* w, void* y) {
    int32_t* acc = (int32_t*)malloc(sizeof(int32_t) * (size_t)p->N * p->OC * p->oH * p->oW);
    if (g_vnni && p->group == 1 && orc_vnni_conv_acc_layout(p, x, w, acc, 1) == 0) {
        int br = conv_epilogue(p, acc, y, 1);
        free(acc);
        return br;
    }
    orc_conv_acc(p, x, w, acc);
    int br = orc_qlinear_conv_from_acc(p, acc, y);
    free(acc);
    return br;
}

/* ---- QLinearConv on 3-D tensors (1-D convolution) ------------------------
 * QLinearConv::exec() sends every non-4-D input to exec_typed<T>
 * (QLinearConv.cpp:1355-1368), whose ndim == 3 branch (:286-334) is scalar
 * loops with requantize RQ-S:
 *   cs = fl(x_scale * w_scale[oc]); bf = fl(float(bias[oc]) * cs)   (:301-303)
 *   result = float(sum) * cs + bf       C++ expression (:327), no contraction
 *                                       unless orc_set_contract(1)
 *   q = (int32_t)nearbyint(fl(result / y_scale)) + y_zp, clamp  (:328-329)
 * exec_typed reads x_zp, y_zp, w_zp AND the weights through the activation
 * type T (:194-206: `const T* pw = (const T*)w->data`), so with uint8
 * activations an int8 weight byte counts as its uint8 value.
 * Layout [N][C][W] in and [N][OC][oW] out; p->H == p->kH == 1. */
int orc_qlinear_conv1d(const orc_conv_params* p, const void* x, const int8_t* w, void* y) {
    const int N = p->N, C = p->C, iW = p->W, OC = p->OC, kW = p->kW, G = p->group;
    const int Cg = C / G, OCg = OC / G, oW = p->oW;
    const int u8 = p->act_dtype == ORC_U8;
    int lo, hi; dtype_range(p->act_dtype, &lo, &hi);
    const int pcz = conv_per_channel_zp(p);
    for (int n = 0; n < N; n++)
        for (int oc = 0; oc < OC; oc++) {
            const int g = oc / OCg;
            const float ws = p->w_scale_count > 1 ? p->w_scale[oc] : p->w_scale[0];
            const int8_t zb = pcz ? p->w_zp[oc] : (p->w_zp_count > 0 ? p->w_zp[0] : 0);
            const int32_t wzp = u8 ? (int32_t)(uint8_t)zb : (int32_t)zb;
            const float cs = p->x_scale * ws;
            const float bf = p->bias ? (float)p->bias[oc] * cs : 0.0f;
            for (int ow = 0; ow < oW; ow++) {
                int32_t sum = 0;
                for (int c = 0; c < Cg; c++) {
                    const int ic = g * Cg + c;
                    for (int kw = 0; kw < kW; kw++) {
                        const int iw = ow * p->sW - p->pad_l + kw * p->dW;
                        if (iw < 0 || iw >= iW) continue;
                        const size_t xi = ((size_t)n * C + ic) * iW + iw;
                        const int32_t xv = (u8 ? (int32_t)((const uint8_t*)x)[xi]
                                               : (int32_t)((const int8_t*)x)[xi]) - p->x_zp;
                        const int8_t wb = w[((size_t)oc * Cg + c) * kW + kw];
                        const int32_t wv = (u8 ? (int32_t)(uint8_t)wb : (int32_t)wb) - wzp;
                        sum = (int32_t)((uint32_t)sum + (uint32_t)(xv * wv));
                    }
                }
                const float result = mul_add_expr((float)sum, cs, bf);
                const float q = result / p->y_scale;
                int v = x86_f2i(nearbyintf(q));
                v = (int)((uint32_t)v + (uint32_t)p->y_zp);
                st_q(y, p->act_dtype, ((size_t)n * OC + oc) * oW + ow, clampi(v, lo, hi));
            }
        }
    return ORC_BR_TYPED;
}

/* ---- QLinearAdd: src/backend/cpu/QLinearAdd.cpp:33-265 ----------------- */
void orc_qlinear_add(int kind, const void* a, const void* b, void* y, size_t n,
                     int N, int C, int HW, int y_nhwc, int dt,
                     float a_s, int a_zp, float b_s, int b_zp, float y_s, int y_zp) {
    int lo, hi; dtype_range(dt, &lo, &hi);
    const float sa = a_s / y_s, sb = b_s / y_s;
    if (kind == ORC_ADD_SAME) {
        /* :61-104; SIMD body on 16-chunks, scalar tail on the last n%16 */
        float fixed;
        if (g_contract) fixed = (float)y_zp - fmaf(sa, (float)a_zp, sb * (float)b_zp);
        else { float t1 = sa * (float)a_zp, t2 = sb * (float)b_zp; fixed = (float)y_zp - (t1 + t2); }
        size_t body = n - n % 16;
        #pragma omp parallel for schedule(static) num_threads(orc_get_threads())
        for (long long ii = 0; ii < (long long)body; ii++) {
            size_t i = (size_t)ii;
            float fa = (float)ld_q(a, dt, i), fb = (float)ld_q(b, dt, i);
            float v = fmaf(fb, sb, fixed);
            v = fmaf(fa, sa, v);
            int r = (int)rintf(v);
            st_q(y, dt, i, clampi(r, lo, hi));   /* max(.,0)+cvtusepi32 / cvtsepi32 */
        }
        for (size_t i = body; i < n; i++) {
            float da = (float)(ld_q(a, dt, i) - a_zp), db = (float)(ld_q(b, dt, i) - b_zp);
            float v;
            if (g_contract) v = fmaf(sa, da, sb * db) + (float)y_zp;
            else { float t1 = sa * da, t2 = sb * db; v = (t1 + t2) + (float)y_zp; }
            st_q(y, dt, i, clampi((int)nearbyintf(v), lo, hi));
        }
        return;
    }
    if (kind == ORC_ADD_B_SCALAR || kind == ORC_ADD_A_SCALAR) {
        /* :108-119 */
        int sc_is_b = kind == ORC_ADD_B_SCALAR;
        float cval = sc_is_b ? sb * (float)(ld_q(b, dt, 0) - b_zp)
                             : sa * (float)(ld_q(a, dt, 0) - a_zp);
        for (size_t i = 0; i < n; i++) {
            float v;
            if (sc_is_b) v = mul_add_expr(sa, (float)(ld_q(a, dt, i) - a_zp), cval) + (float)y_zp;
            else { float t = sb * (float)(ld_q(b, dt, i) - b_zp); v = (cval + t) + (float)y_zp; }
            st_q(y, dt, i, clampi((int)nearbyintf(v), lo, hi));
        }
        return;
    }
    if (kind == ORC_ADD_PER_CHANNEL) {
        /* a is full [N,C,H,W] (physical per y_nhwc), b is [C] (:120-226) */
        const float s_full = sa, s_ch = sb;
        if (y_nhwc) {
            float* ch_off = (float*)malloc(sizeof(float) * C);
            for (int c = 0; c < C; c++)
                ch_off[c] = mul_add_expr(s_ch, (float)(ld_q(b, dt, c) - b_zp), (float)y_zp);
            for (size_t pos = 0; pos < (size_t)N * HW; pos++) {
                int cbody = C - C % 16, c = 0;
                for (; c < cbody; c++) {
                    float fa = (float)ld_q(a, dt, pos * C + c);
                    float v = fmaf(fa - (float)a_zp, s_full, ch_off[c]);
                    v = rintf(v);
                    v = clampf_minmax(v, (float)lo, (float)hi);
                    st_q(y, dt, pos * C + c, (int)v);
                }
                for (; c < C; c++) {
                    float v = mul_add_expr(s_full, (float)(ld_q(a, dt, pos * C + c) - a_zp), ch_off[c]);
                    st_q(y, dt, pos * C + c, clampi((int)nearbyintf(v), lo, hi));
                }
            }
            free(ch_off);
        } else {
            for (size_t nc = 0; nc < (size_t)N * C; nc++) {
                int c = (int)(nc % C);
                float ch_val = s_ch * (float)(ld_q(b, dt, c) - b_zp);
                float voff = ch_val + (float)y_zp;
                int ibody = HW - HW % 16, i = 0;
                for (; i < ibody; i++) {
                    float fa = (float)ld_q(a, dt, nc * HW + i);
                    float v = fmaf(fa - (float)a_zp, s_full, voff);
                    v = rintf(v);
                    v = clampf_minmax(v, (float)lo, (float)hi);
                    st_q(y, dt, nc * HW + i, (int)v);
                }
                for (; i < HW; i++) {
                    float v = mul_add_expr(s_full, (float)(ld_q(a, dt, nc * HW + i) - a_zp), ch_val) + (float)y_zp;
                    st_q(y, dt, nc * HW + i, clampi((int)nearbyintf(v), lo, hi));
                }
            }
        }
    }
}

/* ---- MaxPool uint8 NHWC: src/backend/x64/pool_x64.h:396-436 ------------ */
/* ---- the rest of the QLinear family (QOperator models) ----------------- */

/* QLinearGlobalAveragePool_operator::exec_typed (QLinearGlobalAveragePool.cpp:28-60),
 * RQ-F: rs = fl(x_s / fl(y_s * float(spatial))); per (n, c) the int32 sum of
 * the raw values minus (int32)(x_zp * spatial), then nearbyint(fl(sum * rs))
 * + y_zp and the clamp. x is NCHW, or NHWC with x_nhwc (the same sums). */
void orc_qlinear_global_avgpool(const void* x, void* y, int N, int C, int spatial, int x_nhwc, int dt,
                                float x_s, int x_zp, float y_s, int y_zp) {
    int lo, hi; dtype_range(dt, &lo, &hi);
    const float rs = x_s / (y_s * (float)spatial);                       /* :46 */
    for (int n = 0; n < N; n++)
        for (int c = 0; c < C; c++) {
            uint32_t sum = 0;                                               /* :52-54 */
            for (int s = 0; s < spatial; s++) {
                size_t i = x_nhwc ? ((size_t)n * spatial + s) * C + c : ((size_t)n * C + c) * spatial + s;
                sum += (uint32_t)ld_q(x, dt, i);
            }
            sum -= (uint32_t)x_zp * (uint32_t)spatial;                      /* :55 */
            int32_t q = x86_f2i(nearbyintf((float)(int32_t)sum * rs));      /* :56 */
            q = (int32_t)((uint32_t)q + (uint32_t)y_zp);
            st_q(y, dt, (size_t)n * C + c, clampi(q, lo, hi));              /* :57 */
        }
}

/* QLinearAveragePool_operator::exec_typed (QLinearAveragePool.cpp:67-115): 2-D,
 * count_include_pad never set (:41-42), so the count is the in-image taps;
 * avg = fl(fl(float(sum) * x_s) / float(count)), q = nearbyint(fl(avg / y_s))
 * + y_zp, clamp. x / y NCHW, or NHWC with nhwc. */
void orc_qlinear_avgpool(const void* x, void* y, int N, int C, int iH, int iW, int oH, int oW,
                         int kH, int kW, int sH, int sW, int pH, int pW, int nhwc, int dt,
                         float x_s, int x_zp, float y_s, int y_zp) {
    int lo, hi; dtype_range(dt, &lo, &hi);
    for (int n = 0; n < N; n++)
        for (int c = 0; c < C; c++)
            for (int oh = 0; oh < oH; oh++)
                for (int ow = 0; ow < oW; ow++) {
                    int32_t sum = 0;
                    int count = 0;
                    for (int kh = 0; kh < kH; kh++) {
                        int ih = oh * sH - pH + kh;
                        if (ih < 0 || ih >= iH) continue;
                        for (int kw = 0; kw < kW; kw++) {
                            int iw = ow * sW - pW + kw;
                            if (iw < 0 || iw >= iW) continue;
                            size_t i = nhwc ? (((size_t)n * iH + ih) * iW + iw) * C + c
                                            : (((size_t)n * C + c) * iH + ih) * iW + iw;
                            sum += ld_q(x, dt, i) - x_zp;
                            count++;
                        }
                    }
                    if (count == 0) count = 1;                              /* :104 */
                    float avg = (float)sum * x_s / (float)count;            /* :105 */
                    int32_t q = x86_f2i(nearbyintf(avg / y_s));
                    q = (int32_t)((uint32_t)q + (uint32_t)y_zp);
                    size_t o = nhwc ? (((size_t)n * oH + oh) * oW + ow) * C + c
                                    : (((size_t)n * C + c) * oH + oh) * oW + ow;
                    st_q(y, dt, o, clampi(q, lo, hi));
                }
}

/* QLinearConcat_operator (QLinearConcat.cpp:70-104 requantize_chunk, :119-166
 * NCHW, :170-236 NHWC): y is `outer` rows of the inputs' chunks side by side
 * (chunk t = count[t] elements). An input with the output's scale and zero
 * point is copied; otherwise each chunk is requantized with rs = fl(x_s / y_s):
 * its first count - count % 16 elements (when count >= 16) by the 16-wide
 * body, q = rne(clamp(fma(rs, fl(x - x_zp), y_zp), lo, hi)), the rest by the
 * scalar tail, q = clamp(nearbyint(fl(rs * (x - x_zp)) + y_zp)). */
void orc_qlinear_concat(int ntens, const void* const* xs, const long long* count, long long outer, int dt,
                        const float* x_s, const int* x_zp, float y_s, int y_zp, void* y) {
    int lo, hi; dtype_range(dt, &lo, &hi);
    long long row = 0;
    for (int t = 0; t < ntens; t++) row += count[t];
    for (long long o = 0; o < outer; o++) {
        long long yoff = o * row;
        for (int t = 0; t < ntens; t++) {
            const long long cnt = count[t];
            const size_t src = (size_t)(o * cnt);
            const int same = x_s[t] == y_s && x_zp[t] == y_zp;           /* :147 */
            const float rs = same ? 0.f : x_s[t] / y_s;
            const long long body = cnt >= 16 ? cnt - cnt % 16 : 0;
            for (long long i = 0; i < cnt; i++) {
                int32_t xv = ld_q(xs[t], dt, src + (size_t)i);
                int q;
                if (same) q = xv;
                else if (i < body) {                                        /* :84-100 */
                    float v = fmaf(rs, (float)xv - (float)x_zp[t], (float)y_zp);
                    v = v > (float)lo ? v : (float)lo;
                    v = v < (float)hi ? v : (float)hi;
                    q = (int)rintf(v);
                } else {                                                    /* :101-104 */
                    float v = mul_add_expr(rs, (float)(xv - x_zp[t]), (float)y_zp);
                    q = clampi(x86_f2i(nearbyintf(v)), lo, hi);
                }
                st_q(y, dt, (size_t)(yoff + i), q);
            }
            yoff += cnt;
        }
    }
}

/* QLinearMul_operator::exec_typed (QLinearMul.cpp:25-231), AVX-512 build:
 * cs = fl(fl(a_s * b_s) / y_s). kind as QLinearAdd: 0 same shape (16-wide
 * body v = fma(fl(fl(a - a_zp) * fl(b - b_zp)), cs, y_zp), rne, clamp; the
 * last n % 16 by the scalar expression fl(fl(cs * A) * B) + y_zp), 1 B scalar,
 * 2 A scalar (scalar expression with the constant factor fl(cs * (s - zp))),
 * 3 per channel: a is the full tensor, b the [C] one (the caller swaps
 * operands and zero points when A is the per-channel one, as :127-131 do);
 * 16-wide body over channels (NHWC) or over each plane (NCHW). */
void orc_qlinear_mul(int kind, const void* a, const void* b, void* y, size_t n,
                     int N, int C, int HW, int y_nhwc, int dt,
                     float a_s, int a_zp, float b_s, int b_zp, float y_s, int y_zp) {
    int lo, hi; dtype_range(dt, &lo, &hi);
    const float cs = a_s * b_s / y_s;                                       /* :39 */
    const float yz = (float)y_zp;
    if (kind == ORC_ADD_SAME) {
        size_t body = n - n % 16;
        for (size_t i = 0; i < n; i++) {
            int32_t av = ld_q(a, dt, i), bv = ld_q(b, dt, i);
            int q;
            if (i < body) {                                                 /* :54-74 */
                float va = (float)av - (float)a_zp, vb = (float)bv - (float)b_zp;
                float v = fmaf(va * vb, cs, yz);
                v = rintf(v);
                v = clampf_minmax(v, (float)lo, (float)hi);
                q = (int)v;
            } else {                                                        /* :76-79 */
                float t1 = cs * (float)(av - a_zp);
                float v = mul_add_expr(t1, (float)(bv - b_zp), yz);
                q = clampi(x86_f2i(nearbyintf(v)), lo, hi);
            }
            st_q(y, dt, i, q);
        }
        return;
    }
    if (kind == ORC_ADD_B_SCALAR || kind == ORC_ADD_A_SCALAR) {            /* :88-99 */
        const int b_sc = kind == ORC_ADD_B_SCALAR;
        const float cval = b_sc ? cs * (float)(ld_q(b, dt, 0) - b_zp) : cs * (float)(ld_q(a, dt, 0) - a_zp);
        for (size_t i = 0; i < n; i++) {
            float d = b_sc ? (float)(ld_q(a, dt, i) - a_zp) : (float)(ld_q(b, dt, i) - b_zp);
            float v = mul_add_expr(cval, d, yz);
            st_q(y, dt, i, clampi(x86_f2i(nearbyintf(v)), lo, hi));
        }
        return;
    }
    /* per channel: a full, b [C] */
    if (y_nhwc) {                                                           /* :138-177 */
        for (size_t pos = 0; pos < (size_t)N * HW; pos++) {
            const int cbody = C - C % 16;
            for (int c = 0; c < C; c++) {
                const float cv = cs * (float)(ld_q(b, dt, c) - b_zp);
                const size_t i = pos * C + c;
                int32_t xv = ld_q(a, dt, i);
                int q;
                if (c < cbody) {
                    float v = fmaf((float)xv - (float)a_zp, cv, yz);
                    v = rintf(v);
                    q = (int)clampf_minmax(v, (float)lo, (float)hi);
                } else {
                    float v = mul_add_expr(cv, (float)(xv - a_zp), yz);
                    q = clampi(x86_f2i(nearbyintf(v)), lo, hi);
                }
                st_q(y, dt, i, q);
            }
        }
        return;
    }
    for (size_t nc = 0; nc < (size_t)N * C; nc++) {                        /* :180-200 */
        const int c = (int)(nc % (size_t)C);
        const float bval = cs * (float)(ld_q(b, dt, c) - b_zp);
        const int body = HW - HW % 16;
        for (int i = 0; i < HW; i++) {
            const size_t k = nc * HW + i;
            int32_t xv = ld_q(a, dt, k);
            int q;
            if (i < body) {
                float v = fmaf((float)xv - (float)a_zp, bval, yz);
                v = rintf(v);
                q = (int)clampf_minmax(v, (float)lo, (float)hi);
            } else {
                float v = mul_add_expr(bval, (float)(xv - a_zp), yz);
                q = clampi(x86_f2i(nearbyintf(v)), lo, hi);
            }
            st_q(y, dt, k, q);
        }
    }
}

void orc_maxpool_u8_nhwc(const uint8_t* x, uint8_t* y, int N, int C, int iH,
                         int iW, int oH, int oW, int kH, int kW, int sH, int sW,
                         int pH, int pW) {
    #pragma omp parallel for schedule(static) num_threads(orc_get_threads())
    for (long long r = 0; r < (long long)N * oH; r++) {
        int n = (int)(r / oH), oh = (int)(r % oH);
        int ih0 = oh * sH - pH;
        int kh0 = ih0 < 0 ? -ih0 : 0, kh1 = kH < iH - ih0 ? kH : iH - ih0;
        for (int ow = 0; ow < oW; ow++) {
            int iw0 = ow * sW - pW;
            int kw0 = iw0 < 0 ? -iw0 : 0, kw1 = kW < iW - iw0 ? kW : iW - iw0;
            for (int c = 0; c < C; c++) {
                uint8_t m = 0;
                for (int a = kh0; a < kh1; a++)
                    for (int b = kw0; b < kw1; b++) {
                        uint8_t v = x[(((size_t)n * iH + ih0 + a) * iW + (iw0 + b)) * C + c];
                        if (v > m) m = v;
                    }
                y[(((size_t)n * oH + oh) * oW + ow) * C + c] = m;
            }
        }
    }
}

void orc_nchw_to_nhwc_u8(const uint8_t* x, uint8_t* y, int N, int C, int HW) {
    for (int n = 0; n < N; n++)
        for (int c = 0; c < C; c++)
            for (int s = 0; s < HW; s++)
                y[((size_t)n * HW + s) * C + c] = x[((size_t)n * C + c) * HW + s];
}

/* fold_bn_qdq (src/graph_optimizer/fold_bn_qdq.cpp:138-147, :230-236), the
 * combined per-channel scale and offset, in float with the reference's
 * expression order:
 *   gamma = sc / sqrtf(var + eps), beta = bias - gamma * mean
 *   DQ -> BN -> Q (has_dq): A = dq_s * gamma / q_s,
 *                           B = (beta - dq_zp * dq_s * gamma) / q_s + q_zp
 *   BN -> Q:                A = gamma / q_s,  B = beta / q_s + q_zp       */
void orc_fold_bn(int C, const float* sc, const float* bias, const float* mean, const float* var, float eps,
                 int has_dq, float dq_s, int dq_zp, float q_s, int q_zp, float* A, float* B) {
    for (int c = 0; c < C; ++c) {
        const float gamma = sc[c] / sqrtf(var[c] + eps);
        const float beta = bias[c] - gamma * mean[c];
        if (has_dq) {
            A[c] = dq_s * gamma / q_s;
            B[c] = (beta - (float)dq_zp * dq_s * gamma) / q_s + (float)q_zp;
        } else {
            A[c] = gamma / q_s;
            B[c] = beta / q_s + (float)q_zp;
        }
    }
}

/* BatchNormalization's folded execution (BatchNormalization.cpp:248-376 and
 * ops_x64.h:110-155, AVX-512 build): y = uint8(A[c] * x + B[c]).
 *   NCHW: per (n, c) plane, the first HW - HW%16 elements 16 wide:
 *         fma(x, a, b), _mm512_max_ps(_mm512_min_ps(v, 255), 0),
 *         cvtps_epi32 (nearest even), cvtusepi32_epi8; the rest
 *         std::max(0, std::min(255, x * a + b)), roundf.
 *   NHWC: per pixel, the first C - C%16 channels 16 wide: fma(x, A, B)
 *         (clamped as above only for fp32 input), cvtps_epi32, then
 *         cvtusepi32_epi8, an UNSIGNED saturation (a negative int32 is a
 *         large unsigned value and becomes 255); the rest
 *         std::max(0, std::min(255, A * x + B)), lrintf.
 * x: uint8, or fp32 when x_f32. */
static inline float simd_clamp255(float v) {
    const float m = v < 255.0f ? v : 255.0f;   /* minps(v, 255): NaN -> 255 */
    return m > 0.0f ? m : 0.0f;
}
static inline float std_clamp255(float v) {
    const float m = v < 255.0f ? v : 255.0f;   /* std::min(255.0f, v) */
    return 0.0f < m ? m : 0.0f;                /* std::max(0.0f, m) */
}
static inline uint8_t cvtus_epi8(int32_t r) {
    return (uint32_t)r > 255u ? 255 : (uint8_t)r;
}

void orc_batchnorm_u8(const void* x, int x_f32, uint8_t* y, const float* A, const float* B, long long N, int C,
                      long long HW, int nhwc) {
    const uint8_t* xu = (const uint8_t*)x;
    const float* xf = (const float*)x;
#define XV(i) (x_f32 ? xf[i] : (float)xu[i])
    if (nhwc) {
        const int body = C - C % 16;
        for (long long p = 0; p < N * HW; ++p) {
            const long long o = p * C;
            for (int c = 0; c < C; ++c) {
                const float v0 = XV(o + c);
                if (c < body) {
                    float v = fmaf(v0, A[c], B[c]);
                    if (x_f32) v = simd_clamp255(v);
                    y[o + c] = cvtus_epi8(x86_f2i(nearbyintf(v)));
                } else {
                    y[o + c] = (uint8_t)lrintf(std_clamp255(A[c] * v0 + B[c]));
                }
            }
        }
    } else {
        const long long body = HW - HW % 16;
        for (long long nc = 0; nc < N * C; ++nc) {
            const int c = (int)(nc % C);
            const long long o = nc * HW;
            for (long long i = 0; i < HW; ++i) {
                const float v0 = XV(o + i);
                if (i < body)
                    y[o + i] = cvtus_epi8(x86_f2i(nearbyintf(simd_clamp255(fmaf(v0, A[c], B[c])))));
                else
                    y[o + i] = (uint8_t)roundf(std_clamp255(v0 * A[c] + B[c]));
            }
        }
    }
#undef XV
}

/* ConvInteger, 4-D (ConvInteger.cpp:236-354, the integer loops; the 4-D
 * float im2col path :146-233 gives the same values while every partial sum
 * is exact in float): y[n][oc][oh][ow] = sum (x - x_zp)(w - w_zp[oc]) over
 * in-image taps, int32 with wrap-around. wzp: int32 [OC]. */
void orc_conv_integer(const void* x, int x_dt, const void* w, int w_dt, int x_zp, const int32_t* wzp, int N, int C,
                      int iH, int iW, int OC, int kH, int kW, int sH, int sW, int pH, int pW, int dH, int dW, int oH,
                      int oW, int group, int32_t* y) {
    const int CC = C / group, MM = OC / group;
    if (g_vnni && group == 1 && w_dt) {
        /* the same values from the AVX-512 VNNI convolution: acc = sum
         * (x - x_zp) w over in-image taps, then y = acc - w_zp[oc] S with
         * S = sum (x - x_zp) over the output pixel's in-image taps */
        orc_conv_params p;
        memset(&p, 0, sizeof p);
        p.N = N; p.C = C; p.H = iH; p.W = iW; p.OC = OC; p.kH = kH; p.kW = kW; p.group = 1;
        p.sH = sH; p.sW = sW; p.dH = dH; p.dW = dW; p.pad_t = p.pad_b = pH; p.pad_l = p.pad_r = pW;
        p.oH = oH; p.oW = oW; p.act_dtype = x_dt ? ORC_S8 : ORC_U8; p.x_zp = x_zp;
        if (orc_vnni_conv_acc(&p, x, (const int8_t*)w, y) == 0) {
            #pragma omp parallel for schedule(static) num_threads(orc_get_threads())
            for (int n = 0; n < N; ++n) {
                int32_t* xs = (int32_t*)malloc(sizeof(int32_t) * (size_t)iH * iW);
                for (int i = 0; i < iH * iW; ++i) xs[i] = 0;
                for (int c = 0; c < C; ++c)
                    for (int i = 0; i < iH * iW; ++i)
                        xs[i] += (x_dt ? (int)((const int8_t*)x)[((size_t)n * C + c) * iH * iW + i]
                                       : (int)((const uint8_t*)x)[((size_t)n * C + c) * iH * iW + i]) - x_zp;
                for (int oh = 0; oh < oH; ++oh)
                    for (int ow = 0; ow < oW; ++ow) {
                        int32_t s = 0;
                        for (int kh = 0; kh < kH; ++kh) {
                            const int ih = oh * sH - pH + kh * dH;
                            if (ih < 0 || ih >= iH) continue;
                            for (int kw = 0; kw < kW; ++kw) {
                                const int iw = ow * sW - pW + kw * dW;
                                if (iw >= 0 && iw < iW) s += xs[ih * iW + iw];
                            }
                        }
                        for (int oc = 0; oc < OC; ++oc)
                            y[(((size_t)n * OC + oc) * oH + oh) * oW + ow] -=
                                (int32_t)((uint32_t)wzp[oc] * (uint32_t)s);
                    }
                free(xs);
            }
            return;
        }
    }
#define LX(i) (x_dt ? (int)((const int8_t*)x)[i] : (int)((const uint8_t*)x)[i])
#define LW(i) (w_dt ? (int)((const int8_t*)w)[i] : (int)((const uint8_t*)w)[i])
    for (int n = 0; n < N; ++n)
        for (int oc = 0; oc < OC; ++oc) {
            const int g = oc / MM;
            for (int oh = 0; oh < oH; ++oh)
                for (int ow = 0; ow < oW; ++ow) {
                    uint32_t sum = 0;
                    for (int c = 0; c < CC; ++c)
                        for (int kh = 0; kh < kH; ++kh) {
                            const int ih = oh * sH - pH + kh * dH;
                            if (ih < 0 || ih >= iH) continue;
                            for (int kw = 0; kw < kW; ++kw) {
                                const int iw = ow * sW - pW + kw * dW;
                                if (iw < 0 || iw >= iW) continue;
                                const int xv = LX((((size_t)n * C + g * CC + c) * iH + ih) * iW + iw) - x_zp;
                                const int wv = LW((((size_t)oc * CC + c) * kH + kh) * kW + kw) - wzp[oc];
                                sum += (uint32_t)xv * (uint32_t)wv;
                            }
                        }
                    y[(((size_t)n * OC + oc) * oH + oh) * oW + ow] = (int32_t)sum;
                }
        }
#undef LX
#undef LW
}
