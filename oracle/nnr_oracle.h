/*
 * nnr_oracle.h -- CPU restatement of NNR's int8 QDQ compute path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the
 * HIP backend in nnr_amd/. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product path never does.
 *
 * Every function restates the arithmetic of a file in the reference
 * (paths relative to the reference root, cited per function in
 * nnr_oracle.c). Conventions:
 *   - int32 accumulators are exact sum (x - x_zp)(w - w_zp) modulo 2^32;
 *   - float arithmetic is IEEE binary32 with round-to-nearest-even and NO
 *     implicit contraction (compiled with -ffp-contract=off); explicit
 *     fmaf() sits exactly where the reference uses _mm512_fmadd_ps;
 *   - the reference's scalar-tail C++ expressions (a*b + c) can contract to
 *     FMA under GCC/Clang; orc_set_contract(1) switches those sites to fmaf
 *     (documented variant, default off = MSVC semantics).
 */
#ifndef NNR_ORACLE_H
#define NNR_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- configuration -------------------------------------------------- */
/* 1: conv / matmul accumulators through the AVX-512 VNNI restatement of
 * nnr_vnni.c (the CPU baseline; same exact int32 values), when the host has
 * AVX-512 VNNI; 0 (default): the scalar loops */
void orc_set_vnni(int on);
int orc_get_vnni(void);
void orc_set_contract(int on);
int  orc_get_contract(void);

/* ---- fp16 helpers (src/nnrconf.h:147-199 semantics) ------------------ */
uint16_t orc_f32_to_f16(float v);
float    orc_f16_to_f32(uint16_t v);

/* ---- requantize primitives (one output element each) ----------------- */
/* RQ-A : clamp(fl(rne(fl(fma(acc,cs,bf)*inv_y)) + y_zp), L, hi)          */
int orc_rq_a(int32_t acc, float cs, float bf, float inv_y, int y_zp, int L, int hi);
/* RQ-A': clamp(nearbyint(fl(v*inv_y)) + y_zp, L, hi), v = acc*cs + bf     */
int orc_rq_a_tail(int32_t acc, float cs, float bf, float inv_y, int y_zp, int L, int hi);
/* RQ-B : v = acc+bias (wrap); f = clamp(fl(v*os), lo-yzp, hi-yzp); rne(f)+yzp */
int orc_rq_b(int32_t acc, int32_t bias, float os, int y_zp, int lo, int hi);
/* RQ-B': as RQ-B with roundf (half away from zero)                       */
int orc_rq_b_roundf(int32_t acc, int32_t bias, float os, int y_zp, int lo, int hi);
/* RQ-C : rne(clamp(fma(fma(acc,cs,bf), inv_y, y_zp), qmin, qmax))        */
int orc_rq_c(int32_t acc, float cs, float bf, float inv_y, int y_zp, int qmin, int qmax);
/* RQ-D : clamp(nearbyint(acc*cm + y_zp), lo, hi)                         */
int orc_rq_d(int32_t acc, float cm, int y_zp, int lo, int hi);

/* ---- tensor element types ------------------------------------------- */
enum orc_dtype { ORC_U8 = 0, ORC_S8 = 1, ORC_I32 = 2, ORC_F32 = 3, ORC_F16 = 4 };

/* ---- QuantizeLinear (per-tensor) ------------------------------------- */
void orc_quantize_linear(const float* x, size_t n, float scale, int zp,
                         int y_dtype, void* y);
/* ---- DequantizeLinear (per-tensor) ----------------------------------- */
/* HardSwish fp32 (HardSwish.cpp:18-50); post_op: fused form (zero bias added) */
void orc_hardswish_f32(const float* x, float* y, size_t n, int post_op);
void orc_dequantize_linear(const void* x, int x_dtype, size_t n, float scale,
                           int zp, float* y);
/* ---- DynamicQuantizeLinear ------------------------------------------- */
void orc_dynamic_quantize_linear(const float* x, size_t n, uint8_t* y,
                                 float* y_scale, uint8_t* y_zp);

/* ---- QLinearMatMul ---------------------------------------------------- */
/* a: [batch_a, m, k] (batch_a is 1 or batch), b: [batch_b, k, n],
 * y: [batch, m, n]. Scales given as raw pointers of scale_dtype (F32/F16).
 * Batch offsets follow the reference's flat rule (QLinearMatMul.cpp:156). */
int orc_qlinear_matmul(int batch, int m, int n, int k,
                       const void* a, int a_dtype, int batch_a,
                       const void* a_scale, const void* a_zp,
                       const void* b, int b_dtype, int batch_b,
                       const void* b_scale, const void* b_zp,
                       const void* y_scale, const void* y_zp,
                       int scale_dtype, void* y, int y_dtype);
/* combined scale of RQ-D (QLinearMatMul.cpp:124-135) */
float orc_qmatmul_combined_scale(const void* a_s, const void* b_s,
                                 const void* y_s, int scale_dtype);

/* ---- MatMulInteger ---------------------------------------------------- */
/* Full numpy-style broadcasting over leading dims (nd <= 6).           */
int orc_matmul_integer(const int* a_dims, int a_nd, const void* a, int a_dtype,
                       const int* b_dims, int b_nd, const void* b, int b_dtype,
                       int a_zp, int b_zp, int32_t* y);

/* ---- QLinearConv (4-D) ----------------------------------------------- */
typedef struct orc_conv_params {
    int N, C, H, W;                 /* input, logical NCHW              */
    int OC, kH, kW, group;          /* weights [OC, C/group, kH, kW]    */
    int sH, sW, dH, dW;
    int pad_t, pad_l, pad_b, pad_r; /* resolved pads (cpads)            */
    int oH, oW;
    int x_nhwc, y_nhwc;             /* physical layout flags            */
    int post_fn;                    /* a unary op was fused (post_fn)   */
    int act_dtype;                  /* ORC_U8 or ORC_S8 (x and y)       */
    float x_scale; int x_zp;
    const float* w_scale; int w_scale_count;
    const int8_t* w_zp; int w_zp_count;
    float y_scale; int y_zp;
    const int32_t* bias;            /* NULL if absent                   */
    int vnni;                       /* 1: x64 AVX-512 VNNI host         */
} orc_conv_params;

/* kernel branch chosen by QLinearConv::exec_simd_4d (QLinearConv.cpp:1337) */
enum orc_conv_branch {
    ORC_BR_DW = 1,          /* exec_dw_int8_nhwc           RQ-A, [lo,hi]     */
    ORC_BR_FIRST = 2,       /* exec_first_layer_int8       RQ-C (+RQ-A')     */
    ORC_BR_DIRECT = 3,      /* exec_direct_int8            RQ-A qmin (+A')   */
    ORC_BR_PACKED = 4,      /* exec_packed_nr48, NR48      RQ-B (+B')        */
    ORC_BR_NR16 = 5,        /* exec_packed_nr48, NR16      RQ-B              */
    ORC_BR_IM2COL_S1 = 6,   /* exec_vnni_im2col fused      RQ-A, [lo,hi]     */
    ORC_BR_IM2COL = 7,      /* exec_vnni_im2col tiled      RQ-A qmin (+A')   */
    ORC_BR_FLOAT = 8,       /* exec_float_fallback         RQ-A qmin (+A')   */
    ORC_BR_TYPED = 9        /* exec_typed, 3-D tensors     RQ-S              */
};

/* output spatial size (conv_shape.h:21-81, NOTSET / explicit pads) */
int orc_conv_out_dim(int in, int k, int d, int s, int pb, int pe);
int orc_conv_dispatch(const orc_conv_params* p);
/* exact accumulators, laid out [N][OC][oH][oW] */
void orc_conv_acc(const orc_conv_params* p, const void* x, const int8_t* w,
                  int32_t* acc);
/* full op: returns the branch id, writes y in the layout y_nhwc selects */
int orc_qlinear_conv(const orc_conv_params* p, const void* x, const int8_t* w,
                     void* y);
/* 1-D convolution on 3-D tensors (exec_typed, RQ-S); H == kH == 1 */
int orc_qlinear_conv1d(const orc_conv_params* p, const void* x, const int8_t* w, void* y);
/* same, given precomputed accumulators (lets tests reuse one acc array) */
int orc_qlinear_conv_from_acc(const orc_conv_params* p, const int32_t* acc,
                              void* y);

/* ---- QLinearAdd -------------------------------------------------------- */
/* kind: 0 SAME_SHAPE, 1 B scalar, 2 A scalar, 3 per-channel B[C] on y[N,C,H,W] */
enum { ORC_ADD_SAME = 0, ORC_ADD_B_SCALAR = 1, ORC_ADD_A_SCALAR = 2, ORC_ADD_PER_CHANNEL = 3 };
void orc_qlinear_add(int kind, const void* a, const void* b, void* y, size_t n,
                     int N, int C, int HW, int y_nhwc, int dtype,
                     float a_s, int a_zp, float b_s, int b_zp, float y_s, int y_zp);

/* ---- MaxPool, uint8 NHWC (x64/pool_x64.h:396-436) ---------------------- */
/* QLinearGlobalAveragePool / QLinearAveragePool / QLinearConcat / QLinearMul */
void orc_qlinear_global_avgpool(const void* x, void* y, int N, int C, int spatial, int x_nhwc, int dt,
                                float x_s, int x_zp, float y_s, int y_zp);
void orc_qlinear_avgpool(const void* x, void* y, int N, int C, int iH, int iW, int oH, int oW,
                         int kH, int kW, int sH, int sW, int pH, int pW, int nhwc, int dt,
                         float x_s, int x_zp, float y_s, int y_zp);
void orc_qlinear_concat(int ntens, const void* const* xs, const long long* count, long long outer, int dt,
                        const float* x_s, const int* x_zp, float y_s, int y_zp, void* y);
void orc_qlinear_mul(int kind, const void* a, const void* b, void* y, size_t n,
                     int N, int C, int HW, int y_nhwc, int dt,
                     float a_s, int a_zp, float b_s, int b_zp, float y_s, int y_zp);
void orc_maxpool_u8_nhwc(const uint8_t* x, uint8_t* y, int N, int C, int iH,
                         int iW, int oH, int oW, int kH, int kW, int sH, int sW,
                         int pH, int pW);

/* ---- layout helper ------------------------------------------------------ */
void orc_nchw_to_nhwc_u8(const uint8_t* x, uint8_t* y, int N, int C, int HW);

/* ---- threading for the CPU baseline (0 = OpenMP default) ---------------- */
void orc_set_threads(int n);
int  orc_get_threads(void);


/* fold_bn_qdq's combined per-channel A / B (fold_bn_qdq.cpp:138-147, 230-236) */
void orc_fold_bn(int C, const float* sc, const float* bias, const float* mean, const float* var, float eps,
                 int has_dq, float dq_s, int dq_zp, float q_s, int q_zp, float* A, float* B);
/* folded BatchNormalization execution (BatchNormalization.cpp:248-376) */
void orc_batchnorm_u8(const void* x, int x_f32, uint8_t* y, const float* A, const float* B, long long N, int C,
                      long long HW, int nhwc);

/* ConvInteger, 4-D (ConvInteger.cpp:146-354), exact int32 */
void orc_conv_integer(const void* x, int x_dt, const void* w, int w_dt, int x_zp, const int32_t* wzp, int N, int C,
                      int iH, int iW, int OC, int kH, int kW, int sH, int sW, int pH, int pW, int dH, int dW, int oH,
                      int oW, int group, int32_t* y);

/* ---- AVX-512 VNNI restatement (nnr_vnni.c) -------------------------- */
int orc_vnni_available(void);
/* physical cores / logical threads for int8_compute_threads (0: detect) */
void orc_set_host_threads(int physical, int logical);
int orc_int8_compute_threads(int work_items, long long total_ops);
/* 1: keep packed weights across calls (keyed by address, shape and a hash
 * of the bytes), as the reference packs once in reshape(); 0: pack per
 * call. Either call drops the cache. */
void orc_vnni_cache(int on);
/* group-1 convolution; -1 when not applicable (no VNNI, groups, per-channel
 * w_zp): exact accumulators [N][OC][oH][oW] as orc_conv_acc */
int orc_vnni_conv_acc(const orc_conv_params* p, const void* x, const int8_t* w, int32_t* acc);
/* acc_nhwc: accumulators [N][oH][oW][OC] (the GEMM's own row-major order) */
int orc_vnni_conv_acc_layout(const orc_conv_params* p, const void* x, const int8_t* w, int32_t* acc,
                             int acc_nhwc);
/* depthwise on NHWC input, 16 channels per vector (vpmulld) */
int orc_vnni_depthwise_acc(const orc_conv_params* p, const void* x, const int8_t* w, int32_t* acc);
/* y[b][m][n] = sum_k (a - a_zp)(b - b_zp); A [batch] x [m][k] at a_bstride,
 * B [k][n] shared */
int orc_vnni_matmul_integer(int batch, int m, int n, int k, const void* a, int a_dtype, long long a_bstride,
                            const void* b, int b_dtype, int a_zp, int b_zp, int32_t* y);

#ifdef __cplusplus
}
#endif
#endif
