// nnrh_internal.h -- shared declarations between the HIP kernel files and
// the C-ABI layer (capi.cpp). Not installed; the public surface is
// include/nnr_hip.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace nnrh {

// ---------------------------------------------------------------------------
// Requantize epilogue selectors for the MFMA GEMM kernel.
enum EpiMode : int {
    EPI_I32 = 0,   // store the exact int32 accumulator (MatMulInteger)
    EPI_RQA = 1,   // fma(acc,cs,bf) * inv_y, rne, +y_zp, clamp [L,hi]
    EPI_RQB = 2,   // (acc+bias)*os, clamp [lo-zp,hi-zp], rne, +zp
    EPI_RQC = 3,   // fma(fma(acc,cs,bf), inv_y, zp), clamp, rne
    EPI_RQD = 4,   // acc*cm + zp, nearbyint, clamp
    EPI_I32S = 5,  // fp32 fl(float(acc) * fl(a_s * cs[n])) (+ bias): MatMulInteger
                   // -> Cast -> Mul by the per-column scale product (-> Add)
};

// Which output elements take the reference's scalar-tail expression (RQ-A')
// instead of the SIMD body (RQ-A / RQ-C).
enum TailMode : int {
    TAIL_NONE = 0,
    TAIL_SPATIAL = 1,   // s = pixel index in image; tail when s >= sp - sp%16
    TAIL_OW = 2,        // tail when ow >= oW - oW%16
    TAIL_TILED = 3,     // tiled im2col: tiles of tile_h rows, tail per tile
};

// A-operand (activation) addressing.
enum AMode : int {
    A_DENSE = 0,   // A[m*lda + k]
    A_CONV = 1,    // implicit im2col over an NHWC tensor, K order (kh,kw,c)
    A_CONV4 = 2,   // first layer: NHWC with 4 channels, K order (kh, kw < kWp, c)
    A_CONVU = 3,   // A_CONV with C % 64 == 0 and kH*kW <= 32: every 64-byte K step
                   // lies in one tap, so the tap walk is uniform across the block
};

struct GemmArgs {
    // ---- A (activations) ----
    const uint8_t* a;     // dense matrix or NHWC tensor base
    long long lda;        // dense row stride (bytes)
    long long a_bstride;  // per-batch stride (blockIdx.z)
    int a_xor;            // 0x80 for uint8 activations (x-128), 0 for int8
    int M, N, K, Kp;      // K real, Kp = K rounded up to 64 (packed B row length)
    // conv geometry (A_CONV)
    int H, W, C, oH, oW, kH, kW, sH, sW, dH, dW, pad_t, pad_l;
    int Cs;               // channel stride of the NHWC tensor (>= C; groups)
    int kWp;              // > 0: first-layer layout (kW padded to a multiple of 4)
    int pad_byte;         // raw byte for out-of-image taps (x_zp)
    // ---- B (weights), packed [Np][Kp] int8 with the 64-column permutation ----
    const int8_t* b;
    long long b_bstride;
    int Np;
    // ---- zero-point corrections: v = acc' - alpha*colsum[n] - beta*rowsum[m]
    // alpha = x_zp - a_sub (a_sub = 128 for uint8 activations, else 0); when
    // alpha_zp_dev is set the activation zero point is read from device memory.
    const int32_t* colsum;
    const int32_t* c0;    // per-column constant: bias(RQ-B) - alpha*colsum; NULL:
                          // computed from colsum/bias/alpha in the epilogue
    int alpha;
    const void* alpha_zp_dev;  // nullable: uint8 (a_xor) or int8 zero point
    int a_sub;
    const int32_t* rowsum;  // nullable
    long long rowsum_bstride;
    int beta;
    const int32_t* beta_col;  // nullable: per-column beta (per-channel w_zp)
    // pipelined kernel, EPI_I32 of a convolution only: v = acc' + row_coef[n] *
    // sum_k (a[m][k] - (alpha + a_sub)) (int32 wrap-around), the row sum over
    // the Kp bytes of im2col row m (padding reads pad_byte, which must be the
    // zero point alpha + a_sub) taken from the A fragments in the kernel
    const int32_t* row_coef;
    // ---- epilogue ----
    int epi;
    int tail;
    int tile_h;             // TAIL_TILED
    const float* os;        // RQ-B
    const int32_t* bias;    // RQ-B (nullable)
    const float* cs;        // RQ-A / RQ-C
    const float* bf;        // RQ-A / RQ-C
    long long param_bstride;  // per-batch (z) offset of every per-column array
                              // (colsum, c0, beta_col, os, bias, cs, bf); all
                              // per-column arrays are padded to Np entries
    float inv_y;
    float cm;               // RQ-D combined scale fl(fl(a_s*b_s)/y_s);
                            // EPI_I32S: the host activation scale a_s
    const float* cm_a_scale_dev;  // RQ-D: nullable device a_scale; then
    float cm_b, cm_y;             //   cm = fl(fl(a_s*cm_b)/cm_y) in-kernel
    int y_zp;
    int L, hi, lo;          // clamp bounds
    int bprime_from;        // RQ-B: columns >= this use roundf (RQ-B')
    // ---- output ----
    void* y;
    long long ldy;          // row stride in elements (NHWC / row-major);
                            // with y_nchw: total channel count of y
    long long y_bstride;    // per-batch stride in elements
    int y_type;             // 0 u8, 1 s8, 2 i32
    int y_nchw;             // 1: scatter to NCHW [img][n][s] (s = m % (oH*oW))
    int nbatch;             // batch count (set by the launcher)
    // first layer on the pipelined kernel (kWp > 0, copy_stride > 0): A is the
    // padded multi-copy NHWC4 image of launch_first_layer_copies; H/W are its
    // padded height / row length and the pads are already applied
    int copy_shift;
    long long copy_stride;  // bytes per copy
    // max |c0[n]| (host); the pipelined kernel starts its int32 accumulators
    // at c0 when 128*128*K + c0_absmax cannot overflow
    long long c0_absmax;
    // n / d for n < 2^31 as (n * mul) >> (31 + shift) (set by the launcher)
    uint32_t div_sp_mul, div_sp_shift, div_ow_mul, div_ow_shift;
    // tile index -> (z, m-block, n-block) (set by the pipelined launcher)
    uint32_t div_pz_mul, div_pz_shift, div_nbn_mul, div_nbn_shift;
    // QLinearAdd (same shape) fused into the RQ-B epilogue: the conv byte q
    // and the residual byte r of the same NHWC element are A and B of the
    // add (or B and A), requantized with RQ-E. Flat element index >=
    // add_body takes the scalar-tail expression.
    // DequantizeLinear + per-column fp32 bias fused after RQ-D: y is float,
    // y = fl(fl((q - dq_zp) * dq_scale) + dq_bias[n]) with dq_zp = y_zp
    const float* dq_bias;       // NULL: no fused dequantize (padded to Np)
    float dq_scale;
    int dq_gelu;                // then Gelu (erf form) of the fp32 value
    int dq_nobias;              // EPI_I32S: no bias Add in the fused chain
    // fused dequantize: (min, max) of each (tile, wave)'s outputs, pair
    // 4 * tile + wave, for a DynamicQuantizeLinear that reads y (NULL: none)
    float* mm_parts;
    // fused dequantize: y receives the uint8 QLinearMatMul bytes (same
    // element strides) instead of the fp32 values, which the reader forms
    // from them per column; the values still feed mm_parts when it is set
    int dq_codes;
    // grouped fused-dequantize launch (QLinearMatMuls sharing A): batch index
    // z is the member, with its own combined scale, zero point, dequantize
    // scale and output; B and the per-column arrays advance by b_bstride /
    // param_bstride, A is shared (a_bstride 0). ngrp = 0: not grouped
    int ngrp;
    float grp_cm[4], grp_cm_b[4], grp_cm_y[4], grp_dq_scale[4];
    int grp_y_zp[4];
    void* grp_y[4];
    const uint8_t* add_other;   // NULL: no fused add
    int add_conv_is_a;
    float add_sa, add_sb, add_fixed;
    int add_a_zp, add_b_zp, add_y_zp;
    long long add_body;
};

// Multiply-shift constants of an unsigned division by d >= 1 for dividends
// n < 2^31: s = ceil(log2 d), mul = ceil(2^(31+s) / d) < 2^32, and
// floor(n / d) = (n * mul) >> (31 + s), since the rounding error of mul is
// below d and n * (mul * d - 2^(31+s)) < 2^(31+s).
inline void fast_div_consts(uint32_t d, uint32_t* mul, uint32_t* shift) {
    uint32_t s = 0;
    while ((1ull << s) < d) ++s;
    const unsigned long long p = 1ull << (31 + s);
    *mul = (uint32_t)((p + d - 1) / d);
    *shift = s;
}
__device__ __forceinline__ uint32_t fast_div(uint32_t n, uint32_t mul, uint32_t shift) {
    return (uint32_t)(((unsigned long long)n * mul) >> (31 + shift));
}

// Tile shapes available to the launcher (BM x BN, 256 threads).
// TILE_256x128: 8 waves (512 threads), pipelined kernel only (the register-
// staged kernel runs it as 128x128)
// the launch profiler (nnrh_profile_*): whether it records, and a count of
// one launch of a kernel instantiation under `name` ("variant:...")
bool prof_enabled();
void prof_count(const char* name);

enum TileCfg : int { TILE_128x128 = 0, TILE_256x64 = 1, TILE_64x256 = 2, TILE_256x128 = 3 };

hipError_t launch_qgemm(const GemmArgs& g, int batch, int tile, int vec,
                        hipStream_t s);
// pipelined direct-to-LDS variant (nnrh_qgemm_dma.hip) and its eligibility
bool qgemm_dma_eligible(const GemmArgs& g, int vec);
hipError_t launch_qgemm_dma(const GemmArgs& g, int batch, int tile, hipStream_t s);
// barrier-free short-K kernel (nnrh_qgemm_dma.hip): dense A, Kp = 64, RQ-B
bool qgemm_direct_eligible(const GemmArgs& g, int batch);
hipError_t launch_qgemm_direct(const GemmArgs& g, hipStream_t s);

// ---- first convolution with the input quantize fused (nnrh_stem.hip) ----
// NCHW fp32 (or uint8) image with C <= 4 channels -> NHWC uint8, RQ-C.
struct StemArgs {
    const void* x;          // [N][C][H][W] fp32 or uint8
    const int8_t* w;        // packed weights [64][Kp], K order (kh, kw < 4 * cpr, c < 4)
    const int32_t* c0;      // [64] accumulator start (-(x_zp - 128) * colsum)
    const float* cs;        // [64] RQ-C scale
    const float* bf;        // [64] RQ-C bias term
    uint8_t* y;             // [N][oH][oW][OC]
    int N, C, H, W, oH, oW, kH, sH, sW, pad_t, pad_l;
    int cpr;                // 16-byte K chunks per kernel row (kWp / 4)
    int KS, Kp;             // MFMA K-steps (Kp / 64), packed K
    int OC;                 // output channels (16..64, multiple of 16)
    int L;                  // padded pixels per staged input row
    int R;                  // output rows per group
    int WR;                 // staged rows in the LDS ring
    int strip;              // output rows per block
    int align8;             // fragments as 8-byte LDS reads (even stride and L)
    int sat;                // RQ-C bounds are [0, 255]: one saturating convert
    float inv_y;
    int y_zp, qmin, qmax;
    uint32_t fill;          // the input zero point (pad value), one byte
    // QuantizeLinear of the fp32 input (body / tail split of the whole tensor)
    float q_scale, q_inv;
    int q_zp;
    long long qbody;
    // the 3x3 / stride 2 / padding 1 MaxPool after the conv fused (pool = 1):
    // y is then [N][pH][pW][OC] and strip counts pooled rows (even)
    int pool, pH, pW;
};
bool stem_eligible(const StemArgs& a, bool f32);
hipError_t launch_stem_conv(const StemArgs& a, bool f32, hipStream_t s);

// ---- misc kernels (nnrh_misc.hip) ----
hipError_t launch_nchw_to_nhwc_u8(const uint8_t* x, uint8_t* y, int N, int C,
                                  int HW, int Cpad, uint8_t fill, hipStream_t s);
hipError_t launch_depthwise(const uint8_t* x, const int8_t* w, uint8_t* y,
                            const float* cs, const float* bf, int N, int C,
                            int H, int W, int oH, int oW, int kH, int kW,
                            int sH, int sW, int dH, int dW, int pad_t,
                            int pad_l, int x_zp, int w_zp, float inv_y,
                            int y_zp, int L, int hi, int act_signed,
                            int y_nchw, int tail_mode, int tail_tile_h,
                            hipStream_t s);
// depthwise, NHWC in/out, C % 16 == 0, w_zp 0, at most 12 taps, no tails
// (nnrh_misc.hip); wdot [ceil(taps/4)][C] 4 taps per dword, corr[C]
// 3x3 depthwise, stride 1 or 2, dilation 1, NHWC in and out, C % 8 == 0
hipError_t launch_depthwise3x3(const uint8_t* x, const uint32_t* wrow, const int32_t* corr, uint8_t* y,
                               const float* cs, const float* bf, int N, int C, int H, int W, int oH, int oW,
                               int stride, int pad_t, int pad_l, int x_zp, int a_xor, float inv_y, int y_zp,
                               int L, int hi, hipStream_t s);
hipError_t launch_depthwise16(const uint8_t* x, const uint32_t* wdot, const int32_t* corr,
                              uint8_t* y, const float* cs, const float* bf, int N, int C, int H,
                              int W, int oH, int oW, int kH, int kW, int sH, int sW, int dH, int dW,
                              int pad_t, int pad_l, int x_zp, int a_xor, float inv_y, int y_zp,
                              int L, int hi, hipStream_t s);
hipError_t launch_rowsum_dense(const uint8_t* a, long long lda,
                               long long a_bstride, int M, int K, int a_signed,
                               int a_zp, const void* a_zp_dev, int32_t* out,
                               int batch, hipStream_t s);
hipError_t launch_fill_u8(void* p, uint8_t v, long long n, hipStream_t s);
hipError_t launch_pad_channels_u8(const uint8_t* x, uint8_t* y, long long pixels, int C, int Cpad,
                                  uint8_t fill, hipStream_t s);
hipError_t launch_conv1d_typed(const uint8_t* x, const int8_t* w, const int32_t* wzp, const float* cs,
                               const float* bf, uint8_t* y, int N, int C, int iW, int OC, int G, int kW,
                               int oW, int sW, int dW, int pad_l, int x_zp, int y_zp, float y_scale, int u8,
                               hipStream_t s);
hipError_t launch_quantize_first_layer_copies(const float* x, uint8_t* y, int N, int C, int H, int W,
                                              int Hp, int Wc, int pad_t, int pad_l, int copy_shift,
                                              uint8_t fill, float scale, int zp, hipStream_t s);
hipError_t launch_first_layer_copies(const uint8_t* x, uint8_t* y, int N, int C, int H, int W,
                                     int Hp, int Wc, int pad_t, int pad_l, int copy_shift,
                                     uint8_t fill, hipStream_t s);
// rowsum[z][m] = sum over the patch of pixel m of (x - x_zp), the Cg channels
// of group z starting at channel z * cg_stride; out + z * out_bstride + m
hipError_t launch_rowsum_conv(const uint8_t* x, int N, int H, int W, int Cs,
                              int Cg, int cg_stride, int groups, int oH, int oW, int kH,
                              int kW, int sH, int sW, int dH, int dW,
                              int pad_t, int pad_l, int a_signed, int x_zp,
                              int32_t* out, long long out_bstride, hipStream_t s);
// ConvInteger's per-call preparation, one launch: the NCHW input x to NHWC xs
// with each group's Cg channels padded to Cgp (a multiple of 16) with the fill
// byte, xs[n][p][z * Cgp + c] = c < Cg ? x[n][z * Cg + c][p] : fill; and the
// weights W[G * OCg][Cg][kH][kW] (int8 / uint8) packed to [G][Np][Kp] int8
// (uint8 shifted by 128), K order (kh, kw, c < Cgp), zero padded, with c0[n] =
// -alpha * colsum[n] (alpha = x_zp - a_sub) and row_coef[n] = b_sub - w_zp[oc]
// (w_zp_dev[oc] when given, else w_zp)
struct ConvIntPrepArgs {
    const uint8_t* x;
    uint8_t* xs;
    int N, HW, G, Cg, Cgp;
    uint32_t fill;
    const uint8_t* w;
    int w_u8, OCg, kH, kW, Kp, Np, alpha, w_zp;
    const int32_t* w_zp_dev;
    int8_t* wpack;
    int32_t* c0;
    int32_t* row_coef;
    int copy_blocks, vec;   // set by the launcher
};
hipError_t launch_conv_integer_prep(ConvIntPrepArgs a, hipStream_t s);
// Pack a row-major B[K][N] (int8 or uint8) into the kernel's [Np][Kp]
// permuted layout and compute colsum[n] = sum_k (b - b_sub).
hipError_t launch_pack_b_dense(const void* b, long long b_bstride, int K,
                               int N, int Kp, int Np, int b_xor, int8_t* out,
                               long long out_bstride, int32_t* colsum,
                               long long colsum_bstride, int batch,
                               hipStream_t s);

// Row permutation of packed B inside each 64-column group: storage row of
// logical column n. The MFMA epilogue then sees 16 consecutive columns per
// lane (see nnrh_qgemm.hip).
__host__ __device__ inline int packed_row_of_col(int n) {
    int g = n >> 6, nl = n & 63;
    int tn = (nl & 15) >> 2;
    int j = ((nl >> 4) << 2) | (nl & 3);
    return (g << 6) | (tn << 4) | j;
}

}  // namespace nnrh
