// nnrh_f32.h -- launchers of the fp32 glue kernels (nnrh_f32.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace nnrh {

// A fused QLinearMatMul -> DequantizeLinear -> Add(bias) chain stored as its
// uint8 QLinearMatMul bytes: the fp32 value of byte b in column n is
// fl(fl((b - zp) * scale) + bias[n]), the GEMM epilogue's operations in its
// order (bias padded past the last column, 16-byte aligned)
struct DqCodes {
    const uint8_t* q;
    int zp;
    float scale;
    const float* bias;
};

hipError_t launch_gap_f32(const float* x, float* y, int N, int C, int HW, int x_nhwc,
                          hipStream_t s);
// DequantizeLinear (uint8 or int8, per-tensor) fused into GlobalAveragePool
hipError_t launch_gap_dq(const uint8_t* x, float* y, int N, int C, int HW, int x_nhwc, int x_signed,
                         float scale, int zp, hipStream_t s);
// c_mode: 0 none, 1 scalar, 2 per-column [N], 3 full [M][N], 4 per-row [M]
hipError_t launch_gemm_f32(const float* A, const float* B, const float* C, float* Y, int M, int N,
                           int K, int transA, int transB, float alpha, float beta, int c_mode,
                           hipStream_t s);
// batched: A/B/Y advance by a_bstride/b_bstride/y_bstride elements per batch
// (0: shared); C is the same for every batch
hipError_t launch_gemm_f32_batched(const float* A, const float* B, const float* C, float* Y, int M,
                                   int N, int K, int transA, int transB, float alpha, float beta,
                                   int c_mode, int batch, long long a_bstride, long long b_bstride,
                                   long long y_bstride, hipStream_t s);
// op: 0 add, 1 mul, 2 sub, 3 div; b_mode: 0 same shape, 1 scalar, 2 last-axis
// vector of D; b_first: compute b (op) a
hipError_t launch_binary_f32(const float* a, const float* b, float* y, long long n, int D, int b_mode,
                             int op, int b_first, hipStream_t s);
hipError_t launch_softmax_f32(const float* x, float* y, long long rows, int D, hipStream_t s);
// r (nullable): second same-shape input added first; parts (nullable): one
// (min, max) pair of the outputs per row
hipError_t launch_layernorm_f32(const float* x, const float* r, const float* gamma, const float* beta, float* y,
                                long long rows, int D, float eps, float* parts, hipStream_t s);
// the same with the first input given as chain bytes (columns = the D axis)
hipError_t launch_layernorm_codes_f32(const DqCodes& x, const float* r, const float* gamma, const float* beta,
                                      float* y, long long rows, int D, float eps, float* parts, hipStream_t s);
hipError_t launch_cast_to_f32(const void* x, int dt, float* y, long long n, hipStream_t s);
hipError_t launch_gelu_f32(const float* x, float* y, long long n, hipStream_t s);
hipError_t launch_transpose_f32(const float* x, float* y, int ndim, const int* in_dims, const int* perm,
                                hipStream_t s);
size_t mha_workspace_bytes(int B, int S, int nh);
// the fused head-64 attention kernel's shapes, and those with aligned tensors
bool mha_fused_shape(int S, int Hd, int nh);
bool mha_fused_ok(const float* q, const float* k, const float* v, const float* y, int S, int Hd, int nh);
hipError_t launch_mha_f32(const float* q, const float* k, const float* v, float* y, int B, int S, int Hd, int nh,
                          float scale, float* parts, void* ws, hipStream_t s);
// the fused kernel with q, k, v given as chain bytes (columns = the hidden
// axis; 4-byte aligned, y 16-byte aligned, mha_fused_shape)
hipError_t launch_mha_codes_f32(const DqCodes& q, const DqCodes& k, const DqCodes& v, float* y, int B, int S,
                                int Hd, int nh, float scale, float* parts, hipStream_t s);
// (min, max) pairs the fused kernel writes (4 per (batch, head)); 0 when the
// shape takes the batched-GEMM path, which writes none
int mha_minmax_pairs(int B, int S, int Hd, int nh);
hipError_t launch_hardswish_f32(const float* x, float* y, long long n, int post_op, hipStream_t s);
hipError_t launch_clip_f32(const float* x, float* y, long long n, float lo, float hi,
                           hipStream_t s);

}  // namespace nnrh
