// nnrh_elem.h -- launchers of the memory-bound int8 kernels (nnrh_elem.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace nnrh {

struct QAddArgs {
    int kind;            // 0 same shape, 1 B scalar, 2 A scalar, 3 per-channel B[C]
    const void* a;
    const void* b;
    void* y;
    long long n;
    int C, HW, y_nhwc;   // per-channel layout
    int dt;              // 0 u8, 1 s8
    float sa, sb;        // a_s / y_s, b_s / y_s
    float fixed;         // same-shape body constant
    int a_zp, b_zp, y_zp;
    int lo, hi;
    int tail_all;        // every element takes the scalar tail expression
};

struct QMulArgs {
    int kind;            // 0 same shape, 1 B scalar, 2 A scalar, 3 per-channel B[C]
    const void* a;
    const void* b;
    void* y;
    long long n;
    int C, HW, y_nhwc;   // per-channel layout
    int dt;              // 0 u8, 1 s8
    float cs;            // fl(fl(a_s * b_s) / y_s)
    int a_zp, b_zp, y_zp;
    int lo, hi;
};
hipError_t launch_qmul(const QMulArgs& p, hipStream_t s);
hipError_t launch_qgap(const void* x, void* y, int N, int C, int spatial, int nhwc, int dt, float rs, int x_zp,
                       int y_zp, int lo, int hi, hipStream_t s);
hipError_t launch_qavgpool(const void* x, void* y, int N, int C, int iH, int iW, int oH, int oW, int kH, int kW,
                           int sH, int sW, int pH, int pW, int nhwc, int dt, float x_s, int x_zp, float y_s,
                           int y_zp, int lo, int hi, hipStream_t s);
hipError_t launch_qconcat_part(const void* x, void* y, long long outer, long long count, long long y_row,
                               long long y_off, int dt, int copy, float rs, int x_zp, int y_zp, int lo, int hi,
                               hipStream_t s);

// QLinearConcat in one launch: up to QCONCAT_MAX_PARTS inputs
constexpr int QCONCAT_MAX_PARTS = 8;
struct QConcatRows {
    int n;
    const void* x[QCONCAT_MAX_PARTS];
    long long cnt[QCONCAT_MAX_PARTS], off[QCONCAT_MAX_PARTS], body[QCONCAT_MAX_PARTS];
    int copy[QCONCAT_MAX_PARTS], zp[QCONCAT_MAX_PARTS];
    float rs[QCONCAT_MAX_PARTS];
    void* y;
    long long row, outer;
    int dt, y_zp, lo, hi;
};
hipError_t launch_qconcat_rows(const QConcatRows& a, hipStream_t s);
hipError_t launch_bn_affine_u8(const void* x, int x_f32, uint8_t* y, const float* A, const float* B, long long N,
                               int C, long long HW, int nhwc, hipStream_t s);
hipError_t launch_bn_f32(const float* x, float* y, const float* A, const float* B, long long N, int C, long long HW,
                         int nhwc, hipStream_t s);

hipError_t launch_quantize(const float* x, long long n, float scale, int zp, int dt, void* y,
                           hipStream_t s);
hipError_t launch_dequantize(const void* x, long long n, int dt, float scale, int zp, float* y,
                             hipStream_t s);
size_t dynamic_quantize_workspace();
hipError_t launch_dynamic_quantize(const float* x, long long n, uint8_t* y, float* y_scale,
                                   uint8_t* y_zp, void* workspace, hipStream_t s);
// scale / zero point from nparts (min, max) pairs, then the quantize pass
// as launch_dynamic_quantize, with the partials in the library's own
// per-device scratch array (no workspace argument, no allocation)
hipError_t launch_dynamic_quantize_noalloc(const float* x, long long n, uint8_t* y, float* y_scale,
                                           uint8_t* y_zp, hipStream_t s);
hipError_t launch_dynamic_quantize_parts(const float* x, long long n, const float* parts, int nparts,
                                         uint8_t* y, float* y_scale, uint8_t* y_zp, hipStream_t s);
// DynamicQuantizeLinear of a fused dequantize chain from its GEMM's uint8
// bytes (codes, rows x N contiguous) and (min, max) pairs: the chain's value
// of byte q in column n is [Gelu](fl(fl((q - q_zp) * dq_scale) + bias[n]));
// table: dynamic_quantize_codes_table_bytes(Np) bytes (Np = N rounded up to
// 64, bias padded to Np), 16-byte aligned
size_t dynamic_quantize_codes_table_bytes(int Np);
hipError_t launch_dynamic_quantize_codes(const uint8_t* codes, long long rows, int N, int Np, const float* bias,
                                         float dq_scale, int q_zp, int gelu, const float* parts, int nparts,
                                         uint8_t* table, uint8_t* y, float* y_scale, uint8_t* y_zp,
                                         hipStream_t s);
hipError_t launch_qadd(const QAddArgs& p, hipStream_t s);
hipError_t launch_maxpool_u8_nhwc(const uint8_t* x, uint8_t* y, int N, int C, int iH, int iW,
                                  int oH, int oW, int kH, int kW, int sH, int sW, int pH, int pW,
                                  hipStream_t s);

}  // namespace nnrh
