// nnrh_misc.hip -- non-MFMA kernels of the conv / matmul path:
//   * NCHW -> NHWC uint8 transpose (transpose_nchw_nhwc_u8.h:1-126), with
//     optional channel padding used by the first-layer (IC<=4) path;
//   * depthwise QLinearConv on NHWC (depthwise_int8_avx512.h:207-351);
//   * zero-point row sums for per-tensor / per-channel w_zp != 0;
//   * packing of a dynamic B operand for MatMulInteger / QLinearMatMul.
#include "nnrh_internal.h"
#include "nnrh_rq.h"

namespace nnrh {

// ---------------------------------------------------------------------------
// NCHW [N][C][HW] -> NHWC [N][HW][Cpad]; channels C..Cpad-1 get `fill`.
// One block per (image, 64-pixel strip); the C x 64 tile goes through LDS so
// both the reads (pixels contiguous) and the writes (channels contiguous)
// are coalesced.
__global__ __launch_bounds__(256) void nchw_to_nhwc_kernel(const uint8_t* __restrict x,
                                                           uint8_t* __restrict y, int C,
                                                           int HW, int Cpad, uint8_t fill) {
    __shared__ uint8_t tile[64][65];
    const int n = blockIdx.y;
    const int p0 = blockIdx.x * 64;
    const uint8_t* xn = x + (long long)n * C * HW;
    uint8_t* yn = y + (long long)n * HW * Cpad;
    for (int c0 = 0; c0 < Cpad; c0 += 64) {
        // load C-chunk x 64 pixels
        for (int i = threadIdx.x; i < 64 * 64; i += 256) {
            int cc = i >> 6, pp = i & 63;
            int c = c0 + cc, p = p0 + pp;
            uint8_t v = fill;
            if (c < C && p < HW) v = xn[(long long)c * HW + p];
            tile[cc][pp] = v;
        }
        __syncthreads();
        for (int i = threadIdx.x; i < 64 * 64; i += 256) {
            int pp = i >> 6, cc = i & 63;
            int c = c0 + cc, p = p0 + pp;
            if (c < Cpad && p < HW) yn[(long long)p * Cpad + c] = tile[cc][pp];
        }
        __syncthreads();
    }
}

// small channel counts (first-layer input, C <= 4 padded to 4): one thread
// per pixel, channel planes read coalesced, one 32-bit store per pixel
__global__ __launch_bounds__(256) void nchw_to_nhwc4_kernel(const uint8_t* __restrict x,
                                                            uint32_t* __restrict y, int C, long long HW,
                                                            long long total, uint8_t fill) {
    long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    long long n = i / HW, p = i - n * HW;
    const uint8_t* xn = x + n * C * HW + p;
    uint32_t w = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) w |= (uint32_t)(c < C ? xn[(long long)c * HW] : fill) << (8 * c);
    y[i] = w;
}

hipError_t launch_nchw_to_nhwc_u8(const uint8_t* x, uint8_t* y, int N, int C, int HW,
                                  int Cpad, uint8_t fill, hipStream_t s) {
    if (N <= 0 || HW <= 0 || Cpad <= 0) return hipSuccess;
    if (Cpad == 4 && C <= 4 && ((uintptr_t)y & 3) == 0) {
        long long total = (long long)N * HW;
        hipLaunchKernelGGL(nchw_to_nhwc4_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                           x, (uint32_t*)y, C, (long long)HW, total, fill);
        return hipGetLastError();
    }
    dim3 grid((HW + 63) / 64, N);
    hipLaunchKernelGGL(nchw_to_nhwc_kernel, grid, dim3(256), 0, s, x, y, C, HW, Cpad, fill);
    return hipGetLastError();
}

// First-layer input for the pipelined GEMM: NCHW uint8 with C <= 4 becomes
// zero-point padded NHWC4 rows of Wc pixels, stored as ncopy copies where
// copy i starts (i << copy_shift) pixels further right. A 4-tap chunk of the
// implicit im2col starting at padded pixel p then sits 16-byte aligned in
// copy (p & 3) >> copy_shift, at pixel p - (p & 3).
// y: [ncopy][N][Hp][Wc] x uint32 (4 channels, padding = fill).
__global__ __launch_bounds__(256) void first_layer_copies_kernel(
    const uint8_t* __restrict x, uint32_t* __restrict y, int C, int H, int W, int Hp, int Wc,
    int pad_t, int pad_l, int copy_shift, long long per_copy, long long total, uint8_t fill) {
    long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const long long ci = i / per_copy;
    long long rem = i - ci * per_copy;
    const int j = (int)(rem % Wc);
    rem /= Wc;
    const int ihp = (int)(rem % Hp);
    const long long n = rem / Hp;
    const int ih = ihp - pad_t;
    const int iw = j + ((int)ci << copy_shift) - pad_l;
    uint32_t w = (uint32_t)fill * 0x01010101u;
    if ((unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W) {
        const long long HW = (long long)H * W;
        const uint8_t* xp = x + n * C * HW + (long long)ih * W + iw;
        w = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) w |= (uint32_t)(c < C ? xp[(long long)c * HW] : fill) << (8 * c);
    }
    y[i] = w;
}

hipError_t launch_first_layer_copies(const uint8_t* x, uint8_t* y, int N, int C, int H, int W,
                                     int Hp, int Wc, int pad_t, int pad_l, int copy_shift,
                                     uint8_t fill, hipStream_t s) {
    if (N <= 0 || C > 4 || ((uintptr_t)y & 15)) return hipErrorInvalidValue;
    const int ncopy = 4 >> copy_shift;
    const long long per_copy = (long long)N * Hp * Wc;
    const long long total = per_copy * ncopy;
    hipLaunchKernelGGL(first_layer_copies_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       x, (uint32_t*)y, C, H, W, Hp, Wc, pad_t, pad_l, copy_shift, per_copy, total, fill);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Depthwise QLinearConv, NHWC in / NHWC or NCHW out, requantize RQ-A with
// clamp [L, hi]. Each thread computes 4 consecutive channels of one output
// pixel: acc = sum_taps (x - x_zp)(w - w_zp), exact int32. Out-of-image taps
// read x_zp in the reference (zero_buf), i.e. contribute 0, so they are
// skipped. Weights are repacked [kH*kW][C] (repack_depthwise_weights).
// tail_tile_h > 0 selects the tiled-im2col tail rule (RQ-A' on the last
// tsp%16 pixels of each tile), used when a depthwise conv writes NCHW.
__global__ __launch_bounds__(256) void depthwise_kernel(
    const uint8_t* __restrict x, const int8_t* __restrict w, uint8_t* __restrict y,
    const float* __restrict cs, const float* __restrict bf, int N, int C, int H, int W,
    int oH, int oW, int kH, int kW, int sH, int sW, int dH, int dW, int pad_t, int pad_l,
    int x_zp, int w_zp, float inv_y, int y_zp, int L, int hi, int act_signed, int y_nchw,
    int tail_mode, int tail_tile_h) {
    const int C4 = (C + 3) >> 2;
    const long long total = (long long)N * oH * oW * C4;
    long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int cg = (int)(idx % C4);
    const long long pix = idx / C4;
    const int ow = (int)(pix % oW);
    const int oh = (int)((pix / oW) % oH);
    const int n = (int)(pix / ((long long)oW * oH));
    const int c0 = cg * 4;
    const bool vec_ok = ((C & 3) == 0);
    int32_t acc[4] = {0, 0, 0, 0};
    const uint8_t* xn = x + (long long)n * H * W * C;
    for (int a = 0; a < kH; ++a) {
        int ih = oh * sH - pad_t + a * dH;
        if ((unsigned)ih >= (unsigned)H) continue;
        for (int b = 0; b < kW; ++b) {
            int iw = ow * sW - pad_l + b * dW;
            if ((unsigned)iw >= (unsigned)W) continue;
            const uint8_t* xp = xn + ((long long)ih * W + iw) * C + c0;
            const int8_t* wp = w + (long long)(a * kW + b) * C + c0;
            int xv[4], wv[4];
            if (vec_ok) {
                uint32_t xw = *(const uint32_t*)xp;
                uint32_t ww = *(const uint32_t*)wp;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint32_t xb = (xw >> (8 * i)) & 0xff, wb = (ww >> (8 * i)) & 0xff;
                    xv[i] = act_signed ? (int)(int8_t)xb : (int)xb;
                    wv[i] = (int)(int8_t)wb;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    bool ok = c0 + i < C;
                    xv[i] = ok ? (act_signed ? (int)(int8_t)xp[i] : (int)xp[i]) : x_zp;
                    wv[i] = ok ? (int)wp[i] : w_zp;
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[i] = wrap_add(acc[i], wrap_mul(xv[i] - x_zp, wv[i] - w_zp));
        }
    }
    bool tail = false;
    if (tail_mode == TAIL_SPATIAL) {
        const int sp = oH * oW, s = oh * oW + ow;
        tail = s >= sp - sp % 16;
    } else if (tail_mode == TAIL_TILED) {
        int oh0 = (oh / tail_tile_h) * tail_tile_h;
        int th = oH - oh0 < tail_tile_h ? oH - oh0 : tail_tile_h;
        int tsp = th * oW, ts = (oh - oh0) * oW + ow;
        tail = ts >= tsp - tsp % 16;
    }
    int q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int c = c0 + i < C ? c0 + i : C - 1;
        q[i] = tail ? rq_a_tail(acc[i], cs[c], bf[c], inv_y, y_zp, L, hi)
                    : rq_a(acc[i], cs[c], bf[c], inv_y, y_zp, L, hi);
    }
    if (y_nchw) {
        const long long sp = (long long)oH * oW, s = (long long)oh * oW + ow;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (c0 + i < C) y[((long long)n * C + c0 + i) * sp + s] = (uint8_t)q[i];
    } else {
        uint8_t* yp = y + pix * C + c0;
        if (vec_ok) {
            *(uint32_t*)yp = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
                             ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (c0 + i < C) yp[i] = (uint8_t)q[i];
        }
    }
}

hipError_t launch_depthwise(const uint8_t* x, const int8_t* w, uint8_t* y, const float* cs,
                            const float* bf, int N, int C, int H, int W, int oH, int oW,
                            int kH, int kW, int sH, int sW, int dH, int dW, int pad_t,
                            int pad_l, int x_zp, int w_zp, float inv_y, int y_zp, int L,
                            int hi, int act_signed, int y_nchw, int tail_mode,
                            int tail_tile_h, hipStream_t s) {
    long long total = (long long)N * oH * oW * ((C + 3) / 4);
    if (total <= 0) return hipSuccess;
    unsigned blocks = (unsigned)((total + 255) / 256);
    hipLaunchKernelGGL(depthwise_kernel, dim3(blocks), dim3(256), 0, s, x, w, y, cs, bf, N, C,
                       H, W, oH, oW, kH, kW, sH, sW, dH, dW, pad_t, pad_l, x_zp, w_zp, inv_y,
                       y_zp, L, hi, act_signed, y_nchw, tail_mode, tail_tile_h);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// rowsum[m] = sum_k (a[m][k] - a_zp): one wave per row.
__global__ __launch_bounds__(256) void rowsum_dense_kernel(const uint8_t* __restrict a,
                                                           long long lda, long long a_bstride,
                                                           int M, int K, int a_signed,
                                                           int a_zp, const void* a_zp_dev,
                                                           int32_t* __restrict out) {
    const int z = blockIdx.y;
    if (a_zp_dev)
        a_zp = a_signed ? (int)*(const int8_t*)a_zp_dev : (int)*(const uint8_t*)a_zp_dev;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    const uint8_t* ar = a + (long long)z * a_bstride + (long long)row * lda;
    int32_t s = 0;
    for (int k = lane; k < K; k += 64) {
        int v = a_signed ? (int)(int8_t)ar[k] : (int)ar[k];
        s += v - a_zp;
    }
    for (int off = 32; off > 0; off >>= 1) s += __shfl_down(s, off, 64);
    if (lane == 0) out[(long long)z * M + row] = s;
}

hipError_t launch_rowsum_dense(const uint8_t* a, long long lda, long long a_bstride, int M,
                               int K, int a_signed, int a_zp, const void* a_zp_dev, int32_t* out,
                               int batch, hipStream_t s) {
    if (M <= 0 || batch <= 0) return hipSuccess;
    dim3 grid((M + 3) / 4, batch);
    hipLaunchKernelGGL(rowsum_dense_kernel, grid, dim3(256), 0, s, a, lda, a_bstride, M, K,
                       a_signed, a_zp, a_zp_dev, out);
    return hipGetLastError();
}

// rowsum over the im2col row of output pixel m (NHWC input, channels
// [c_off, c_off+Cg) of a Cs-channel tensor): sum over in-image taps of
// (x - x_zp); out-of-image taps hold x_zp in the reference and contribute 0.
__global__ __launch_bounds__(256) void rowsum_conv_kernel(const uint8_t* __restrict x, int N,
                                                          int H, int W, int Cs, int Cg,
                                                          int oH, int oW, int kH, int kW,
                                                          int sH, int sW, int dH, int dW,
                                                          int pad_t, int pad_l, int a_signed,
                                                          int x_zp, int32_t* __restrict out) {
    const int z = blockIdx.y;   // group
    const long long m = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const long long M = (long long)N * oH * oW;
    if (m >= M) return;
    const int ow = (int)(m % oW), oh = (int)((m / oW) % oH), n = (int)(m / ((long long)oW * oH));
    int32_t s = 0;
    const int taps = kH * kW;
    for (int t = 0; t < taps; ++t) {
        int a = t / kW, b = t - a * kW;
        int ih = oh * sH - pad_t + a * dH, iw = ow * sW - pad_l + b * dW;
        if ((unsigned)ih >= (unsigned)H || (unsigned)iw >= (unsigned)W) continue;
        const uint8_t* xp = x + (((long long)n * H + ih) * W + iw) * Cs + (long long)z * Cg;
        for (int c = lane; c < Cg; c += 64) {
            int v = a_signed ? (int)(int8_t)xp[c] : (int)xp[c];
            s += v - x_zp;
        }
    }
    for (int off = 32; off > 0; off >>= 1) s += __shfl_down(s, off, 64);
    if (lane == 0) out[(long long)z * M + m] = s;
}

hipError_t launch_rowsum_conv(const uint8_t* x, int N, int H, int W, int Cs, int Cg, int groups,
                              int oH, int oW, int kH, int kW, int sH, int sW, int dH, int dW,
                              int pad_t, int pad_l, int a_signed, int x_zp, int32_t* out,
                              hipStream_t s) {
    long long M = (long long)N * oH * oW;
    if (M <= 0) return hipSuccess;
    dim3 grid((unsigned)((M + 3) / 4), groups);
    hipLaunchKernelGGL(rowsum_conv_kernel, grid, dim3(256), 0, s, x, N, H, W, Cs, Cg, oH, oW, kH,
                       kW, sH, sW, dH, dW, pad_t, pad_l, a_signed, x_zp, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Pack a row-major B[K][N] into [Np][Kp] (row = packed_row_of_col(n)), XOR
// shifting uint8 B to int8, zero padding; colsum[n] = sum_k b'[k][n].
// One thread per (n, 16-byte k chunk); colsum by a second pass per column.
__global__ __launch_bounds__(256) void pack_b_kernel(const uint8_t* __restrict b,
                                                     long long b_bstride, int K, int N, int Kp,
                                                     int Np, int b_xor, int8_t* __restrict out,
                                                     long long out_bstride) {
    const int z = blockIdx.y;
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int kch = Kp >> 4;
    if (idx >= (long long)Np * kch) return;
    const int n = (int)(idx / kch), kc = (int)(idx % kch);
    const uint8_t* bz = b + (long long)z * b_bstride;
    uint8_t v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        int k = kc * 16 + i;
        v[i] = (n < N && k < K) ? (uint8_t)(bz[(long long)k * N + n] ^ (uint8_t)b_xor) : 0;
    }
    int8_t* o = out + (long long)z * out_bstride + (long long)packed_row_of_col(n) * Kp + kc * 16;
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
        w[q] = v[4 * q] | (v[4 * q + 1] << 8) | (v[4 * q + 2] << 16) | ((uint32_t)v[4 * q + 3] << 24);
    *(uint4*)o = make_uint4(w[0], w[1], w[2], w[3]);
}

__global__ __launch_bounds__(256) void colsum_kernel(const uint8_t* __restrict b,
                                                     long long b_bstride, int K, int N, int b_xor,
                                                     int32_t* __restrict colsum,
                                                     long long colsum_bstride) {
    const int z = blockIdx.y;
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= N) return;
    const uint8_t* bz = b + (long long)z * b_bstride;
    int32_t s = 0;
    for (int k = 0; k < K; ++k) s += (int)(int8_t)(bz[(long long)k * N + n] ^ (uint8_t)b_xor);
    colsum[(long long)z * colsum_bstride + n] = s;
}

hipError_t launch_pack_b_dense(const void* b, long long b_bstride, int K, int N, int Kp, int Np,
                               int b_xor, int8_t* out, long long out_bstride, int32_t* colsum,
                               long long colsum_bstride, int batch, hipStream_t s) {
    if (batch <= 0) return hipSuccess;
    long long items = (long long)Np * (Kp >> 4);
    dim3 grid((unsigned)((items + 255) / 256), batch);
    hipLaunchKernelGGL(pack_b_kernel, grid, dim3(256), 0, s, (const uint8_t*)b, b_bstride, K, N,
                       Kp, Np, b_xor, out, out_bstride);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (colsum) {
        dim3 g2((N + 255) / 256, batch);
        hipLaunchKernelGGL(colsum_kernel, g2, dim3(256), 0, s, (const uint8_t*)b, b_bstride, K, N,
                           b_xor, colsum, colsum_bstride);
        e = hipGetLastError();
    }
    return e;
}

// ---------------------------------------------------------------------------
// byte fill (used instead of hipMemsetAsync so callers may capture it)
__global__ __launch_bounds__(256) void fill_u8_kernel(uint8_t* __restrict p, uint8_t v,
                                                      long long n) {
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (long long)gridDim.x * 256)
        p[i] = v;
}

hipError_t launch_fill_u8(void* p, uint8_t v, long long n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    long long b = (n + 255) / 256;
    if (b > 65536) b = 65536;
    hipLaunchKernelGGL(fill_u8_kernel, dim3((unsigned)b), dim3(256), 0, s, (uint8_t*)p, v, n);
    return hipGetLastError();
}

}  // namespace nnrh
