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

// 4 x 4 byte transpose of dwords a, b, c, d (row i = bytes of the i-th
// dword): o[j] = {a.byte j, b.byte j, c.byte j, d.byte j}. v_perm_b32's
// selector picks bytes of {S0 (bytes 4-7), S1 (bytes 0-3)}.
__device__ __forceinline__ void transpose4x4_u8(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t (&o)[4]) {
    const uint32_t t0 = __builtin_amdgcn_perm(b, a, 0x06020400u);   // a0 b0 a2 b2
    const uint32_t t1 = __builtin_amdgcn_perm(b, a, 0x07030501u);   // a1 b1 a3 b3
    const uint32_t t2 = __builtin_amdgcn_perm(d, c, 0x06020400u);   // c0 d0 c2 d2
    const uint32_t t3 = __builtin_amdgcn_perm(d, c, 0x07030501u);   // c1 d1 c3 d3
    o[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);              // a0 b0 c0 d0
    o[1] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);              // a1 b1 c1 d1
    o[2] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);              // a2 b2 c2 d2
    o[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);              // a3 b3 c3 d3
}

// NCHW -> NHWC with Cpad % 16 == 0 and HW % 16 == 0 (16-byte aligned
// tensors): a thread per (image, 16 pixels, 16 channels) loads the 16
// channel rows of its pixels (one 16-byte load each; channels past C are
// the fill byte), transposes the 16 x 16 bytes in registers and stores 16
// pixels of 16 channels (one 16-byte store each). Consecutive threads take
// consecutive channel groups of one pixel group, so a store instruction
// writes whole 16 x Cpad-byte pixel runs. One-wave blocks: a thread moves
// 256 bytes, so the grid is small and is spread over every CU.
__global__ __launch_bounds__(64) void nchw_to_nhwc16_kernel(const uint8_t* __restrict x, uint8_t* __restrict y,
                                                            int C, int HW, int Cpad, long long total,
                                                            uint8_t fill) {
    const long long t = (long long)blockIdx.x * 64 + threadIdx.x;
    if (t >= total) return;
    const int cgs = Cpad >> 4, pgs = HW >> 4;
    const long long rest = t / cgs;
    const int cg = (int)(t - rest * cgs);
    const long long n = rest / pgs;
    const int pg = (int)(rest - n * pgs);
    const uint8_t* xp = x + (n * C + cg * 16) * (long long)HW + pg * 16;
    const uint32_t fw = (uint32_t)fill * 0x01010101u;
    uint4 r[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
        r[i] = cg * 16 + i < C ? *(const uint4*)(xp + (long long)i * HW) : make_uint4(fw, fw, fw, fw);
    uint8_t* yp = y + (n * HW + pg * 16) * (long long)Cpad + cg * 16;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
        // pixels 4 jb .. 4 jb + 3: dword jb of every channel row
        uint32_t o[4][4];   // [channel quad q][pixel jj]
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t* a = (const uint32_t*)&r[4 * q];
            const uint32_t* b = (const uint32_t*)&r[4 * q + 1];
            const uint32_t* c = (const uint32_t*)&r[4 * q + 2];
            const uint32_t* d = (const uint32_t*)&r[4 * q + 3];
            transpose4x4_u8(a[jb], b[jb], c[jb], d[jb], o[q]);
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
            *(uint4*)(yp + (long long)(4 * jb + jj) * Cpad) = make_uint4(o[0][jj], o[1][jj], o[2][jj], o[3][jj]);
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
    if (Cpad % 16 == 0 && HW % 16 == 0 && C <= Cpad && ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0) {
        const long long total = (long long)N * (HW / 16) * (Cpad / 16);
        hipLaunchKernelGGL(nchw_to_nhwc16_kernel, dim3((unsigned)((total + 63) / 64)), dim3(64), 0, s, x, y, C,
                           HW, Cpad, total, fill);
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
// grid: x over 4-pixel groups of one padded row (copy index fastest), y =
// padded row, z = image
__global__ __launch_bounds__(256) void first_layer_copies_kernel(
    const uint8_t* __restrict x, uint32_t* __restrict y, int C, int H, int W, int Hp, int Wc,
    int pad_t, int pad_l, int copy_shift, int ncopy_log2, long long per_copy, uint8_t fill) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    const int ci = t & ((1 << ncopy_log2) - 1);
    const int j0 = (t >> ncopy_log2) * 4;
    if (j0 >= Wc) return;
    const int ihp = blockIdx.y, n = blockIdx.z;
    const int ih = ihp - pad_t;
    const long long HW = (long long)H * W;
    const uint8_t* xr = x + (long long)n * C * HW + (long long)ih * W;
    uint32_t out[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int iw = j0 + k + (ci << copy_shift) - pad_l;
        uint32_t w = (uint32_t)fill * 0x01010101u;
        if ((unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W) {
            w = 0;
#pragma unroll
            for (int c = 0; c < 4; ++c) w |= (uint32_t)(c < C ? xr[(long long)c * HW + iw] : fill) << (8 * c);
        }
        out[k] = w;
    }
    uint32_t* yp = y + (long long)ci * per_copy + ((long long)n * Hp + ihp) * Wc + j0;
    if (j0 + 4 <= Wc) {
        *(uint4*)yp = make_uint4(out[0], out[1], out[2], out[3]);
    } else {
        for (int k = 0; k < 4 && j0 + k < Wc; ++k) yp[k] = out[k];
    }
}

hipError_t launch_first_layer_copies(const uint8_t* x, uint8_t* y, int N, int C, int H, int W,
                                     int Hp, int Wc, int pad_t, int pad_l, int copy_shift,
                                     uint8_t fill, hipStream_t s) {
    if (N <= 0 || C > 4 || ((uintptr_t)y & 15) || (Wc & 3) || N > 65535 || Hp > 65535)
        return hipErrorInvalidValue;
    const int ncopy_log2 = 2 - copy_shift;
    const long long per_copy = (long long)N * Hp * Wc;
    const long long threads_x = (long long)(Wc / 4) << ncopy_log2;
    const dim3 grid((unsigned)((threads_x + 255) / 256), (unsigned)Hp, (unsigned)N);
    hipLaunchKernelGGL(first_layer_copies_kernel, grid, dim3(256), 0, s, x, (uint32_t*)y, C, H, W, Hp, Wc,
                       pad_t, pad_l, copy_shift, ncopy_log2, per_copy, fill);
    return hipGetLastError();
}

// QuantizeLinear of the fp32 NCHW network input fused into the multi-copy
// image above: element (n, c, ih, iw) is quantized with the formula
// quantize_kernel (nnrh_elem.hip) applies at its flat NCHW index -- the
// 16-wide SIMD body multiplies by fl(1/s), the last n%16 elements (and all
// of them when n < 64) divide, QuantizeLinear.cpp:128-194 -- and placed
// where first_layer_copies_kernel places that byte. The copy index varies
// fastest, so the copies of one pixel read the same input lines.
__device__ __forceinline__ uint32_t quant_u8(float xv, long long idx, long long body, float scale,
                                             float inv, int zp) {
    int q;
    if (idx < body) {
        float v = xv * inv;
        v = __builtin_rintf(v) + (float)zp;
        v = clamp_minmax(v, 0.0f, 255.0f);
        q = (int)v;
    } else {
        q = clampi(wrap_add(x86_f2i(__builtin_rintf(xv / scale)), zp), 0, 255);
    }
    return (uint32_t)q;
}

// R <= QFL_ROWS padded rows per block (y = group of rows, z = image), R * L
// dwords staged (L padded pixels a row): the rows' input pixels are quantized into LDS as packed 4-channel dwords (fill
// outside the image), then every copy writes its shifted Wc-pixel rows with
// 16-byte stores. Every load of a thread's pixels over all the block's rows
// is issued before the first one is used, so each block keeps
// R * C loads per thread in flight (one row per block leaves the kernel
// waiting on memory latency).
constexpr int QFL_MAX_ROW = 4096;   // dwords staged in LDS (all rows of a block)
constexpr int QFL_ROWS = 8;

__global__ __launch_bounds__(256) void quantize_first_layer_copies_kernel(
    const float* __restrict x, uint32_t* __restrict y, int C, int H, int W, int Hp, int Wc,
    int pad_t, int pad_l, int copy_shift, int ncopy, long long per_copy, uint8_t fill,
    float scale, float inv, int zp, long long qbody, int R) {
    extern __shared__ uint32_t row[];   // R x L dwords (launch size)
    const int ihp0 = blockIdx.y * R, n = blockIdx.z;
    const int nrows = min(R, Hp - ihp0);
    // staged pixels: padded columns 0 .. L-1 (input column = p - pad_l)
    const int L = Wc + ((ncopy - 1) << copy_shift);
    const uint32_t fill4 = (uint32_t)fill * 0x01010101u;
    const long long HW = (long long)H * W;
    for (int p = threadIdx.x; p < L; p += 256) {
        const int iw = p - pad_l;
        const bool in_col = (unsigned)iw < (unsigned)W;
        float v[QFL_ROWS][4];
#pragma unroll
        for (int r = 0; r < QFL_ROWS; ++r) {
            const int ih = ihp0 + r - pad_t;
            const bool ok = r < nrows && in_col && (unsigned)ih < (unsigned)H;
            const long long base = (long long)n * C * HW + (long long)ih * W + iw;
#pragma unroll
            for (int c = 0; c < 4; ++c) v[r][c] = (ok && c < C) ? x[base + (long long)c * HW] : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < QFL_ROWS; ++r) {
            const int ih = ihp0 + r - pad_t;
            if (r >= nrows) break;
            uint32_t w = fill4;
            if (in_col && (unsigned)ih < (unsigned)H) {
                w = 0;
                const long long base = (long long)n * C * HW + (long long)ih * W + iw;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    uint32_t bt = fill;
                    if (c < C) {
                        const long long idx = base + (long long)c * HW;
                        bt = quant_u8(v[r][c], idx, qbody, scale, inv, zp);
                    }
                    w |= bt << (8 * c);
                }
            }
            row[r * L + p] = w;
        }
    }
    __syncthreads();
    const int q4 = Wc >> 2;   // 16-byte groups per copy row
    for (int t = threadIdx.x; t < q4 * ncopy * nrows; t += 256) {
        const int r = t / (q4 * ncopy), u = t - r * (q4 * ncopy);
        const int ci = u / q4, g = u - ci * q4;
        const int p0 = r * L + (ci << copy_shift) + 4 * g;
        uint32_t* yp = y + (long long)ci * per_copy + ((long long)n * Hp + ihp0 + r) * Wc + 4 * g;
        *(uint4*)yp = make_uint4(row[p0], row[p0 + 1], row[p0 + 2], row[p0 + 3]);
    }
}

hipError_t launch_quantize_first_layer_copies(const float* x, uint8_t* y, int N, int C, int H, int W,
                                              int Hp, int Wc, int pad_t, int pad_l, int copy_shift,
                                              uint8_t fill, float scale, int zp, hipStream_t s) {
    const int ncopy = 4 >> copy_shift;
    const int L = Wc + ((ncopy - 1) << copy_shift);
    if (N <= 0 || C > 4 || ((uintptr_t)y & 15) || (Wc & 3) || N > 65535 || Hp > 65535 || L > QFL_MAX_ROW)
        return hipErrorInvalidValue;
    const int R = min(QFL_ROWS, QFL_MAX_ROW / L);
    const long long per_copy = (long long)N * Hp * Wc;
    const long long qn = (long long)N * C * H * W;
    const long long qbody = qn >= 64 ? qn - qn % 16 : 0;
    const float inv = 1.0f / scale;
    const dim3 grid(1, (unsigned)((Hp + R - 1) / R), (unsigned)N);
    const size_t lds = sizeof(uint32_t) * (size_t)R * L;
    hipLaunchKernelGGL(quantize_first_layer_copies_kernel, grid, dim3(256), lds, s, x, (uint32_t*)y, C, H, W,
                       Hp, Wc, pad_t, pad_l, copy_shift, ncopy, per_copy, fill, scale, inv, zp, qbody, R);
    return hipGetLastError();
}

// QLinearConv on 3-D tensors, the reference's exec_typed<T> ndim == 3 loop
// (QLinearConv.cpp:286-334), one thread per output [n][oc][ow]:
//   sum = sum_{c,kw} (x - x_zp) * (w - w_zp), with x, x_zp, w and w_zp all read
//   through the activation type (a uint8 activation makes int8 weight bytes
//   count as uint8, :194-206); result = fl(fl(float(sum) * cs) + bf), two
//   roundings (this file is compiled with -ffp-contract=off);
//   y = clamp((int32)nearbyint(fl(result / y_scale)) + y_zp)   (RQ-S)
__global__ __launch_bounds__(256) void conv1d_typed_kernel(
    const uint8_t* __restrict x, const int8_t* __restrict w, const int32_t* __restrict wzp,
    const float* __restrict cs, const float* __restrict bf, uint8_t* __restrict y, int N, int C, int iW,
    int OC, int G, int kW, int oW, int sW, int dW, int pad_l, int x_zp, int y_zp, float y_scale, int u8,
    int lo, int hi) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long total = (long long)N * OC * oW;
    if (i >= total) return;
    const int ow = (int)(i % oW);
    const long long r = i / oW;
    const int oc = (int)(r % OC), n = (int)(r / OC);
    const int Cg = C / G, g = oc / (OC / G);
    const int32_t wz = wzp[oc];
    uint32_t sum = 0;
    for (int c = 0; c < Cg; ++c) {
        const int ic = g * Cg + c;
        const uint8_t* xr = x + ((long long)n * C + ic) * iW;
        const int8_t* wr = w + ((long long)oc * Cg + c) * kW;
        for (int kw = 0; kw < kW; ++kw) {
            const int iw = ow * sW - pad_l + kw * dW;
            if (iw < 0 || iw >= iW) continue;
            const int32_t xv = (u8 ? (int32_t)xr[iw] : (int32_t)(int8_t)xr[iw]) - x_zp;
            const int32_t wv = (u8 ? (int32_t)(uint8_t)wr[kw] : (int32_t)wr[kw]) - wz;
            sum += (uint32_t)(xv * wv);
        }
    }
    const float t = (float)(int32_t)sum * cs[oc];
    const float result = t + bf[oc];
    const float q = result / y_scale;
    const int v = wrap_add(x86_f2i(__builtin_rintf(q)), y_zp);
    y[i] = (uint8_t)clampi(v, lo, hi);
}

hipError_t launch_conv1d_typed(const uint8_t* x, const int8_t* w, const int32_t* wzp, const float* cs,
                               const float* bf, uint8_t* y, int N, int C, int iW, int OC, int G, int kW,
                               int oW, int sW, int dW, int pad_l, int x_zp, int y_zp, float y_scale, int u8,
                               hipStream_t s) {
    const long long total = (long long)N * OC * oW;
    if (total <= 0) return hipSuccess;
    if ((total + 255) / 256 > 0x7fffffffLL) return hipErrorInvalidValue;
    hipLaunchKernelGGL(conv1d_typed_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, x, w, wzp,
                       cs, bf, y, N, C, iW, OC, G, kW, oW, sW, dW, pad_l, x_zp, y_zp, y_scale, u8,
                       u8 ? 0 : -128, u8 ? 255 : 127);
    return hipGetLastError();
}

// NHWC [pixels][C] -> [pixels][Cpad] with the tail channels set to `fill`
// (Cpad % 4 == 0); one thread per output dword.
__global__ __launch_bounds__(256) void pad_channels_kernel(const uint8_t* __restrict x,
                                                           uint32_t* __restrict y, long long total,
                                                           int C, int Cpad4, uint8_t fill) {
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (long long)gridDim.x * 256) {
        const long long p = i / Cpad4;
        const int c0 = (int)(i - p * Cpad4) * 4;
        const uint8_t* xp = x + p * C;
        uint32_t w = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) w |= (uint32_t)(c0 + j < C ? xp[c0 + j] : fill) << (8 * j);
        y[i] = w;
    }
}

hipError_t launch_pad_channels_u8(const uint8_t* x, uint8_t* y, long long pixels, int C, int Cpad,
                                  uint8_t fill, hipStream_t s) {
    if (pixels <= 0) return hipSuccess;
    if (Cpad % 4 || Cpad < C || ((uintptr_t)y & 3)) return hipErrorInvalidValue;
    const long long total = pixels * (Cpad / 4);
    long long blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(pad_channels_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, (uint32_t*)y,
                       total, C, Cpad / 4, fill);
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
// Depthwise QLinearConv, NHWC in and out, 16 channels per thread, RQ-A with
// clamp [L, hi] and no scalar tails (the DW branch,
// depthwise_int8_avx512.h:207-351). The tap sum runs on v_dot4_i32_i8:
//   sum_t (x_t - x_zp) w_t = sum_t x'_t w_t + corr[c],
//   x' = x ^ a_xor (x - 128 for uint8), corr[c] = (a_sub - x_zp) * sum_t w_t,
// with the 4-tap byte groups of one channel assembled by a 4x4 byte
// transpose (v_perm) and the weights pre-packed [group][C] as 4 taps per
// dword (zero past the last tap). Out-of-image taps read the pad byte x_zp,
// whose product cancels against corr, so they contribute 0 exactly as the
// reference's zero_buf does. All int32 arithmetic wraps like vpmulld/vpaddd.
// Requantize: clamp(rne(u) + zp, L, hi) == rne(clamp(u, L - zp, hi - zp)) + zp
// for integer bounds, evaluated with the 1.5 * 2^23 rounding constant.
struct Dw16Args {
    const uint8_t* x;
    const uint32_t* wdot;   // [G4][C]
    const int32_t* corr;    // [C]
    const float* cs;
    const float* bf;
    uint8_t* y;
    int N, C, H, W, oH, oW, kW, taps, sH, sW, dH, dW, pad_t, pad_l;
    uint32_t pad4, xmask;
    float inv_y;
    int y_zp, L, hi;
    int c16, groups_per_block;        // channel chunks; pixel groups a block holds
    uint32_t n_groups;                // rows * owbs
    uint32_t owbs, owb_mul, owb_shift;
};

constexpr int DW16_PX = 4;   // output pixels along a row per thread

__device__ __forceinline__ void transpose4x4_bytes(uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3,
                                                   uint32_t* y) {
    const uint32_t lo01 = __builtin_amdgcn_perm(x1, x0, 0x05010400u);   // x0b0 x1b0 x0b1 x1b1
    const uint32_t hi01 = __builtin_amdgcn_perm(x1, x0, 0x07030602u);   // x0b2 x1b2 x0b3 x1b3
    const uint32_t lo23 = __builtin_amdgcn_perm(x3, x2, 0x05010400u);
    const uint32_t hi23 = __builtin_amdgcn_perm(x3, x2, 0x07030602u);
    y[0] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);              // x0b0 x1b0 x2b0 x3b0
    y[1] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);              // x0b1 x1b1 x2b1 x3b1
    y[2] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
    y[3] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
}

// Block = groups_per_block pixel groups x c16 channel chunks (thread ->
// chunk threadIdx % c16, so each thread keeps one chunk's weights); a pixel
// group is DW16_PX consecutive output pixels of one row; blocks stride over
// the pixel groups.
template <int G4>
__global__ __launch_bounds__(256) void dw16_kernel(Dw16Args p) {
    const int tid = threadIdx.x;
    if (tid >= p.c16 * p.groups_per_block) return;
    const int cg = tid % p.c16;
    const int gl = tid / p.c16;
    const int c0 = cg * 16;
    uint32_t wd[G4][16];
#pragma unroll
    for (int g = 0; g < G4; ++g)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint4 v = *(const uint4*)(p.wdot + (long long)g * p.C + c0 + 4 * q);
            wd[g][4 * q] = v.x; wd[g][4 * q + 1] = v.y; wd[g][4 * q + 2] = v.z; wd[g][4 * q + 3] = v.w;
        }
    int32_t corr[16];
    float cs[16], bf[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int4 cv = *(const int4*)(p.corr + c0 + 4 * q);
        const float4 sv = *(const float4*)(p.cs + c0 + 4 * q);
        const float4 bv = *(const float4*)(p.bf + c0 + 4 * q);
        corr[4 * q] = cv.x; corr[4 * q + 1] = cv.y; corr[4 * q + 2] = cv.z; corr[4 * q + 3] = cv.w;
        cs[4 * q] = sv.x; cs[4 * q + 1] = sv.y; cs[4 * q + 2] = sv.z; cs[4 * q + 3] = sv.w;
        bf[4 * q] = bv.x; bf[4 * q + 1] = bv.y; bf[4 * q + 2] = bv.z; bf[4 * q + 3] = bv.w;
    }
    const float lo_f = (float)(p.L - p.y_zp), hi_f = (float)(p.hi - p.y_zp);
    const bool zp_even = (p.y_zp & 1) == 0;
    const float magic = zp_even ? 12582912.0f + (float)p.y_zp : 12582912.0f;
    const uint32_t zp_add = zp_even ? 0u : (uint32_t)p.y_zp;
    const uint32_t stride = gridDim.x * (uint32_t)p.groups_per_block;

    for (uint32_t pg = blockIdx.x * (uint32_t)p.groups_per_block + gl; pg < p.n_groups; pg += stride) {
        const int row = (int)fast_div(pg, p.owb_mul, p.owb_shift);
        const int owb = (int)pg - row * (int)p.owbs;
        const int n = row / p.oH;
        const int oh = row - n * p.oH;
        const uint8_t* xn = p.x + (long long)n * p.H * p.W * p.C + c0;
        uint8_t* yrow = p.y + (long long)row * p.oW * p.C + c0;
#pragma unroll 1
        for (int px = 0; px < DW16_PX; ++px) {
            const int ow = owb * DW16_PX + px;
            if (ow >= p.oW) break;
            int32_t acc[16];
#pragma unroll
            for (int c = 0; c < 16; ++c) acc[c] = corr[c];
#pragma unroll
            for (int g = 0; g < G4; ++g) {
                uint32_t xt[4][4];   // [tap in group][dword = 4 channels]
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) {
                    const int t = 4 * g + tt;
                    uint4 v = make_uint4(p.pad4, p.pad4, p.pad4, p.pad4);
                    if (t < p.taps) {
                        const int a = t / p.kW;
                        const int b = t - a * p.kW;
                        const int ih = oh * p.sH - p.pad_t + a * p.dH;
                        const int iw = ow * p.sW - p.pad_l + b * p.dW;
                        if ((unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W)
                            v = *(const uint4*)(xn + ((long long)ih * p.W + iw) * p.C);
                    }
                    xt[tt][0] = v.x ^ p.xmask; xt[tt][1] = v.y ^ p.xmask;
                    xt[tt][2] = v.z ^ p.xmask; xt[tt][3] = v.w ^ p.xmask;
                }
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    uint32_t tr[4];
                    transpose4x4_bytes(xt[0][d], xt[1][d], xt[2][d], xt[3][d], tr);
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[4 * d + j] = __builtin_amdgcn_sdot4((int)tr[j], (int)wd[g][4 * d + j],
                                                               acc[4 * d + j], false);
                }
            }
            uint32_t ob[16];
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                const float t = __builtin_fmaf((float)acc[c], cs[c], bf[c]);
                float u = t * p.inv_y;
                u = __builtin_amdgcn_fmed3f(u, lo_f, hi_f);
                ob[c] = (uint32_t)__float_as_int(u + magic) + zp_add;
            }
            uint32_t w4[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t ab = __builtin_amdgcn_perm(ob[4 * q + 1], ob[4 * q], 0x0c0c0400u);
                const uint32_t cd = __builtin_amdgcn_perm(ob[4 * q + 3], ob[4 * q + 2], 0x0c0c0400u);
                w4[q] = __builtin_amdgcn_perm(cd, ab, 0x05040100u);
            }
            *(uint4*)(yrow + (long long)ow * p.C) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
    }
}

// ---------------------------------------------------------------------------
// 3x3 depthwise, stride 1 or 2, 8 channels (two dwords) a thread and 4
// consecutive output pixels of one row. A filter row contributes through one
// sdot4 per (pixel, channel): its weights are packed {w0, w1, w2, 0}, and the
// window of 4 input bytes starting at the pixel's first column comes from
// the byte transpose of 4 input columns by v_alignbyte (the 4th byte meets
// the 0 weight). Each filter row's input columns (6 for stride 1, 9 for
// stride 2) are loaded once for all 4 pixels, every load issued before the
// first use. Same arithmetic as dw16_kernel: x ^ 0x80 against signed weights,
// the per-channel constant (128 - x_zp) * sum(w), RQ-A.
struct Dw3Args {
    const uint8_t* x;
    const uint32_t* wrow;   // [3][C]: {w[c][a][0], w[c][a][1], w[c][a][2], 0}
    const int32_t* corr;    // [C]
    const float* cs;
    const float* bf;
    uint8_t* y;
    int N, C, H, W, oH, oW, pad_t, pad_l;
    uint32_t pad4, xmask;
    float inv_y;
    int y_zp, L, hi;
    int c8, groups_per_block;         // channel chunks; pixel groups a block holds
    uint32_t n_groups;                // rows * owbs
    uint32_t owbs, owb_mul, owb_shift;
};

template <int SW>
__global__ __launch_bounds__(256) void dw3x3_kernel(Dw3Args p) {
    constexpr int NCOL = 3 + 3 * SW;            // input columns of 4 output pixels
    constexpr int NG = (NCOL + 3) / 4;          // 4-column transpose groups
    const int tid = threadIdx.x;
    if (tid >= p.c8 * p.groups_per_block) return;
    const int cg = tid % p.c8;
    const int gl = tid / p.c8;
    const int c0 = cg * 8;
    uint32_t wd[3][8];
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint4 v = *(const uint4*)(p.wrow + (long long)a * p.C + c0 + 4 * q);
            wd[a][4 * q] = v.x; wd[a][4 * q + 1] = v.y; wd[a][4 * q + 2] = v.z; wd[a][4 * q + 3] = v.w;
        }
    int32_t corr[8];
    float cs[8], bf[8];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int4 cv = *(const int4*)(p.corr + c0 + 4 * q);
        const float4 sv = *(const float4*)(p.cs + c0 + 4 * q);
        const float4 bv = *(const float4*)(p.bf + c0 + 4 * q);
        corr[4 * q] = cv.x; corr[4 * q + 1] = cv.y; corr[4 * q + 2] = cv.z; corr[4 * q + 3] = cv.w;
        cs[4 * q] = sv.x; cs[4 * q + 1] = sv.y; cs[4 * q + 2] = sv.z; cs[4 * q + 3] = sv.w;
        bf[4 * q] = bv.x; bf[4 * q + 1] = bv.y; bf[4 * q + 2] = bv.z; bf[4 * q + 3] = bv.w;
    }
    const float lo_f = (float)(p.L - p.y_zp), hi_f = (float)(p.hi - p.y_zp);
    const bool zp_even = (p.y_zp & 1) == 0;
    const float magic = zp_even ? 12582912.0f + (float)p.y_zp : 12582912.0f;
    const uint32_t zp_add = zp_even ? 0u : (uint32_t)p.y_zp;
    const uint32_t stride = gridDim.x * (uint32_t)p.groups_per_block;

    for (uint32_t pg = blockIdx.x * (uint32_t)p.groups_per_block + gl; pg < p.n_groups; pg += stride) {
        const int row = (int)fast_div(pg, p.owb_mul, p.owb_shift);
        const int owb = (int)pg - row * (int)p.owbs;
        const int n = row / p.oH;
        const int oh = row - n * p.oH;
        const int ow0 = owb * 4;
        int32_t acc[4][8];
#pragma unroll
        for (int px = 0; px < 4; ++px)
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[px][c] = corr[c];
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            const int ih = oh * SW - p.pad_t + a;
            const bool row_ok = (unsigned)ih < (unsigned)p.H;
            // 32-bit offsets from the tensor base (N H W C < 2^31: checked by
            // the launcher); taps outside the image load an in-image byte and
            // take the zero point instead, with no branch around the load
            const int rbase = ((n * p.H + (row_ok ? ih : 0)) * p.W) * p.C + c0;
            uint2 v[4 * NG];
#pragma unroll
            for (int j = 0; j < 4 * NG; ++j) {
                v[j] = make_uint2(0u, 0u);   // columns past NCOL meet 0 weights only
                if (j < NCOL) {
                    const int iw = ow0 * SW - p.pad_l + j;
                    const bool ok = row_ok && (unsigned)iw < (unsigned)p.W;
                    uint2 t = *(const uint2*)(p.x + (uint32_t)(rbase + (ok ? iw : 0) * p.C));
                    t.x = ok ? t.x : p.pad4;
                    t.y = ok ? t.y : p.pad4;
                    v[j] = make_uint2(t.x ^ p.xmask, t.y ^ p.xmask);
                }
            }
#pragma unroll
            for (int d = 0; d < 2; ++d) {
                uint32_t T[NG][4];   // [column group][channel]: bytes = 4 columns
#pragma unroll
                for (int gq = 0; gq < NG; ++gq) {
                    const uint32_t c0w = d ? v[4 * gq].y : v[4 * gq].x;
                    const uint32_t c1w = d ? v[4 * gq + 1].y : v[4 * gq + 1].x;
                    const uint32_t c2w = d ? v[4 * gq + 2].y : v[4 * gq + 2].x;
                    const uint32_t c3w = d ? v[4 * gq + 3].y : v[4 * gq + 3].x;
                    transpose4x4_bytes(c0w, c1w, c2w, c3w, T[gq]);
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int ch = 4 * d + j;
                    const int w = (int)wd[a][ch];
#pragma unroll
                    for (int px = 0; px < 4; ++px) {
                        const int b0 = px * SW;          // first column of the pixel's window
                        const int gq = b0 >> 2, sh = b0 & 3;
                        const uint32_t win = sh == 0 ? T[gq][j] : __builtin_amdgcn_alignbyte(T[gq + 1][j], T[gq][j], sh);
                        acc[px][ch] = __builtin_amdgcn_sdot4((int)win, w, acc[px][ch], false);
                    }
                }
            }
        }
        uint8_t* yrow = p.y + (long long)row * p.oW * p.C + c0;
#pragma unroll
        for (int px = 0; px < 4; ++px) {
            const int ow = ow0 + px;
            if (ow >= p.oW) break;
            uint32_t ob[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const float t = __builtin_fmaf((float)acc[px][c], cs[c], bf[c]);
                float u = t * p.inv_y;
                u = __builtin_amdgcn_fmed3f(u, lo_f, hi_f);
                ob[c] = (uint32_t)__float_as_int(u + magic) + zp_add;
            }
            uint32_t w2[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const uint32_t ab = __builtin_amdgcn_perm(ob[4 * q + 1], ob[4 * q], 0x0c0c0400u);
                const uint32_t cd = __builtin_amdgcn_perm(ob[4 * q + 3], ob[4 * q + 2], 0x0c0c0400u);
                w2[q] = __builtin_amdgcn_perm(cd, ab, 0x05040100u);
            }
            *(uint2*)(yrow + (long long)ow * p.C) = make_uint2(w2[0], w2[1]);
        }
    }
}

hipError_t launch_depthwise3x3(const uint8_t* x, const uint32_t* wrow, const int32_t* corr, uint8_t* y,
                               const float* cs, const float* bf, int N, int C, int H, int W, int oH, int oW,
                               int stride, int pad_t, int pad_l, int x_zp, int a_xor, float inv_y, int y_zp,
                               int L, int hi, hipStream_t s) {
    if (C % 8 || C > 8 * 256 || (stride != 1 && stride != 2) || N <= 0 || oH <= 0 || oW <= 0)
        return hipErrorInvalidValue;
    if ((long long)N * H * W * C >= (1LL << 31)) return hipErrorInvalidValue;   // 32-bit input offsets
    if ((((uintptr_t)x) | ((uintptr_t)y)) & 7) return hipErrorInvalidValue;
    Dw3Args a{};
    a.x = x; a.wrow = wrow; a.corr = corr; a.cs = cs; a.bf = bf; a.y = y;
    a.N = N; a.C = C; a.H = H; a.W = W; a.oH = oH; a.oW = oW; a.pad_t = pad_t; a.pad_l = pad_l;
    a.pad4 = (uint32_t)(x_zp & 0xff) * 0x01010101u;
    a.xmask = (uint32_t)(a_xor & 0xff) * 0x01010101u;
    a.inv_y = inv_y; a.y_zp = y_zp; a.L = L; a.hi = hi;
    a.c8 = C / 8;
    a.groups_per_block = 256 / a.c8;
    a.owbs = (uint32_t)((oW + 3) / 4);
    const long long groups = (long long)N * oH * a.owbs;
    if (groups >= (1LL << 31)) return hipErrorInvalidValue;
    a.n_groups = (uint32_t)groups;
    fast_div_consts(a.owbs, &a.owb_mul, &a.owb_shift);
    long long blocks = (groups + a.groups_per_block - 1) / a.groups_per_block;
    if (blocks > 8192) blocks = 8192;
    if (stride == 1) hipLaunchKernelGGL(dw3x3_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, s, a);
    else hipLaunchKernelGGL(dw3x3_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_depthwise16(const uint8_t* x, const uint32_t* wdot, const int32_t* corr,
                              uint8_t* y, const float* cs, const float* bf, int N, int C, int H,
                              int W, int oH, int oW, int kH, int kW, int sH, int sW, int dH, int dW,
                              int pad_t, int pad_l, int x_zp, int a_xor, float inv_y, int y_zp,
                              int L, int hi, hipStream_t s) {
    const int taps = kH * kW;
    if (C % 16 || C > 16 * 256 || taps < 1 || taps > 12 || N <= 0 || oH <= 0 || oW <= 0)
        return hipErrorInvalidValue;
    if ((((uintptr_t)x) | ((uintptr_t)y)) & 15) return hipErrorInvalidValue;
    Dw16Args a{};
    a.x = x; a.wdot = wdot; a.corr = corr; a.cs = cs; a.bf = bf; a.y = y;
    a.N = N; a.C = C; a.H = H; a.W = W; a.oH = oH; a.oW = oW; a.kW = kW; a.taps = taps;
    a.sH = sH; a.sW = sW; a.dH = dH; a.dW = dW; a.pad_t = pad_t; a.pad_l = pad_l;
    a.pad4 = (uint32_t)(x_zp & 0xff) * 0x01010101u;
    a.xmask = (uint32_t)(a_xor & 0xff) * 0x01010101u;
    a.inv_y = inv_y; a.y_zp = y_zp; a.L = L; a.hi = hi;
    a.c16 = C / 16;
    a.groups_per_block = 256 / a.c16;
    a.owbs = (uint32_t)((oW + DW16_PX - 1) / DW16_PX);
    const long long groups = (long long)N * oH * a.owbs;
    if (groups >= (1LL << 31)) return hipErrorInvalidValue;
    a.n_groups = (uint32_t)groups;
    fast_div_consts(a.owbs, &a.owb_mul, &a.owb_shift);
    long long blocks = (groups + a.groups_per_block - 1) / a.groups_per_block;
    if (blocks > 4096) blocks = 4096;
    const int G4 = (taps + 3) / 4;
    if (G4 == 1) hipLaunchKernelGGL(dw16_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, s, a);
    else if (G4 == 2) hipLaunchKernelGGL(dw16_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, s, a);
    else hipLaunchKernelGGL(dw16_kernel<3>, dim3((unsigned)blocks), dim3(256), 0, s, a);
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
                                                          int H, int W, int Cs, int Cg, int cg_stride,
                                                          int oH, int oW, int kH, int kW,
                                                          int sH, int sW, int dH, int dW,
                                                          int pad_t, int pad_l, int a_signed,
                                                          int x_zp, int32_t* __restrict out,
                                                          long long out_bstride) {
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
        const uint8_t* xp = x + (((long long)n * H + ih) * W + iw) * Cs + (long long)z * cg_stride;
        for (int c = lane; c < Cg; c += 64) {
            int v = a_signed ? (int)(int8_t)xp[c] : (int)xp[c];
            s += v - x_zp;
        }
    }
    for (int off = 32; off > 0; off >>= 1) s += __shfl_down(s, off, 64);
    if (lane == 0) out[(long long)z * out_bstride + m] = s;
}

hipError_t launch_rowsum_conv(const uint8_t* x, int N, int H, int W, int Cs, int Cg, int cg_stride, int groups,
                              int oH, int oW, int kH, int kW, int sH, int sW, int dH, int dW,
                              int pad_t, int pad_l, int a_signed, int x_zp, int32_t* out,
                              long long out_bstride, hipStream_t s) {
    long long M = (long long)N * oH * oW;
    if (M <= 0) return hipSuccess;
    dim3 grid((unsigned)((M + 3) / 4), groups);
    hipLaunchKernelGGL(rowsum_conv_kernel, grid, dim3(256), 0, s, x, N, H, W, Cs, Cg, cg_stride, oH, oW, kH,
                       kW, sH, sW, dH, dW, pad_t, pad_l, a_signed, x_zp, out, out_bstride);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// ConvInteger on the pipelined implicit-GEMM kernel: the NCHW input as NHWC
// with every group's channels padded to a multiple of 16, and the weights
// packed per call (they are an input of the operator).

// ConvInteger's per-call preparation in one launch: the first blocks copy the
// NCHW input to group-padded NHWC, the rest pack the weights.
//
// Copy: one thread per (image, 4 consecutive pixels, 16-channel output chunk),
// the chunk index fastest so that the chunks of a pixel row are neighbouring
// lanes (whole-row stores). A thread loads 16 channel planes x 4 pixels as
// dwords (bytes when HW % 4 != 0 or x is not 4-byte aligned) and transposes
// them with byte permutes into 4 pixels x 16 channels.
__device__ __forceinline__ void ci_copy(const ConvIntPrepArgs& a, long long i) {
    const int cpp = a.G * a.Cgp / 16;     // 16-channel chunks per pixel
    const int qpi = (a.HW + 3) / 4;       // pixel quads per image
    if (i >= (long long)a.N * qpi * cpp) return;
    const int c = (int)(i % cpp);
    const long long t = i / cpp;
    const int q = (int)(t % qpi);
    const int n = (int)(t / qpi);
    const int z = c * 16 / a.Cgp, c0 = c * 16 - z * a.Cgp;
    const int p = 4 * q;
    const uint8_t* src = a.x + ((long long)n * a.G + z) * a.Cg * (long long)a.HW + p;
    const uint32_t fill4 = a.fill * 0x01010101u;
    uint32_t v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int ch = c0 + j;
        uint32_t d = fill4;
        if (ch < a.Cg) {
            const uint8_t* sp = src + (long long)ch * a.HW;
            if (a.vec) {
                d = *(const uint32_t*)sp;
            } else {
                d = 0;
                for (int b = 0; b < 4; ++b) d |= (p + b < a.HW ? (uint32_t)sp[b] : 0u) << (8 * b);
            }
        }
        v[j] = d;
    }
    uint8_t* dst = a.xs + ((long long)n * a.HW + p) * (a.G * a.Cgp) + (long long)z * a.Cgp + c0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        if (p + b >= a.HW) break;
        // byte b of v[4k .. 4k + 3] -> dword k
        const uint32_t sel = (uint32_t)b | ((uint32_t)(4 + b) << 8) | 0x0c0c0000u;
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = __builtin_amdgcn_perm(v[4 * k + 1], v[4 * k], sel);
            const uint32_t hi = __builtin_amdgcn_perm(v[4 * k + 3], v[4 * k + 2], sel);
            w[k] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
        }
        *(uint4*)(dst + (long long)b * (a.G * a.Cgp)) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// Pack: one block per packed row (z, n): the row's Kp bytes in (kh, kw, c)
// order, its column sum, the accumulator start c0 and the row-term coefficient
__device__ __forceinline__ void ci_pack(const ConvIntPrepArgs& a, int n, int z) {
    __shared__ int32_t part[4];
    const int oc = z * a.OCg + n;
    const int K = a.kH * a.kW * a.Cgp;
    const uint8_t bx = a.w_u8 ? 0x80 : 0;
    int8_t* row = a.wpack + ((long long)z * a.Np + packed_row_of_col(n)) * a.Kp;
    int32_t s = 0;
    for (int k = threadIdx.x; k < a.Kp; k += blockDim.x) {
        int8_t v = 0;
        if (n < a.OCg && k < K) {
            const int c = k % a.Cgp, t = k / a.Cgp;
            const int kh = t / a.kW, kw = t - kh * a.kW;
            if (c < a.Cg) v = (int8_t)(a.w[(((long long)oc * a.Cg + c) * a.kH + kh) * a.kW + kw] ^ bx);
        }
        row[k] = v;
        s += v;
    }
    for (int off = 32; off > 0; off >>= 1) s += __shfl_down(s, off, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        const int32_t cs = part[0] + part[1] + part[2] + part[3];
        const long long pi = (long long)z * a.Np + n;
        a.c0[pi] = (int32_t)(0u - (uint32_t)a.alpha * (uint32_t)cs);
        int coef = 0;
        if (n < a.OCg) coef = (a.w_u8 ? 128 : 0) - (a.w_zp_dev ? a.w_zp_dev[oc] : a.w_zp);
        a.row_coef[pi] = coef;
    }
}

__global__ __launch_bounds__(256) void conv_integer_prep_kernel(ConvIntPrepArgs a) {
    // block-uniform split: copy blocks first, then one block per packed row
    const int b = blockIdx.x;
    if (b < a.copy_blocks) {
        ci_copy(a, (long long)b * blockDim.x + threadIdx.x);
    } else {
        const int r = b - a.copy_blocks;
        ci_pack(a, r % a.Np, r / a.Np);
    }
}

hipError_t launch_conv_integer_prep(ConvIntPrepArgs a, hipStream_t s) {
    if (a.Cgp % 16 || a.Cg > a.Cgp || a.G <= 0 || a.OCg <= 0 || a.Np < a.OCg ||
        (long long)a.kH * a.kW * a.Cgp > a.Kp)
        return hipErrorInvalidValue;
    const long long total = (long long)a.N * ((a.HW + 3) / 4) * (a.G * a.Cgp / 16);
    const long long copy_blocks = (total + 255) / 256;
    const long long blocks = copy_blocks + (long long)a.Np * a.G;
    if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
    a.copy_blocks = (int)copy_blocks;
    a.vec = (a.HW % 4 == 0 && (((uintptr_t)a.x) & 3) == 0) ? 1 : 0;
    hipLaunchKernelGGL(conv_integer_prep_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
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
