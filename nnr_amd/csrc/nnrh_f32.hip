// nnrh_f32.hip -- fp32 glue kernels of the configuration graphs. They keep
// tensors resident in HBM between the int8 operators; none is a performance
// target and their parity bar is the reference's float tolerance (1e-3 abs,
// tensor_equal, src/nnr.cpp:557-563).
//   GlobalAveragePool (src/backend/cpu/global_pool.cpp), NCHW or NHWC input
//   Gemm / MatMul     (src/backend/cpu/Gemm.cpp, MatMul.cpp), row-major, on fp32 MFMA
//   Clip / Relu       (src/backend/cpu/Clip.cpp, Relu.cpp)
//   Add / Mul / Sub / Div with scalar or last-axis broadcast (binary_math.cpp)
//   Softmax, LayerNormalization over the last axis, Gelu (erf form), Transpose
//   (the BERT encoder's fp32 glue: Softmax.cpp, LayerNormalization.cpp,
//   Gelu.cpp, Transpose.cpp)
#include "nnrh_f32.h"
#include "nnrh_rq.h"


namespace nnrh {

// one wave per (n, c): mean over HW
__global__ __launch_bounds__(256) void gap_f32_kernel(const float* __restrict x, float* __restrict y,
                                                      int N, int C, int HW, int x_nhwc) {
    const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= (long long)N * C) return;
    const int n = (int)(row / C), c = (int)(row % C);
    float s = 0.0f;
    for (int i = lane; i < HW; i += 64) {
        long long idx = x_nhwc ? ((long long)n * HW + i) * C + c : row * HW + i;
        s += x[idx];
    }
    for (int off = 32; off > 0; off >>= 1) s += __shfl_down(s, off, 64);
    if (lane == 0) y[row] = s / (float)HW;
}

// NHWC: one thread per (n, c); consecutive threads read consecutive channels
__global__ __launch_bounds__(256) void gap_f32_nhwc_kernel(const float* __restrict x,
                                                           float* __restrict y, int N, int C,
                                                           int HW) {
    long long row = (long long)blockIdx.x * 256 + threadIdx.x;
    if (row >= (long long)N * C) return;
    const int n = (int)(row / C), c = (int)(row % C);
    const float* p = x + (long long)n * HW * C + c;
    float s = 0.0f;
    for (int i = 0; i < HW; ++i) s += p[(long long)i * C];
    y[row] = s / (float)HW;
}

// DequantizeLinear fused into GlobalAveragePool: every value is
// fl((float(q) - float(zp)) * s) (DequantizeLinear.cpp:133-152) and the sums
// run in the order of the fp32 kernels above, so the result equals
// DequantizeLinear followed by launch_gap_f32.
__device__ __forceinline__ float dq_one(const uint8_t* x, long long i, int sgn, float zpf, float sc) {
    const float q = sgn ? (float)(int)(int8_t)x[i] : (float)x[i];
    return (q - zpf) * sc;
}
__global__ __launch_bounds__(256) void gap_dq_nchw_kernel(const uint8_t* __restrict x, float* __restrict y,
                                                          int N, int C, int HW, int sgn, float zpf, float sc) {
    const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= (long long)N * C) return;
    float s = 0.0f;
    for (int i = lane; i < HW; i += 64) s += dq_one(x, row * HW + i, sgn, zpf, sc);
    for (int off = 32; off > 0; off >>= 1) s += __shfl_down(s, off, 64);
    if (lane == 0) y[row] = s / (float)HW;
}
__global__ __launch_bounds__(256) void gap_dq_nhwc_kernel(const uint8_t* __restrict x, float* __restrict y,
                                                          int N, int C, int HW, int sgn, float zpf, float sc) {
    const long long row = (long long)blockIdx.x * 256 + threadIdx.x;
    if (row >= (long long)N * C) return;
    const int n = (int)(row / C), c = (int)(row % C);
    const long long base = (long long)n * HW * C + c;
    float s = 0.0f;
    for (int i = 0; i < HW; ++i) s += dq_one(x, base + (long long)i * C, sgn, zpf, sc);
    y[row] = s / (float)HW;
}

// four consecutive channels per thread (one 4-byte load per pixel), each
// channel's sum in the same pixel order
__global__ __launch_bounds__(256) void gap_dq_nhwc4_kernel(const uint8_t* __restrict x, float* __restrict y,
                                                           int N, int C, int HW, int sgn, float zpf, float sc) {
    const int C4 = C >> 2;
    const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
    if (t >= (long long)N * C4) return;
    const int n = (int)(t / C4), cg = (int)(t - (long long)n * C4);
    const uint32_t* p = (const uint32_t*)(x + (long long)n * HW * C) + cg;
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto add = [&](uint32_t w) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float q = sgn ? (float)(int)(int8_t)(w >> (8 * j)) : (float)((w >> (8 * j)) & 0xffu);
            s[j] += (q - zpf) * sc;
        }
    };
    // 16 pixels' loads in flight at a time, then summed in pixel order
    int i = 0;
    for (; i + 16 <= HW; i += 16) {
        uint32_t w[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) w[u] = p[(long long)(i + u) * C4];
#pragma unroll
        for (int u = 0; u < 16; ++u) add(w[u]);
    }
    for (; i < HW; ++i) add(p[(long long)i * C4]);
    *(float4*)(y + (long long)n * C + 4 * cg) =
        make_float4(s[0] / (float)HW, s[1] / (float)HW, s[2] / (float)HW, s[3] / (float)HW);
}

hipError_t launch_gap_dq(const uint8_t* x, float* y, int N, int C, int HW, int x_nhwc, int x_signed,
                         float scale, int zp, hipStream_t s) {
    const long long rows = (long long)N * C;
    if (rows <= 0) return hipSuccess;
    if (x_nhwc && (C & 3) == 0 && (((uintptr_t)x | (uintptr_t)y) & 15) == 0) {
        const long long th = rows / 4;
        hipLaunchKernelGGL(gap_dq_nhwc4_kernel, dim3((unsigned)((th + 255) / 256)), dim3(256), 0, s, x, y, N, C,
                           HW, x_signed, (float)zp, scale);
        return hipGetLastError();
    }
    if (x_nhwc)
        hipLaunchKernelGGL(gap_dq_nhwc_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, x, y, N,
                           C, HW, x_signed, (float)zp, scale);
    else
        hipLaunchKernelGGL(gap_dq_nchw_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, x, y, N, C,
                           HW, x_signed, (float)zp, scale);
    return hipGetLastError();
}

hipError_t launch_gap_f32(const float* x, float* y, int N, int C, int HW, int x_nhwc,
                          hipStream_t s) {
    long long rows = (long long)N * C;
    if (rows <= 0) return hipSuccess;
    if (x_nhwc) {
        hipLaunchKernelGGL(gap_f32_nhwc_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s,
                           x, y, N, C, HW);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(gap_f32_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, x, y, N,
                       C, HW, x_nhwc);
    return hipGetLastError();
}

// Small fp32 GEMMs (too few 64x64 tiles to fill the chip, e.g. a
// classifier over one batch): Y = alpha * A[M][K] . op(B) + beta * Cb with
// fp32 MFMA 16x16x4. A block computes 32x32 outputs; its 4 waves take every
// 4th 64-wide K chunk and their partial sums are added in LDS in wave order.
// Within a chunk the contraction runs over k = 16 (l / 16) + step, so each
// lane reads 16 consecutive floats of its A row (and of its B row when B is
// stored [N][K]); rows and columns past M / N read a clamped row and are not
// stored.
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int TB>
__global__ __launch_bounds__(256) void gemm_f32_mfma_kernel(const float* __restrict A, const float* __restrict B,
                                                            const float* __restrict C, float* __restrict Y, int M,
                                                            int N, int K, float alpha, float beta, int c_mode) {
    __shared__ float red[3][32 * 32];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int lr = lane & 15, g = lane >> 4;
    const int m0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
    const float* ar[2] = {A + (long long)min(m0 + lr, M - 1) * K, A + (long long)min(m0 + 16 + lr, M - 1) * K};
    const int bn[2] = {min(n0 + lr, N - 1), min(n0 + 16 + lr, N - 1)};
    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i) acc[i][0] = acc[i][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto load = [&](int c, float (&a)[2][16], float (&b)[2][16]) {
        const int k0 = c * 64 + 16 * g;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 v = *(const float4*)(ar[t] + k0 + 4 * j);
                a[t][4 * j] = v.x; a[t][4 * j + 1] = v.y; a[t][4 * j + 2] = v.z; a[t][4 * j + 3] = v.w;
            }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            if (TB) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float4 v = *(const float4*)(B + (long long)bn[t] * K + k0 + 4 * j);
                    b[t][4 * j] = v.x; b[t][4 * j + 1] = v.y; b[t][4 * j + 2] = v.z; b[t][4 * j + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int st = 0; st < 16; ++st) b[t][st] = B[(long long)(k0 + st) * N + bn[t]];
            }
        }
    };
    auto mma = [&](const float (&a)[2][16], const float (&b)[2][16]) {
#pragma unroll
        for (int st = 0; st < 16; ++st)
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[mt][st], b[nt][st], acc[mt][nt], 0, 0, 0);
    };
    const int nch = K >> 6;
    float a0[2][16], b0[2][16], a1[2][16], b1[2][16];
    int c = w;
    if (c < nch) load(c, a0, b0);
    for (; c < nch; c += 8) {
        // the next chunk's loads are in flight while this one multiplies
        if (c + 4 < nch) load(c + 4, a1, b1);
        mma(a0, b0);
        if (c + 4 >= nch) break;
        if (c + 8 < nch) load(c + 8, a0, b0);
        mma(a1, b1);
    }
    // acc[mt][nt][i] = partial Y[m0 + 16 mt + 4 g + i][n0 + 16 nt + lr]
    if (w > 0) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i) red[w - 1][(16 * mt + 4 * g + i) * 32 + 16 * nt + lr] = acc[mt][nt][i];
    }
    __syncthreads();
    if (w > 0) return;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 16 * mt + 4 * g + i, cl = 16 * nt + lr;
                const int m = m0 + r, n = n0 + cl;
                float v = acc[mt][nt][i];
                v = v + red[0][r * 32 + cl];
                v = v + red[1][r * 32 + cl];
                v = v + red[2][r * 32 + cl];
                if (m >= M || n >= N) continue;
                v = alpha * v;
                if (c_mode != 0 && beta != 0.0f) {
                    const float cb = c_mode == 1 ? C[0]
                                     : c_mode == 2 ? C[n]
                                     : c_mode == 3 ? C[(long long)m * N + n]
                                                   : C[m];
                    v = v + beta * cb;
                }
                Y[(long long)m * N + n] = v;
            }
}

// Any fp32 GEMM: Y(z)[m][n] = alpha * sum_k A(z)(m, k) B(z)(k, n) (+ beta *
// the broadcast C), with element strides for A and B (so transposes, head
// splits and row strides are strides) and a two-level batch z = z1 * nb2 +
// z2 whose offsets are z1 * s1 + z2 * s2 per operand. 64 x 64 output tiles,
// 4 waves of 32 x 32 (fp32 MFMA 16x16x4); K in steps of 16 staged through
// LDS, loaded along whichever of an operand's two strides is 1; elements
// past M, N or K read 0.
struct GemmF32Gen {
    const float* A; const float* B; const float* C; float* Y;
    int M, N, K, nb2;
    long long sam, sak, as1, as2;   // A(m, k) = A[m * sam + k * sak]
    long long sbk, sbn, bs1, bs2;   // B(k, n) = B[k * sbk + n * sbn]
    long long ldy, ys1, ys2;        // Y[m * ldy + n]
    float alpha, beta;
    int c_mode;                     // 0 none, 1 scalar, 2 per column, 3 [M][N], 4 per row
};

__global__ __launch_bounds__(256) void gemm_f32_gen_kernel(GemmF32Gen p) {
    __shared__ float As[16][64 + 1], Bs[16][64 + 1];   // [k][m], [k][n]
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lr = lane & 15, g = lane >> 4;
    const int wm = w >> 1, wn = w & 1;
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const long long z = blockIdx.z, z1 = z / p.nb2, z2 = z - z1 * p.nb2;
    const float* A = p.A + z1 * p.as1 + z2 * p.as2;
    const float* B = p.B + z1 * p.bs1 + z2 * p.bs2;
    // element (r, c) of a 64 x 16 operand tile for thread slot e: along k
    // when the k stride is 1, else along m / n
    const bool a_k1 = p.sak == 1, b_k1 = p.sbk == 1;
    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i) acc[i][0] = acc[i][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < p.K; k0 += 16) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = tid + 256 * e;
            const int r = a_k1 ? i >> 4 : i & 63, c = a_k1 ? i & 15 : i >> 6;   // r: m, c: k
            const int m = m0 + r, k = k0 + c;
            As[c][r] = (m < p.M && k < p.K) ? A[(long long)m * p.sam + (long long)k * p.sak] : 0.0f;
            const int rn = b_k1 ? i >> 4 : i & 63, ck = b_k1 ? i & 15 : i >> 6;  // rn: n, ck: k
            const int n = n0 + rn, kb = k0 + ck;
            Bs[ck][rn] = (n < p.N && kb < p.K) ? B[(long long)kb * p.sbk + (long long)n * p.sbn] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const int k = 4 * st + g;
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(As[k][wm * 32 + 16 * mt + lr],
                                                                       Bs[k][wn * 32 + 16 * nt + lr], acc[mt][nt],
                                                                       0, 0, 0);
        }
        __syncthreads();
    }
    float* Y = p.Y + z1 * p.ys1 + z2 * p.ys2;
    // acc[mt][nt][i] = Y[m0 + 32 wm + 16 mt + 4 g + i][n0 + 32 wn + 16 nt + lr]
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + 32 * wm + 16 * mt + 4 * g + i, n = n0 + 32 * wn + 16 * nt + lr;
                if (m >= p.M || n >= p.N) continue;
                float v = p.alpha * acc[mt][nt][i];
                if (p.c_mode != 0 && p.beta != 0.0f) {
                    const float cb = p.c_mode == 1 ? p.C[0]
                                     : p.c_mode == 2 ? p.C[n]
                                     : p.c_mode == 3 ? p.C[(long long)m * p.N + n]
                                                     : p.C[m];
                    v = v + p.beta * cb;
                }
                Y[(long long)m * p.ldy + n] = v;
            }
}

hipError_t launch_gemm_f32_gen(const GemmF32Gen& p, long long batch, hipStream_t s) {
    if (p.M <= 0 || p.N <= 0 || batch <= 0) return hipSuccess;
    if (p.nb2 <= 0 || batch > 65535 || (p.M + 63) / 64 > 65535) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((p.N + 63) / 64), (unsigned)((p.M + 63) / 64), (unsigned)batch);
    hipLaunchKernelGGL(gemm_f32_gen_kernel, grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_gemm_f32_batched(const float* A, const float* B, const float* C, float* Y, int M,
                                   int N, int K, int transA, int transB, float alpha, float beta,
                                   int c_mode, int batch, long long a_bstride, long long b_bstride,
                                   long long y_bstride, hipStream_t s) {
    if (M <= 0 || N <= 0 || batch <= 0) return hipSuccess;
    const long long tiles64 = (long long)((M + 63) / 64) * ((N + 63) / 64);
    if (batch == 1 && !transA && K > 0 && (K & 63) == 0 && tiles64 < 512 && M <= 65535 * 32 &&
        (((uintptr_t)A | (uintptr_t)B) & 15) == 0) {
        const dim3 grid((unsigned)((N + 31) / 32), (unsigned)((M + 31) / 32));
        if (transB)
            hipLaunchKernelGGL(gemm_f32_mfma_kernel<1>, grid, dim3(256), 0, s, A, B, C, Y, M, N, K, alpha, beta,
                               c_mode);
        else
            hipLaunchKernelGGL(gemm_f32_mfma_kernel<0>, grid, dim3(256), 0, s, A, B, C, Y, M, N, K, alpha, beta,
                               c_mode);
        return hipGetLastError();
    }
    // every other shape: the general kernel (A [M][K] or, transposed,
    // [K][M]; B [K][N] or [N][K])
    GemmF32Gen p{};
    p.A = A; p.B = B; p.C = C; p.Y = Y;
    p.M = M; p.N = N; p.K = K; p.nb2 = 1;
    p.sam = transA ? 1 : K; p.sak = transA ? M : 1; p.as1 = a_bstride;
    p.sbk = transB ? 1 : N; p.sbn = transB ? K : 1; p.bs1 = b_bstride;
    p.ldy = N; p.ys1 = y_bstride;
    p.alpha = alpha; p.beta = beta; p.c_mode = c_mode;
    return launch_gemm_f32_gen(p, batch, s);
}

hipError_t launch_gemm_f32(const float* A, const float* B, const float* C, float* Y, int M, int N,
                           int K, int transA, int transB, float alpha, float beta, int c_mode,
                           hipStream_t s) {
    return launch_gemm_f32_batched(A, B, C, Y, M, N, K, transA, transB, alpha, beta, c_mode, 1, 0, 0,
                                   0, s);
}

__global__ __launch_bounds__(256) void clip_f32_kernel(const float* __restrict x, float* __restrict y,
                                                       long long n, float lo, float hi) {
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (long long)gridDim.x * 256) {
        float v = x[i];
        v = v < lo ? lo : v;
        y[i] = v > hi ? hi : v;
    }
}

hipError_t launch_clip_f32(const float* x, float* y, long long n, float lo, float hi,
                           hipStream_t s) {
    if (n <= 0) return hipSuccess;
    long long b = (n + 255) / 256;
    if (b > 65536) b = 65536;
    hipLaunchKernelGGL(clip_f32_kernel, dim3((unsigned)b), dim3(256), 0, s, x, y, n, lo, hi);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// HardSwish (src/backend/cpu/HardSwish.cpp:18-50; vec_ops_avx512.h:74-117):
// y = x * clamp(x / 6 + 0.5, 0, 1) with the reference's two expressions.
// 16-wide body (the first n - n % 16 elements): u = fl(fl(x * fl(1/6)) + 0.5),
// t = min_ps(max_ps(u, 0), 1) -- max_ps / min_ps return their second operand
// unless the first compares greater / smaller, so a NaN u gives t = 0.
// Scalar tail: w = fl(fl(x / 6) + 0.5), t = std::max(0, std::min(1, w)) -- a
// NaN w gives t = 1. As a producer's fused post-op (post_op), x is first
// fl(x + 0.0f), the zero bias the reference's bias_hardswish adds.
__global__ __launch_bounds__(256) void hardswish_f32_kernel(const float* __restrict x, float* __restrict y,
                                                            long long n, long long body, int post_op) {
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (long long)gridDim.x * 256) {
        float v = x[i];
        if (post_op) v = v + 0.0f;
        float t;
        if (i < body) {
            const float u = v * (1.0f / 6.0f) + 0.5f;
            const float m = u > 0.0f ? u : 0.0f;
            t = m < 1.0f ? m : 1.0f;
        } else {
            const float w = v / 6.0f + 0.5f;
            const float m = w < 1.0f ? w : 1.0f;
            t = 0.0f < m ? m : 0.0f;
        }
        y[i] = v * t;
    }
}

hipError_t launch_hardswish_f32(const float* x, float* y, long long n, int post_op, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    long long b = (n + 255) / 256;
    if (b > 65536) b = 65536;
    hipLaunchKernelGGL(hardswish_f32_kernel, dim3((unsigned)b), dim3(256), 0, s, x, y, n, n - n % 16, post_op);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// y = a (op) b; b_mode: 0 same shape, 1 scalar, 2 broadcast over the last axis
// (b has D elements); b_first swaps the operands (b op a) for Sub / Div.
__global__ __launch_bounds__(256) void binary_f32_kernel(const float* __restrict a,
                                                         const float* __restrict b,
                                                         float* __restrict y, long long n, int D,
                                                         int b_mode, int op, int b_first) {
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (long long)gridDim.x * 256) {
        const float av = a[i];
        const float bv = b_mode == 0 ? b[i] : (b_mode == 1 ? b[0] : b[i % D]);
        const float l = b_first ? bv : av, r = b_first ? av : bv;
        float v;
        if (op == 0) v = l + r;
        else if (op == 1) v = l * r;
        else if (op == 2) v = l - r;
        else v = l / r;
        y[i] = v;
    }
}

hipError_t launch_binary_f32(const float* a, const float* b, float* y, long long n, int D, int b_mode,
                             int op, int b_first, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    long long blocks = (n + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(binary_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a, b, y, n,
                       D > 0 ? D : 1, b_mode, op, b_first);
    return hipGetLastError();
}

// softmax over rows of D (one wave per row): exp(x - max) / sum
__global__ __launch_bounds__(256) void softmax_f32_kernel(const float* __restrict x,
                                                          float* __restrict y, long long rows, int D) {
    const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* xr = x + row * D;
    float* yr = y + row * D;
    float m = -INFINITY;
    for (int i = lane; i < D; i += 64) m = fmaxf(m, xr[i]);
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    float sum = 0.0f;
    for (int i = lane; i < D; i += 64) sum += expf(xr[i] - m);
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    const float inv = 1.0f / sum;
    for (int i = lane; i < D; i += 64) yr[i] = expf(xr[i] - m) * inv;
}

// the same with each input first multiplied by `scale` (fl(x * scale), what
// a Mul by a constant before the Softmax writes)
__global__ __launch_bounds__(256) void softmax_scaled_f32_kernel(const float* __restrict x,
                                                                 float* __restrict y, long long rows, int D,
                                                                 float scale) {
    const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* xr = x + row * D;
    float* yr = y + row * D;
    float m = -INFINITY;
    for (int i = lane; i < D; i += 64) m = fmaxf(m, xr[i] * scale);
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    float sum = 0.0f;
    for (int i = lane; i < D; i += 64) sum += expf(xr[i] * scale - m);
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    const float inv = 1.0f / sum;
    for (int i = lane; i < D; i += 64) yr[i] = expf(xr[i] * scale - m) * inv;
}

hipError_t launch_softmax_f32(const float* x, float* y, long long rows, int D, hipStream_t s) {
    if (rows <= 0 || D <= 0) return hipSuccess;
    hipLaunchKernelGGL(softmax_f32_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, x, y, rows,
                       D);
    return hipGetLastError();
}

// LayerNormalization over rows of D (one wave per row, 4 rows a block):
// mean, then the mean of squared deviations, then (v - mean) * inv * gamma
// (+ beta). With `r` the row is fl(x + r) of two same-shape inputs (a
// residual Add folded in), the same bits the Add would have stored. With
// `parts`, pair i receives the (min, max) of the outputs of rows 4 i .. 4 i
// + 3 (0 when smaller / larger), for a DynamicQuantizeLinear that reads y.
// Every wave of the block reaches the pairs' barrier (a wave past the last
// row brings the pair (0, 0)).
__device__ __forceinline__ void ln_minmax_store(float mn, float mx, float* parts, int lane) {
    __shared__ float2 wp[4];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        mn = fminf(mn, __shfl_xor(mn, off, 64));
        mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    }
    if (lane == 0) wp[threadIdx.x >> 6] = make_float2(mn, mx);
    __syncthreads();
    if (threadIdx.x == 0)
        *(float2*)(parts + 2 * blockIdx.x) =
            make_float2(fminf(fminf(wp[0].x, wp[1].x), fminf(wp[2].x, wp[3].x)),
                        fmaxf(fmaxf(wp[0].y, wp[1].y), fmaxf(wp[2].y, wp[3].y)));
}

// value of chain byte b in a column with bias bn (DqCodes)
__device__ __forceinline__ float dq_codes_value(uint32_t b, float zp_f, float scale, float bn) {
    const float d = ((float)b - zp_f) * scale;
    return d + bn;
}
// 4 consecutive columns: bytes of one dword, their 4 biases
__device__ __forceinline__ float4 dq_codes_value4(uint32_t w, float zp_f, float scale, float4 bn) {
    return make_float4(dq_codes_value(w & 0xffu, zp_f, scale, bn.x), dq_codes_value((w >> 8) & 0xffu, zp_f, scale, bn.y),
                       dq_codes_value((w >> 16) & 0xffu, zp_f, scale, bn.z), dq_codes_value(w >> 24, zp_f, scale, bn.w));
}

// the row in registers: V float4 per lane (D % 4 == 0, D <= 256 V, 16-byte
// aligned rows; CODES: x given as chain bytes, 4-byte aligned rows); one
// read of x (and r), one write of y
template <int V, bool CODES>
__global__ __launch_bounds__(256) void layernorm_reg_kernel(const float* __restrict x, DqCodes xq,
                                                            const float* __restrict r,
                                                            const float* __restrict gamma,
                                                            const float* __restrict beta,
                                                            float* __restrict y, long long rows, int D,
                                                            float eps, float* __restrict parts) {
    const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const bool live = row < rows;   // (a wave past the last row still takes the pairs' barrier)
    const int D4 = live ? D >> 2 : 0;
    const float4* xr = (const float4*)(x + row * D);
    const uint32_t* xqr = (const uint32_t*)(xq.q + row * D);
    const float zp_f = (float)xq.zp;
    const float4* rr = r ? (const float4*)(r + row * D) : nullptr;
    float4 v[V];
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int c = lane + 64 * j;
        if (c < D4) {
            if constexpr (CODES) v[j] = dq_codes_value4(xqr[c], zp_f, xq.scale, ((const float4*)xq.bias)[c]);
            else v[j] = xr[c];
            if (rr) {
                const float4 t = rr[c];
                v[j].x = v[j].x + t.x; v[j].y = v[j].y + t.y;
                v[j].z = v[j].z + t.z; v[j].w = v[j].w + t.w;
            }
            sum += v[j].x + v[j].y + v[j].z + v[j].w;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    const float mean = sum / (float)D;
    float sq = 0.0f;
#pragma unroll
    for (int j = 0; j < V; ++j)
        if (lane + 64 * j < D4) {
            const float a = v[j].x - mean, b = v[j].y - mean, c = v[j].z - mean, d = v[j].w - mean;
            sq += a * a + b * b + c * c + d * d;
        }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off, 64);
    const float inv = 1.0f / sqrtf(sq / (float)D + eps);
    const float4* g4 = (const float4*)gamma;
    const float4* b4 = (const float4*)beta;
    float4* yr = (float4*)(y + row * D);
    float mn = 0.0f, mx = 0.0f;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int c = lane + 64 * j;
        if (c < D4) {
            const float4 gm = g4[c];
            float4 o;
            o.x = (v[j].x - mean) * inv * gm.x; o.y = (v[j].y - mean) * inv * gm.y;
            o.z = (v[j].z - mean) * inv * gm.z; o.w = (v[j].w - mean) * inv * gm.w;
            if (beta) {
                const float4 bt = b4[c];
                o.x = o.x + bt.x; o.y = o.y + bt.y; o.z = o.z + bt.z; o.w = o.w + bt.w;
            }
            yr[c] = o;
            mn = fminf(mn, fminf(fminf(o.x, o.y), fminf(o.z, o.w)));
            mx = fmaxf(mx, fmaxf(fmaxf(o.x, o.y), fmaxf(o.z, o.w)));
        }
    }
    if (parts) ln_minmax_store(mn, mx, parts, lane);
}

// any D or alignment: three strided passes over the row
template <bool CODES>
__global__ __launch_bounds__(256) void layernorm_f32_kernel(const float* __restrict x, DqCodes xq,
                                                            const float* __restrict r,
                                                            const float* __restrict gamma,
                                                            const float* __restrict beta,
                                                            float* __restrict y, long long rows, int D,
                                                            float eps, float* __restrict parts) {
    const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const bool live = row < rows;   // (a wave past the last row still takes the pairs' barrier)
    const int Dl = live ? D : 0;
    const float* xr = x + row * D;
    const uint8_t* xqr = xq.q + row * D;
    const float zp_f = (float)xq.zp;
    const float* rr = r ? r + row * D : nullptr;
    auto xv = [&](int i) {
        if constexpr (CODES) return dq_codes_value(xqr[i], zp_f, xq.scale, xq.bias[i]);
        else return xr[i];
    };
    auto at = [&](int i) { return rr ? xv(i) + rr[i] : xv(i); };
    float* yr = y + row * D;
    float sum = 0.0f;
    for (int i = lane; i < Dl; i += 64) sum += at(i);
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    const float mean = sum / (float)D;
    float sq = 0.0f;
    for (int i = lane; i < Dl; i += 64) {
        const float d = at(i) - mean;
        sq += d * d;
    }
    for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off, 64);
    const float inv = 1.0f / sqrtf(sq / (float)D + eps);
    float mn = 0.0f, mx = 0.0f;
    for (int i = lane; i < Dl; i += 64) {
        float v = (at(i) - mean) * inv * gamma[i];
        if (beta) v = v + beta[i];
        yr[i] = v;
        mn = fminf(mn, v);
        mx = fmaxf(mx, v);
    }
    if (parts) ln_minmax_store(mn, mx, parts, lane);
}

template <bool CODES>
static hipError_t launch_layernorm_any(const float* x, const DqCodes& xq, const float* r, const float* gamma,
                                       const float* beta, float* y, long long rows, int D, float eps, float* parts,
                                       hipStream_t s) {
    if (rows <= 0 || D <= 0) return hipSuccess;
    const dim3 grid((unsigned)((rows + 3) / 4));
    const uintptr_t al = (uintptr_t)x | (uintptr_t)r | (uintptr_t)gamma | (uintptr_t)beta | (uintptr_t)y |
                         (CODES ? (uintptr_t)xq.bias : 0);
    const bool q4 = !CODES || ((uintptr_t)xq.q & 3) == 0;
    const int v = (D + 255) / 256;
    if ((D & 3) == 0 && (al & 15) == 0 && q4 && v <= 8) {
        switch (v) {
#define NNRH_LN_CASE(V)                                                                                        \
    case V:                                                                                                    \
        hipLaunchKernelGGL((layernorm_reg_kernel<V, CODES>), grid, dim3(256), 0, s, x, xq, r, gamma, beta, y, \
                           rows, D, eps, parts);                                                               \
        return hipGetLastError();
            NNRH_LN_CASE(1) NNRH_LN_CASE(2) NNRH_LN_CASE(3) NNRH_LN_CASE(4)
            NNRH_LN_CASE(5) NNRH_LN_CASE(6) NNRH_LN_CASE(7) NNRH_LN_CASE(8)
#undef NNRH_LN_CASE
        }
    }
    hipLaunchKernelGGL((layernorm_f32_kernel<CODES>), grid, dim3(256), 0, s, x, xq, r, gamma, beta, y, rows, D, eps,
                       parts);
    return hipGetLastError();
}

hipError_t launch_layernorm_f32(const float* x, const float* r, const float* gamma, const float* beta, float* y,
                                long long rows, int D, float eps, float* parts, hipStream_t s) {
    return launch_layernorm_any<false>(x, DqCodes{nullptr, 0, 0.0f, nullptr}, r, gamma, beta, y, rows, D, eps, parts,
                                       s);
}

hipError_t launch_layernorm_codes_f32(const DqCodes& xq, const float* r, const float* gamma, const float* beta,
                                      float* y, long long rows, int D, float eps, float* parts, hipStream_t s) {
    return launch_layernorm_any<true>(nullptr, xq, r, gamma, beta, y, rows, D, eps, parts, s);
}

// Gelu, erf form: 0.5 x (1 + erf(x / sqrt(2)))
__global__ __launch_bounds__(256) void gelu_f32_kernel(const float* __restrict x, float* __restrict y,
                                                       long long n) {
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (long long)gridDim.x * 256)
        y[i] = gelu_erf(x[i]);
}

// Cast to float (src/backend/cpu/Cast.cpp, Cast_array: (float)x, so int32
// rounds to the nearest float, ties to even); dt 0 uint8, 1 int8, 2 int32
__global__ __launch_bounds__(256) void cast_to_f32_kernel(const void* __restrict x, int dt, float* __restrict y,
                                                          long long n) {
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256) {
        float v;
        if (dt == 2) v = (float)((const int32_t*)x)[i];
        else if (dt == 1) v = (float)((const int8_t*)x)[i];
        else v = (float)((const uint8_t*)x)[i];
        y[i] = v;
    }
}

hipError_t launch_cast_to_f32(const void* x, int dt, float* y, long long n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    long long b = (n + 255) / 256;
    if (b > 65536) b = 65536;
    hipLaunchKernelGGL(cast_to_f32_kernel, dim3((unsigned)b), dim3(256), 0, s, x, dt, y, n);
    return hipGetLastError();
}

hipError_t launch_gelu_f32(const float* x, float* y, long long n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    long long blocks = (n + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(gelu_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, y, n);
    return hipGetLastError();
}

// Transpose of a tensor of up to 6 axes: out axis i is in axis perm[i]
struct TransposeArgs {
    int ndim;
    long long out_dims[6];
    long long in_strides_for_out[6];   // stride in x of out axis i
};

__global__ __launch_bounds__(256) void transpose_f32_kernel(const float* __restrict x,
                                                            float* __restrict y, long long n,
                                                            TransposeArgs t) {
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (long long)gridDim.x * 256) {
        long long r = i, src = 0;
        for (int d = t.ndim - 1; d >= 0; --d) {
            const long long c = r % t.out_dims[d];
            r /= t.out_dims[d];
            src += c * t.in_strides_for_out[d];
        }
        y[i] = x[src];
    }
}

hipError_t launch_transpose_f32(const float* x, float* y, int ndim, const int* in_dims, const int* perm,
                                hipStream_t s) {
    if (ndim < 1 || ndim > 6) return hipErrorInvalidValue;
    TransposeArgs t{};
    t.ndim = ndim;
    long long in_strides[6];
    long long st = 1, n = 1;
    for (int d = ndim - 1; d >= 0; --d) {
        in_strides[d] = st;
        st *= in_dims[d];
    }
    for (int d = 0; d < ndim; ++d) {
        if (perm[d] < 0 || perm[d] >= ndim) return hipErrorInvalidValue;
        t.out_dims[d] = in_dims[perm[d]];
        t.in_strides_for_out[d] = in_strides[perm[d]];
        n *= t.out_dims[d];
    }
    if (n <= 0) return hipSuccess;
    long long blocks = (n + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(transpose_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, y, n, t);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Multi-head attention on [B][S][H*hd] fp32 (com.microsoft MultiHeadAttention
// semantics, src/backend/cpu/MultiHeadAttention.cpp): per (b, h) the head's
// rows are read in place (row stride H*hd), scores = Q K^T into a [B][H][S][S]
// workspace, P = softmax(scale * scores) over the key axis, then P V is
// written straight into the output's head columns: two strided GEMMs over a
// (batch, head) grid; no transposes are materialized.
size_t mha_workspace_bytes(int B, int S, int nh) { return sizeof(float) * (size_t)B * nh * S * S; }

// ---------------------------------------------------------------------------
// Fused attention for head size 64 and S <= 128: one block per (batch, head),
// K and V of the head staged in LDS, 4 waves of 32 queries. Scores come from
// fp32 MFMA 16x16x4 as S^T tiles (t rows, s columns): lane l holds
// S^T[16 tt + 4 (l / 16) + i][16 ts + l % 16] in register i, which is exactly
// the A operand of the second product P V when its contraction index runs
// over t = 16 tt + 4 (l / 16) + i. The first product contracts d in the order
// d = 16 (l / 16) + step, so every lane reads 16 consecutive floats of its K
// row and Q row. Softmax of the scaled scores per query column, normalized
// before P V (the order of Softmax then MatMul); padded t rows are -inf.
constexpr int MHA_KP = 68;   // K row stride in LDS (floats): rows 16 bytes apart in the banks

// parts (optional): one (min, max) pair per wave, at 2 (4 blockIdx.x + wave),
// of the values the wave stores (0 stands in for nothing, as for every
// producer that feeds a DynamicQuantizeLinear, whose range includes 0)
// CODES: q, k, v given as chain bytes (DqCodes; columns = the hidden axis),
// each element formed as the producing GEMM's epilogue would have stored it
template <bool CODES>
__global__ __launch_bounds__(256, 3) void mha_fused_hd64_kernel(const float* __restrict q, const float* __restrict k,
                                                             const float* __restrict v, DqCodes qq, DqCodes kq,
                                                             DqCodes vq, float* __restrict y,
                                                             int S, int Hd, int nh, float scale,
                                                             float* __restrict parts) {
    // one buffer: K (row stride MHA_KP) for the scores, then V (stride 64)
    __shared__ __attribute__((aligned(16))) float ks[128 * MHA_KP];
    float* const vs = ks;
    const int b = blockIdx.x / nh, h = blockIdx.x - b * nh;
    const long long base = (long long)b * S * Hd + (long long)h * 64;
    const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
    // 4 elements of row t, columns h * 64 + c .. + 3, of an input
    auto load4 = [&](const float* x, const DqCodes& xq, long long off, int c) -> float4 {
        if constexpr (CODES)
            return dq_codes_value4(*(const uint32_t*)(xq.q + off), (float)xq.zp, xq.scale,
                                   *(const float4*)(xq.bias + h * 64 + c));
        else
            return *(const float4*)(x + off);
    };
    // K: all 8 of a thread's 16-byte pieces in flight before the LDS writes
    {
        float4 kv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = threadIdx.x + 256 * j;
            const int t = i >> 4, c = (i & 15) * 4;
            kv[j] = t < S ? load4(k, kq, base + (long long)t * Hd + c, c) : zero4;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = threadIdx.x + 256 * j;
            *(float4*)(ks + (i >> 4) * MHA_KP + (i & 15) * 4) = kv[j];
        }
    }
    // CODES: V's bytes (4 per dword, 8 dwords a thread) load now, with K's
    // and Q's, and become values only when V takes the LDS buffer
    uint32_t vpre[CODES ? 8 : 1];
    if constexpr (CODES) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = threadIdx.x + 256 * j;
            const int t = i >> 4, c = (i & 15) * 4;
            vpre[j] = t < S ? *(const uint32_t*)(vq.q + base + (long long)t * Hd + c) : 0u;
        }
    }
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int lr = lane & 15, g = lane >> 4;
    const int s0 = 32 * w;   // this wave's first query
    // Q[s][16 g .. 16 g + 15] of the wave's two query tiles
    float qf[2][16];
#pragma unroll
    for (int ts = 0; ts < 2; ++ts) {
        const int sq = s0 + 16 * ts + lr;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 t4 = sq < S ? load4(q, qq, base + (long long)sq * Hd + 16 * g + 4 * j, 16 * g + 4 * j) : zero4;
            qf[ts][4 * j] = t4.x; qf[ts][4 * j + 1] = t4.y; qf[ts][4 * j + 2] = t4.z; qf[ts][4 * j + 3] = t4.w;
        }
    }
    __syncthreads();
    const bool active = s0 < S;   // a wave with no query still takes every barrier

    f32x4 acc[8][2];
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) {
        acc[tt][0] = f32x4{0.f, 0.f, 0.f, 0.f};
        acc[tt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
        float kf[16];
        const float* kr = ks + (16 * tt + lr) * MHA_KP + 16 * g;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 t4 = *(const float4*)(kr + 4 * j);
            kf[4 * j] = t4.x; kf[4 * j + 1] = t4.y; kf[4 * j + 2] = t4.z; kf[4 * j + 3] = t4.w;
        }
#pragma unroll
        for (int st = 0; st < 16; ++st) {
            acc[tt][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[st], qf[0][st], acc[tt][0], 0, 0, 0);
            acc[tt][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[st], qf[1][st], acc[tt][1], 0, 0, 0);
        }
    }
    // softmax over t of fl(score * scale), per query column
#pragma unroll
    for (int ts = 0; ts < 2; ++ts) {
        float m = -INFINITY;
#pragma unroll
        for (int tt = 0; tt < 8; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float x = 16 * tt + 4 * g + i < S ? acc[tt][ts][i] * scale : -INFINITY;
                acc[tt][ts][i] = x;
                m = fmaxf(m, x);
            }
        m = fmaxf(m, __shfl_xor(m, 16, 64));
        m = fmaxf(m, __shfl_xor(m, 32, 64));
        float sum = 0.0f;
#pragma unroll
        for (int tt = 0; tt < 8; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float e = expf(acc[tt][ts][i] - m);
                acc[tt][ts][i] = e;
                sum += e;
            }
        sum += __shfl_xor(sum, 16, 64);
        sum += __shfl_xor(sum, 32, 64);
        const float inv = 1.0f / sum;
#pragma unroll
        for (int tt = 0; tt < 8; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[tt][ts][i] = acc[tt][ts][i] * inv;
    }
    // every wave's scores are done with K: V takes the buffer
    __syncthreads();
    if constexpr (CODES) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = threadIdx.x + 256 * j;
            const int t = i >> 4, c = (i & 15) * 4;
            *(float4*)(vs + t * 64 + c) =
                t < S ? dq_codes_value4(vpre[j], (float)vq.zp, vq.scale, *(const float4*)(vq.bias + h * 64 + c))
                      : zero4;
        }
    } else {
        for (int i = threadIdx.x; i < 128 * 16; i += 256) {
            const int t = i >> 4, c = (i & 15) * 4;
            const long long off = base + (long long)t * Hd + c;
            *(float4*)(vs + t * 64 + c) = t < S ? load4(v, vq, off, c) : zero4;
        }
    }
    __syncthreads();
    if (!active) {   // (after the last barrier)
        if (parts && lane == 0) *(float2*)(parts + 2 * (4 * blockIdx.x + w)) = make_float2(0.0f, 0.0f);
        return;
    }
    // O[s][d] = sum_t P[s][t] V[t][d]; output tile td holds d = 4 (l % 16) + td
    f32x4 o[2][4];
#pragma unroll
    for (int ts = 0; ts < 2; ++ts)
#pragma unroll
        for (int td = 0; td < 4; ++td) o[ts][td] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int tt = 0; tt < 8; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 vv = *(const float4*)(vs + (16 * tt + 4 * g + i) * 64 + 4 * lr);
            const float vb[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
            for (int ts = 0; ts < 2; ++ts)
#pragma unroll
                for (int td = 0; td < 4; ++td)
                    o[ts][td] = __builtin_amdgcn_mfma_f32_16x16x4f32(acc[tt][ts][i], vb[td], o[ts][td], 0, 0, 0);
        }
    // o[ts][td][i] = O[s0 + 16 ts + 4 g + i][4 lr + td]
    float mn = 0.0f, mx = 0.0f;
#pragma unroll
    for (int ts = 0; ts < 2; ++ts)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int sq = s0 + 16 * ts + 4 * g + i;
            if (sq < S) {
                *(float4*)(y + base + (long long)sq * Hd + 4 * lr) =
                    make_float4(o[ts][0][i], o[ts][1][i], o[ts][2][i], o[ts][3][i]);
#pragma unroll
                for (int td = 0; td < 4; ++td) {
                    mn = fminf(mn, o[ts][td][i]);
                    mx = fmaxf(mx, o[ts][td][i]);
                }
            }
        }
    if (parts) {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            mn = fminf(mn, __shfl_xor(mn, off, 64));
            mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        }
        if (lane == 0) *(float2*)(parts + 2 * (4 * blockIdx.x + w)) = make_float2(mn, mx);
    }
}

hipError_t launch_mha_codes_f32(const DqCodes& q, const DqCodes& k, const DqCodes& v, float* y, int B, int S,
                                int Hd, int nh, float scale, float* parts, hipStream_t s) {
    if (B <= 0 || S <= 0) return hipSuccess;
    const uintptr_t a4 = (uintptr_t)q.q | (uintptr_t)k.q | (uintptr_t)v.q;
    const uintptr_t a16 = (uintptr_t)y | (uintptr_t)q.bias | (uintptr_t)k.bias | (uintptr_t)v.bias;
    if (!mha_fused_shape(S, Hd, nh) || (a4 & 3) || (a16 & 15)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mha_fused_hd64_kernel<true>, dim3((unsigned)(B * nh)), dim3(256), 0, s, nullptr, nullptr,
                       nullptr, q, k, v, y, S, Hd, nh, scale, parts);
    return hipGetLastError();
}

int mha_minmax_pairs(int B, int S, int Hd, int nh) {
    if (!mha_fused_shape(S, Hd, nh) || B <= 0) return 0;
    const long long p = 4LL * B * nh;
    return p <= 0x7fffffffLL ? (int)p : 0;
}

bool mha_fused_shape(int S, int Hd, int nh) { return nh > 0 && Hd == 64 * nh && S <= 128; }

bool mha_fused_ok(const float* q, const float* k, const float* v, const float* y, int S, int Hd, int nh) {
    const uintptr_t al = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)y;
    return mha_fused_shape(S, Hd, nh) && (al & 15) == 0;
}

hipError_t launch_mha_f32(const float* q, const float* k, const float* v, float* y, int B, int S, int Hd, int nh,
                          float scale, float* parts, void* ws, hipStream_t s) {
    if (B <= 0 || S <= 0) return hipSuccess;
    if (nh <= 0 || Hd % nh) return hipErrorInvalidValue;
    if (mha_fused_ok(q, k, v, y, S, Hd, nh)) {
        const DqCodes none{nullptr, 0, 0.0f, nullptr};
        hipLaunchKernelGGL(mha_fused_hd64_kernel<false>, dim3((unsigned)(B * nh)), dim3(256), 0, s, q, k, v, none,
                           none, none, y, S, Hd, nh, scale, parts);
        return hipGetLastError();
    }
    if (parts) return hipErrorInvalidValue;   // only the fused kernel writes min / max pairs
    // scores = Q_h K_h^T per (batch, head), the scaled softmax, then P V_h,
    // with the heads read and written in place through strides
    const int hd = Hd / nh;
    float* scores = (float*)ws;
    GemmF32Gen p{};
    p.M = S; p.N = S; p.K = hd; p.nb2 = nh; p.alpha = 1.0f;
    p.A = q; p.sam = Hd; p.sak = 1; p.as1 = (long long)S * Hd; p.as2 = hd;
    p.B = k; p.sbk = 1; p.sbn = Hd; p.bs1 = (long long)S * Hd; p.bs2 = hd;
    p.Y = scores; p.ldy = S; p.ys1 = (long long)nh * S * S; p.ys2 = (long long)S * S;
    hipError_t e = launch_gemm_f32_gen(p, (long long)B * nh, s);
    if (e != hipSuccess) return e;
    const long long rows = (long long)B * nh * S;
    hipLaunchKernelGGL(softmax_scaled_f32_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, scores,
                       scores, rows, S, scale);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    GemmF32Gen o{};
    o.M = S; o.N = hd; o.K = S; o.nb2 = nh; o.alpha = 1.0f;
    o.A = scores; o.sam = S; o.sak = 1; o.as1 = (long long)nh * S * S; o.as2 = (long long)S * S;
    o.B = v; o.sbk = Hd; o.sbn = 1; o.bs1 = (long long)S * Hd; o.bs2 = hd;
    o.Y = y; o.ldy = Hd; o.ys1 = (long long)S * Hd; o.ys2 = hd;
    return launch_gemm_f32_gen(o, (long long)B * nh, s);
}

}  // namespace nnrh
