// nnrh_f32.hip -- fp32 glue kernels of the configuration graphs. They keep
// tensors resident in HBM between the int8 operators; none is a performance
// target and their parity bar is the reference's float tolerance (1e-3 abs,
// tensor_equal, src/nnr.cpp:557-563).
//   GlobalAveragePool (src/backend/cpu/global_pool.cpp), NCHW or NHWC input
//   Gemm              (src/backend/cpu/Gemm.cpp), row-major, transA/transB
//   Clip / Relu       (src/backend/cpu/Clip.cpp, Relu.cpp)
#include "nnrh_f32.h"

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

// Y[M][N] = alpha * op(A)[M][K] * op(B)[K][N] + beta * Cb (broadcast)
// 32x32 tile, 16x16 threads, 2x2 outputs per thread, K step 32 through LDS.
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict A,
                                                       const float* __restrict B,
                                                       const float* __restrict Cb,
                                                       float* __restrict Y, int M, int N, int K,
                                                       int transA, int transB, float alpha,
                                                       float beta, int c_mode) {
    __shared__ float As[32][32 + 1];   // [k][m]
    __shared__ float Bs[32][32 + 1];   // [k][n]
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int m0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
    float acc[2][2] = {};
    for (int k0 = 0; k0 < K; k0 += 32) {
        for (int i = threadIdx.x; i < 32 * 32; i += 256) {
            int r = i / 32, c = i % 32;
            // A: walk the contiguous dimension with c
            int am = m0 + (transA ? c : r), ak = k0 + (transA ? r : c);
            float av = (am < M && ak < K) ? (transA ? A[(long long)ak * M + am] : A[(long long)am * K + ak]) : 0.f;
            As[ak - k0][am - m0] = av;
            int bn = n0 + (transB ? r : c), bk = k0 + (transB ? c : r);
            float bv = (bn < N && bk < K) ? (transB ? B[(long long)bn * K + bk] : B[(long long)bk * N + bn]) : 0.f;
            Bs[bk - k0][bn - n0] = bv;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 32; ++kk) {
            float a0 = As[kk][ty * 2], a1 = As[kk][ty * 2 + 1];
            float b0 = Bs[kk][tx * 2], b1 = Bs[kk][tx * 2 + 1];
            acc[0][0] = __builtin_fmaf(a0, b0, acc[0][0]);
            acc[0][1] = __builtin_fmaf(a0, b1, acc[0][1]);
            acc[1][0] = __builtin_fmaf(a1, b0, acc[1][0]);
            acc[1][1] = __builtin_fmaf(a1, b1, acc[1][1]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        int m = m0 + ty * 2 + i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            int n = n0 + tx * 2 + j;
            if (n >= N) continue;
            float v = alpha * acc[i][j];
            if (c_mode == 1) v = v + beta * Cb[0];
            else if (c_mode == 2) v = v + beta * Cb[n];
            else if (c_mode == 3) v = v + beta * Cb[(long long)m * N + n];
            else if (c_mode == 4) v = v + beta * Cb[m];
            Y[(long long)m * N + n] = v;
        }
    }
}

hipError_t launch_gemm_f32(const float* A, const float* B, const float* C, float* Y, int M, int N,
                           int K, int transA, int transB, float alpha, float beta, int c_mode,
                           hipStream_t s) {
    if (M <= 0 || N <= 0) return hipSuccess;
    dim3 grid((N + 31) / 32, (M + 31) / 32);
    hipLaunchKernelGGL(gemm_f32_kernel, grid, dim3(256), 0, s, A, B, C, Y, M, N, K, transA, transB,
                       alpha, beta, c_mode);
    return hipGetLastError();
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

}  // namespace nnrh
