// nnrh_f32.hip -- fp32 glue kernels of the configuration graphs. They keep
// tensors resident in HBM between the int8 operators; none is a performance
// target and their parity bar is the reference's float tolerance (1e-3 abs,
// tensor_equal, src/nnr.cpp:557-563).
//   GlobalAveragePool (src/backend/cpu/global_pool.cpp), NCHW or NHWC input
//   Gemm / MatMul     (src/backend/cpu/Gemm.cpp, MatMul.cpp), row-major, through rocBLAS
//   Clip / Relu       (src/backend/cpu/Clip.cpp, Relu.cpp)
#include "nnrh_f32.h"

#include <rocblas/rocblas.h>

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

// Y[M][N] = alpha * op(A)[M][K] * op(B)[K][N] + beta * Cb (broadcast), row-major.
// A plain fp32 GEMM, so it goes to rocBLAS: the broadcast C is written into Y
// first and rocBLAS accumulates alpha*A*B + beta*Y onto it. Row-major Y is
// column-major Y^T = op(B)^T op(A)^T, which is the call below.
__global__ __launch_bounds__(256) void bcast_c_kernel(const float* __restrict C, float* __restrict Y,
                                                      int M, int N, int c_mode, long long y_bstride) {
    const long long n = (long long)M * N;
    float* y = Y + (long long)blockIdx.y * y_bstride;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256) {
        const long long r = i / N, c = i - r * N;
        float v;
        if (c_mode == 1) v = C[0];
        else if (c_mode == 2) v = C[c];
        else if (c_mode == 3) v = C[i];
        else v = C[r];
        y[i] = v;
    }
}

namespace {
// one rocBLAS handle per (thread, device)
rocblas_handle blas_handle() {
    thread_local rocblas_handle handles[16] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return nullptr;
    if (!handles[dev] && rocblas_create_handle(&handles[dev]) != rocblas_status_success)
        handles[dev] = nullptr;
    return handles[dev];
}
}  // namespace

hipError_t launch_gemm_f32_batched(const float* A, const float* B, const float* C, float* Y, int M,
                                   int N, int K, int transA, int transB, float alpha, float beta,
                                   int c_mode, int batch, long long a_bstride, long long b_bstride,
                                   long long y_bstride, hipStream_t s) {
    if (M <= 0 || N <= 0 || batch <= 0) return hipSuccess;
    rocblas_handle h = blas_handle();
    if (!h || rocblas_set_stream(h, s) != rocblas_status_success) return hipErrorNotInitialized;
    float beta_eff = 0.0f;
    if (c_mode != 0 && beta != 0.0f) {
        long long n = (long long)M * N;
        long long blocks = (n + 255) / 256;
        if (blocks > 4096) blocks = 4096;
        hipLaunchKernelGGL(bcast_c_kernel, dim3((unsigned)blocks, batch), dim3(256), 0, s, C, Y, M, N,
                           c_mode, y_bstride);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        beta_eff = beta;
    }
    const rocblas_operation opB = transB ? rocblas_operation_transpose : rocblas_operation_none;
    const rocblas_operation opA = transA ? rocblas_operation_transpose : rocblas_operation_none;
    const int ldb = transB ? K : N;
    const int lda = transA ? M : K;
    rocblas_status st;
    if (batch == 1)
        st = rocblas_sgemm(h, opB, opA, N, M, K, &alpha, B, ldb, A, lda, &beta_eff, Y, N);
    else
        st = rocblas_sgemm_strided_batched(h, opB, opA, N, M, K, &alpha, B, ldb, b_bstride, A, lda,
                                           a_bstride, &beta_eff, Y, N, y_bstride, batch);
    return st == rocblas_status_success ? hipSuccess : hipErrorLaunchFailure;
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

}  // namespace nnrh
