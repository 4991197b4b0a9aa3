// nnrh_f32.hip -- fp32 glue kernels of the configuration graphs. They keep
// tensors resident in HBM between the int8 operators; none is a performance
// target and their parity bar is the reference's float tolerance (1e-3 abs,
// tensor_equal, src/nnr.cpp:557-563).
//   GlobalAveragePool (src/backend/cpu/global_pool.cpp), NCHW or NHWC input
//   Gemm / MatMul     (src/backend/cpu/Gemm.cpp, MatMul.cpp), row-major, through rocBLAS
//   Clip / Relu       (src/backend/cpu/Clip.cpp, Relu.cpp)
//   Add / Mul / Sub / Div with scalar or last-axis broadcast (binary_math.cpp)
//   Softmax, LayerNormalization over the last axis, Gelu (erf form), Transpose
//   (the BERT encoder's fp32 glue: Softmax.cpp, LayerNormalization.cpp,
//   Gelu.cpp, Transpose.cpp)
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

hipError_t launch_gap_dq(const uint8_t* x, float* y, int N, int C, int HW, int x_nhwc, int x_signed,
                         float scale, int zp, hipStream_t s) {
    const long long rows = (long long)N * C;
    if (rows <= 0) return hipSuccess;
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

// LayerNormalization over rows of D (one wave per row), two passes over the
// row: mean, then the mean of squared deviations
__global__ __launch_bounds__(256) void layernorm_f32_kernel(const float* __restrict x,
                                                            const float* __restrict gamma,
                                                            const float* __restrict beta,
                                                            float* __restrict y, long long rows, int D,
                                                            float eps) {
    const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* xr = x + row * D;
    float* yr = y + row * D;
    float sum = 0.0f;
    for (int i = lane; i < D; i += 64) sum += xr[i];
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    const float mean = sum / (float)D;
    float sq = 0.0f;
    for (int i = lane; i < D; i += 64) {
        const float d = xr[i] - mean;
        sq += d * d;
    }
    for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off, 64);
    const float inv = 1.0f / sqrtf(sq / (float)D + eps);
    for (int i = lane; i < D; i += 64) {
        const float v = (xr[i] - mean) * inv * gamma[i];
        yr[i] = beta ? v + beta[i] : v;
    }
}

hipError_t launch_layernorm_f32(const float* x, const float* gamma, const float* beta, float* y,
                                long long rows, int D, float eps, hipStream_t s) {
    if (rows <= 0 || D <= 0) return hipSuccess;
    hipLaunchKernelGGL(layernorm_f32_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, x, gamma,
                       beta, y, rows, D, eps);
    return hipGetLastError();
}

// Gelu, erf form: 0.5 x (1 + erf(x / sqrt(2)))
__global__ __launch_bounds__(256) void gelu_f32_kernel(const float* __restrict x, float* __restrict y,
                                                       long long n) {
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (long long)gridDim.x * 256) {
        const float v = x[i];
        y[i] = 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
    }
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
// written straight into the output's head columns. Two pointer-array batched
// GEMMs; no transposes are materialized.
__global__ __launch_bounds__(256) void mha_ptrs_kernel(const float* q, const float* k, const float* v, float* y,
                                                       float* scores, const float** A1, const float** B1,
                                                       float** C1, const float** A2, const float** B2,
                                                       float** C2, int B, int S, int Hd, int nh) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= B * nh) return;
    const int b = i / nh, h = i - b * nh, hd = Hd / nh;
    const long long off = (long long)b * S * Hd + (long long)h * hd;
    float* sc = scores + (long long)i * S * S;
    A1[i] = k + off; B1[i] = q + off; C1[i] = sc;
    A2[i] = v + off; B2[i] = sc; C2[i] = y + off;
}

size_t mha_workspace_bytes(int B, int S, int nh) {
    const size_t nptr = (size_t)B * nh;
    return ((6 * nptr * sizeof(void*) + 255) & ~(size_t)255) + sizeof(float) * nptr * S * S;
}

hipError_t launch_mha_f32(const float* q, const float* k, const float* v, float* y, int B, int S, int Hd, int nh,
                          float scale, void* ws, hipStream_t s) {
    if (B <= 0 || S <= 0) return hipSuccess;
    if (nh <= 0 || Hd % nh) return hipErrorInvalidValue;
    const int hd = Hd / nh, nb = B * nh;
    const float** A1 = (const float**)ws;
    const float** B1 = A1 + nb;
    float** C1 = (float**)(B1 + nb);
    const float** A2 = (const float**)(C1 + nb);
    const float** B2 = A2 + nb;
    float** C2 = (float**)(B2 + nb);
    float* scores = (float*)((char*)ws + ((6 * (size_t)nb * sizeof(void*) + 255) & ~(size_t)255));
    hipLaunchKernelGGL(mha_ptrs_kernel, dim3((nb + 255) / 256), dim3(256), 0, s, q, k, v, y, scores, A1, B1, C1,
                       A2, B2, C2, B, S, Hd, nh);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    rocblas_handle h = blas_handle();
    if (!h || rocblas_set_stream(h, s) != rocblas_status_success) return hipErrorNotInitialized;
    const float one = 1.0f, zero = 0.0f;
    // column-major: scores^T[S x S] = K_h^T-as-stored... i.e. (K rows) . (Q rows)^T:
    // C1 (ld S) = op(A1 = K, D x S col-major, ld Hd)^T * (B1 = Q, D x S, ld Hd)
    rocblas_status st = rocblas_sgemm_batched(h, rocblas_operation_transpose, rocblas_operation_none, S, S, hd,
                                              &one, A1, Hd, B1, Hd, &zero, C1, S, nb);
    if (st != rocblas_status_success) return hipErrorLaunchFailure;
    const long long rows = (long long)nb * S;
    hipLaunchKernelGGL(softmax_scaled_f32_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, scores,
                       scores, rows, S, scale);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    // ctx^T (hd x S, ld Hd) = V^T-as-stored (hd x S, ld Hd) * P^T-as-stored (S x S, ld S)
    st = rocblas_sgemm_batched(h, rocblas_operation_none, rocblas_operation_none, hd, S, S, &one, A2, Hd, B2, S,
                               &zero, C2, Hd, nb);
    return st == rocblas_status_success ? hipSuccess : hipErrorLaunchFailure;
}

}  // namespace nnrh
