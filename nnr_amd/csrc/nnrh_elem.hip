// nnrh_elem.hip -- memory-bound kernels of the int8 path:
//   QuantizeLinear        (src/backend/cpu/QuantizeLinear.cpp:128-194)
//   DequantizeLinear      (src/backend/cpu/DequantizeLinear.cpp:100-152)
//   DynamicQuantizeLinear (src/backend/cpu/DynamicQuantizeLinear.cpp:27-58)
//   QLinearAdd            (src/backend/cpu/QLinearAdd.cpp:33-265)
//   MaxPool uint8 NHWC    (src/backend/x64/pool_x64.h:396-436)
// Each kernel reproduces the reference's per-element formula, including which
// elements take the 16-wide SIMD body and which the scalar tail.
#include "nnrh_elem.h"
#include "nnrh_rq.h"

#include <atomic>
#include <mutex>

namespace nnrh {

__device__ __forceinline__ void st_q(void* y, int dt, long long i, int v) {
    if (dt == 0) ((uint8_t*)y)[i] = (uint8_t)v;
    else ((int8_t*)y)[i] = (int8_t)v;
}
__device__ __forceinline__ int ld_q(const void* p, int dt, long long i) {
    return dt == 0 ? (int)((const uint8_t*)p)[i] : (int)((const int8_t*)p)[i];
}

// ---------------------------------------------------------------------------
// QuantizeLinear, per-tensor. n >= 64: body multiplies by fl(1/s) on 16-wide
// chunks of 4096-element blocks, the last n%16 elements divide (4096 is a
// multiple of 16, so only the final partial chunk is a tail). n < 64: divide.
__global__ __launch_bounds__(256) void quantize_kernel(const float* __restrict x, long long n,
                                                       float scale, float inv, int zp, int dt,
                                                       int lo, int hi, void* __restrict y) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long stride = (long long)gridDim.x * blockDim.x;
    const long long body = n >= 64 ? n - n % 16 : 0;
    for (; i < n; i += stride) {
        float xv = x[i];
        int q;
        if (i < body) {
            float v = xv * inv;
            v = __builtin_rintf(v) + (float)zp;
            v = clamp_minmax(v, (float)lo, (float)hi);
            q = (int)v;
        } else {
            q = clampi(wrap_add(x86_f2i(__builtin_rintf(xv / scale)), zp), lo, hi);
        }
        st_q(y, dt, i, q);
    }
}

hipError_t launch_quantize(const float* x, long long n, float scale, int zp, int dt, void* y,
                           hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int lo = dt == 0 ? 0 : -128, hi = dt == 0 ? 255 : 127;
    float inv = 1.0f / scale;
    long long blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(quantize_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, n, scale, inv,
                       zp, dt, lo, hi, y);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// DequantizeLinear: y = fl((float(q) - float(zp)) * s); dt 0 u8, 1 s8, 2 i32.
__global__ __launch_bounds__(256) void dequantize_kernel(const void* __restrict x, long long n,
                                                         int dt, float scale, int zp,
                                                         float* __restrict y) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (; i < n; i += stride) {
        int q = dt == 2 ? ((const int32_t*)x)[i] : ld_q(x, dt, i);
        float d = (float)q - (float)zp;
        y[i] = d * scale;
    }
}

hipError_t launch_dequantize(const void* x, long long n, int dt, float scale, int zp, float* y,
                             hipStream_t s) {
    if (n <= 0) return hipSuccess;
    long long blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(dequantize_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, n, dt,
                       scale, zp, y);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// DynamicQuantizeLinear: min/max partials -> scale/zp -> quantize (divide).
// min/max are exact, so the result does not depend on the reduction order.
constexpr int DQL_BLOCKS = 1024;

__global__ __launch_bounds__(256) void minmax_partial_kernel(const float* __restrict x,
                                                             long long n, float* __restrict part) {
    __shared__ float smn[256], smx[256];
    float mn = 0.0f, mx = 0.0f;
    // 16-byte loads over the aligned body, scalar over the rest
    const long long n4 = (((uintptr_t)x & 15) == 0) ? n >> 2 : 0;
    const float4* x4 = (const float4*)x;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n4; i += (long long)gridDim.x * 256) {
        const float4 v = x4[i];
        mn = fminf(mn, fminf(fminf(v.x, v.y), fminf(v.z, v.w)));
        mx = fmaxf(mx, fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)));
    }
    for (long long i = 4 * n4 + (long long)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (long long)gridDim.x * 256) {
        float v = x[i];
        mn = v < mn ? v : mn;
        mx = mx < v ? v : mx;
    }
    smn[threadIdx.x] = mn;
    smx[threadIdx.x] = mx;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
        if ((int)threadIdx.x < off) {
            float a = smn[threadIdx.x + off], b = smx[threadIdx.x + off];
            smn[threadIdx.x] = a < smn[threadIdx.x] ? a : smn[threadIdx.x];
            smx[threadIdx.x] = smx[threadIdx.x] < b ? b : smx[threadIdx.x];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        part[2 * blockIdx.x] = smn[0];
        part[2 * blockIdx.x + 1] = smx[0];
    }
}

// scale and zero point from the min/max partials (DynamicQuantizeLinear.cpp:
// 37-48): xmin = min(0, min x), xmax = max(0, max x), s = fl((xmax - xmin) /
// 255) (1 when 0), zp = clamp(nearbyint(fl(-xmin / s)), 0, 255). Every
// quantize block reduces the partials itself (they are exact, so every
// block gets the same values); block 0 also stores them.
__device__ __forceinline__ void dyn_scale_block(const float* __restrict part, int nparts, float* sc_out,
                                                int* zp_out) {
    __shared__ float smn[256], smx[256];
    float mn = 0.0f, mx = 0.0f;
#pragma unroll 4
    for (int i = threadIdx.x; i < nparts; i += 256) {
        float a = part[2 * i], b = part[2 * i + 1];
        mn = a < mn ? a : mn;
        mx = mx < b ? b : mx;
    }
    smn[threadIdx.x] = mn;
    smx[threadIdx.x] = mx;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
        if ((int)threadIdx.x < off) {
            float a = smn[threadIdx.x + off], b = smx[threadIdx.x + off];
            smn[threadIdx.x] = a < smn[threadIdx.x] ? a : smn[threadIdx.x];
            smx[threadIdx.x] = smx[threadIdx.x] < b ? b : smx[threadIdx.x];
        }
        __syncthreads();
    }
    const float xmin = smn[0] < 0.0f ? smn[0] : 0.0f;
    const float xmax = smx[0] > 0.0f ? smx[0] : 0.0f;
    float sc = (xmax - xmin) / 255.0f;
    if (sc == 0.0f) sc = 1.0f;
    *sc_out = sc;
    *zp_out = clampi(x86_f2i(__builtin_rintf(-xmin / sc)), 0, 255);
}

__device__ __forceinline__ uint32_t dyn_q1(float v, float sc, int zp) {
    return (uint32_t)clampi(wrap_add(x86_f2i(__builtin_rintf(v / sc)), zp), 0, 255);
}
// dyn_q1's value, as a float for v_cvt_pk_u8_f32 (which saturates to
// [0, 255]), without a division per element. q = fl(v * r) with
// r = fl(1 / sc) differs from v / sc by at most |v / sc| * (2^-23 + 2^-48),
// and the quotient fl(v / sc) by at most half an ulp, 2^-17 below 256: so
// for |q| < 256, |q - fl(v / sc)| < 2^-14, and where q lies more than 2^-13
// from every half-integer both round to the same integer k = rne(q), and
// k + zp (exact) is the byte before the clamp. Elements near a half-integer
// (about one in 2^11), |q| >= 256, NaN and infinities take the division.
__device__ __forceinline__ float dyn_qf(float v, float r, float sc, int zp) {
    const float q = v * r;
    const float k = __builtin_rintf(q);
    const float d = __builtin_fabsf(q - k);   // exact: q and k are within a factor 2 (or k = 0)
    if (__builtin_expect(!(__builtin_fabsf(q) < 256.0f && __builtin_fabsf(d - 0.5f) > 0x1p-13f), 0))
        return (float)dyn_q1(v, sc, zp);
    return k + (float)zp;
}
// scale and zero point from producer-written (min, max) pairs, reduced by
// every block of the quantize kernel (NT threads): every block gets the
// same values, since min and max are exact in any order
template <int NT = 256>
__device__ __forceinline__ void dyn_scale_parts_block(const float* __restrict part, int nparts, float* sc_out,
                                                      int* zp_out) {
    __shared__ float smn[NT / 64], smx[NT / 64];
    float mn = 0.0f, mx = 0.0f;
    const int n2 = nparts >> 1;   // whole float4s (the pairs are 8-byte aligned)
    const bool vec = ((uintptr_t)part & 15) == 0;
    if (vec) {
        const float4* p4 = (const float4*)part;
#pragma unroll 4
        for (int i = threadIdx.x; i < n2; i += NT) {
            const float4 v = p4[i];
            mn = fminf(mn, fminf(v.x, v.z));
            mx = fmaxf(mx, fmaxf(v.y, v.w));
        }
    }
    for (int i = (vec ? 2 * n2 : 0) + threadIdx.x; i < nparts; i += NT) {
        mn = fminf(mn, part[2 * i]);
        mx = fmaxf(mx, part[2 * i + 1]);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        mn = fminf(mn, __shfl_xor(mn, off, 64));
        mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        smn[w] = mn;
        smx[w] = mx;
    }
    __syncthreads();
    mn = smn[0];
    mx = smx[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) {
        mn = fminf(mn, smn[i]);
        mx = fmaxf(mx, smx[i]);
    }
    const float xmin = mn < 0.0f ? mn : 0.0f;
    const float xmax = mx > 0.0f ? mx : 0.0f;
    float sc = (xmax - xmin) / 255.0f;
    if (sc == 0.0f) sc = 1.0f;
    *sc_out = sc;
    *zp_out = clampi(x86_f2i(__builtin_rintf(-xmin / sc)), 0, 255);
}

// y = clamp(nearbyint(fl(x / s)) + zp, 0, 255): 16 elements per thread over the
// 16-byte aligned body (one 16-byte store), scalar over the rest. PARTS: part
// holds nparts producer-written (min, max) pairs, reduced by every block;
// else the minmax_partial_kernel's pairs (dyn_scale_block)
template <bool PARTS>
__global__ __launch_bounds__(256) void dyn_quantize_kernel(const float* __restrict x, long long n,
                                                           const float* __restrict part, int nparts,
                                                           float* __restrict y_scale,
                                                           uint8_t* __restrict y_zp,
                                                           uint8_t* __restrict y) {
    float sc;
    int zp;
    if (PARTS) dyn_scale_parts_block(part, nparts, &sc, &zp);
    else dyn_scale_block(part, nparts, &sc, &zp);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        *y_scale = sc;
        *y_zp = (uint8_t)zp;
    }
    const bool vec = (((uintptr_t)x | (uintptr_t)y) & 15) == 0;
    const long long n16 = vec ? n >> 4 : 0;
    const float4* x4 = (const float4*)x;
    const float r = 1.0f / sc;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n16; i += (long long)gridDim.x * 256) {
        float4 v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = x4[4 * i + q];
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t t = __builtin_amdgcn_cvt_pk_u8_f32(dyn_qf(v[q].x, r, sc, zp), 0, 0u);
            t = __builtin_amdgcn_cvt_pk_u8_f32(dyn_qf(v[q].y, r, sc, zp), 1, t);
            t = __builtin_amdgcn_cvt_pk_u8_f32(dyn_qf(v[q].z, r, sc, zp), 2, t);
            w[q] = __builtin_amdgcn_cvt_pk_u8_f32(dyn_qf(v[q].w, r, sc, zp), 3, t);
        }
        *(uint4*)(y + 16 * i) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    for (long long i = 16 * n16 + (long long)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (long long)gridDim.x * 256)
        y[i] = (uint8_t)dyn_q1(x[i], sc, zp);
}

size_t dynamic_quantize_workspace() { return sizeof(float) * 2 * DQL_BLOCKS; }

hipError_t launch_dynamic_quantize(const float* x, long long n, uint8_t* y, float* y_scale,
                                   uint8_t* y_zp, void* workspace, hipStream_t s) {
    float* part = (float*)workspace;
    long long nb = (n + 255) / 256;
    int blocks = (int)(nb < DQL_BLOCKS ? (nb > 0 ? nb : 1) : DQL_BLOCKS);
    hipLaunchKernelGGL(minmax_partial_kernel, dim3(blocks), dim3(256), 0, s, x, n, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    long long qb = (n / 16 + 255) / 256;
    if (qb < 1) qb = 1;
    if (qb > 2048) qb = 2048;
    hipLaunchKernelGGL(dyn_quantize_kernel<false>, dim3((unsigned)qb), dim3(256), 0, s, x, n, part, blocks,
                       y_scale, y_zp, y);
    return hipGetLastError();
}

// DynamicQuantizeLinear with its min / max partials in a file-scope device
// array instead of a caller's workspace, for callers that cannot allocate.
// Every GPU the library runs on holds its own copy (8 KiB) until the process
// ends; calls on one GPU share it, so calls that overlap on one GPU race.
// Nothing in it needs clearing: the partial kernel writes every pair the
// quantize kernel then reads.
constexpr int DQL_SCRATCH_FLOATS = 2 * DQL_BLOCKS;
static __device__ __align__(256) float scratch[DQL_SCRATCH_FLOATS];

constexpr int DQL_MAX_DEVICES = 64;
static std::atomic<float*> g_scratch_dev[DQL_MAX_DEVICES];
static std::mutex g_scratch_mu;

// Device address of this GPU's copy of `scratch`, looked up once per device
// with that device current. The array's name is only a host-side stand-in:
// kernels get this address, never the name.
static hipError_t dynq_scratch(float** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= DQL_MAX_DEVICES) return hipErrorInvalidDevice;
    float* p = g_scratch_dev[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        p = g_scratch_dev[dev].load(std::memory_order_relaxed);
        if (!p) {
            void* sym = nullptr;
            e = hipGetSymbolAddress(&sym, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return e;
            if (!sym) return hipErrorInvalidSymbol;
            p = (float*)sym;
            g_scratch_dev[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return hipSuccess;
}

hipError_t launch_dynamic_quantize_noalloc(const float* x, long long n, uint8_t* y, float* y_scale,
                                           uint8_t* y_zp, hipStream_t s) {
    static_assert(sizeof(scratch) >= sizeof(float) * 2 * DQL_BLOCKS, "scratch holds every partial");
    float* part = nullptr;
    hipError_t e = dynq_scratch(&part);
    if (e != hipSuccess) return e;
    return launch_dynamic_quantize(x, n, y, y_scale, y_zp, part, s);
}

hipError_t launch_dynamic_quantize_parts(const float* x, long long n, const float* parts, int nparts,
                                         uint8_t* y, float* y_scale, uint8_t* y_zp, hipStream_t s) {
    // one launch: every block reduces the pairs (nparts * 8 bytes from L2)
    // and quantizes its share; a grid of at most 512 blocks keeps the
    // repeated reads of the pairs small against the tensor
    long long qb = (n / 16 + 255) / 256;
    if (qb < 1) qb = 1;
    if (qb > 512) qb = 512;
    hipLaunchKernelGGL(dyn_quantize_kernel<true>, dim3((unsigned)qb), dim3(256), 0, s, x, n, parts, nparts,
                       y_scale, y_zp, y);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// DynamicQuantizeLinear after a fused QLinearMatMul -> DequantizeLinear ->
// Add(bias) [-> Gelu] chain whose GEMM stored the uint8 QLinearMatMul bytes
// instead of the fp32 chain values, with the (min, max) pairs of those values.
// The fp32 value of byte q in column n depends on (n, q) alone,
//   f(n, q) = [Gelu] (fl(fl((q - q_zp) * dq_scale) + bias[n])),
// the GEMM epilogue's expression operation for operation, so its quantized
// byte does too. The table kernel reduces the pairs to the scale / zero point
// (DynamicQuantizeLinear.cpp:37-48) and builds T[q][n] = quantize(f(n, q)) for
// every column and byte; the gather kernel maps every stored byte through its
// column's table. The bytes equal quantizing the fp32 tensor (each element
// gets the same value and the same scale / zero point).
constexpr int DQC_SLICE = 256;     // gather: columns a block (table slice 256 x 256 bytes of LDS)
constexpr int DQC_THREADS = 512;   // gather: 8 waves a block
constexpr int DQC_RPT = 32;        // gather: rows a thread at most (a block: 8 x 32 rows)
constexpr int DQC_RESIDENT = 512;  // gather blocks resident at once (2 a CU: 64 KiB of LDS each)

// grid (Np / 64, 4), 1024 threads: columns 64 bx .. + 63, bytes 64 by .. + 63
__global__ __launch_bounds__(1024) void dynq_codes_table_kernel(const float* __restrict part, int nparts,
                                                               const float* __restrict bias, float dq_scale,
                                                               int q_zp, int gelu, int Np,
                                                               uint8_t* __restrict table,
                                                               float* __restrict y_scale,
                                                               uint8_t* __restrict y_zp) {
    float sc;
    int zp;
    dyn_scale_parts_block<1024>(part, nparts, &sc, &zp);
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
        *y_scale = sc;
        *y_zp = (uint8_t)zp;
    }
    const float r = 1.0f / sc;
    const int n = blockIdx.x * 64 + (threadIdx.x & 63);
    const float b = bias[n];
    const float zp_f = (float)q_zp;
    const int q_end = blockIdx.y * 64 + 64;
#pragma unroll
    for (int q = blockIdx.y * 64 + (threadIdx.x >> 6); q < q_end; q += 16) {
        const float d = ((float)q - zp_f) * dq_scale;
        float v = d + b;
        if (gelu) v = gelu_erf(v);
        table[(long long)q * Np + n] = (uint8_t)__builtin_amdgcn_cvt_pk_u8_f32(dyn_qf(v, r, sc, zp), 0, 0u);
    }
}

// 4 bytes of one row through the table slice (tl: the slice at the first of
// the 4 columns; byte value q of column j sits at tl[q * DQC_SLICE + j]).
// With a lane's 4 columns at 4 lane, the 64 lanes of a wave read 64
// different dwords of each table row: no two lanes share a bank
__device__ __forceinline__ uint32_t codes_lut4(const uint8_t* tl, uint32_t x) {
    const uint32_t b0 = tl[(x & 0xffu) * DQC_SLICE];
    const uint32_t b1 = tl[((x >> 8) & 0xffu) * DQC_SLICE + 1];
    const uint32_t b2 = tl[((x >> 16) & 0xffu) * DQC_SLICE + 2];
    const uint32_t b3 = tl[(x >> 24) * DQC_SLICE + 3];
    return b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
}

// grid (ceil(Np / 256), ceil(rows / R)), R <= 8 x 32 rows a block (a
// multiple of 8, chosen so that the grid fits the resident blocks): lane l of
// every wave holds columns 4 l .. 4 l + 3 of the block's slice, so each load
// or store instruction of a wave covers 256 contiguous bytes of one row; wave
// w holds rows w, w + 8, ... The block's table slice (a full one: 8 16-byte
// chunks a thread) and all of a thread's rows are loaded with no wait in
// between; the slice goes to LDS as its loads land.
__global__ __launch_bounds__(DQC_THREADS) void dynq_codes_gather_kernel(const uint8_t* __restrict codes,
                                                                        long long rows, int N, int Np, int R,
                                                                        const uint8_t* __restrict table,
                                                                        uint8_t* __restrict y) {
    __shared__ __attribute__((aligned(16))) uint8_t t[256 * DQC_SLICE];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c0 = blockIdx.x * DQC_SLICE;
    const int cl = 4 * lane;   // this thread's first column in the slice
    const int c = c0 + cl;
    const long long rw = (long long)blockIdx.y * R + wave;   // this wave's first row
    const long long re = min(rows, (long long)(blockIdx.y + 1) * R);
    // dword loads and stores: N % 4 == 0 and 4-byte aligned buffers (then a
    // lane with c < N has all 4 columns)
    const bool vec = (N & 3) == 0 && ((((uintptr_t)codes) | (uintptr_t)y) & 3) == 0;
    const int w = min(DQC_SLICE, Np - c0);   // a multiple of 64
    // the table slice, 16-byte chunk i = row i / 16, columns 16 (i % 16) ..;
    // in a partial slice the chunks past w load the last one and land in
    // LDS columns no lane reads
    constexpr int TCH = 256 * DQC_SLICE / 16 / DQC_THREADS;   // chunks a thread
    uint4 tv[TCH];
#pragma unroll
    for (int k = 0; k < TCH; ++k) {
        const int i = threadIdx.x + k * DQC_THREADS;
        tv[k] = *(const uint4*)(table + (long long)(i >> 4) * Np + c0 + min(16 * (i & 15), w - 16));
    }
    uint32_t x[DQC_RPT];
    if (vec) {
        // rows past the block's end load its last row, lanes past N the
        // last 4 columns; neither is stored
        const int cc = min(c, N - 4);
#pragma unroll
        for (int i = 0; i < DQC_RPT; ++i) {
            const long long r = min(rw + 8 * i, re - 1);
            x[i] = *(const uint32_t*)(codes + r * N + cc);
        }
    }
#pragma unroll
    for (int k = 0; k < TCH; ++k) {
        const int i = threadIdx.x + k * DQC_THREADS;
        *(uint4*)(t + (i >> 4) * DQC_SLICE + 16 * (i & 15)) = tv[k];
    }
    __syncthreads();
    if (c >= N) return;   // (no barrier below)
    const uint8_t* tl = t + cl;
    if (vec) {
        // (a row past the block's end stores the last row's bytes again)
#pragma unroll
        for (int i = 0; i < DQC_RPT; ++i) {
            const long long r = min(rw + 8 * i, re - 1);
            *(uint32_t*)(y + r * N + c) = codes_lut4(tl, x[i]);
        }
        return;
    }
    const int nc = min(4, N - c);
    for (long long r = rw; r < re; r += 8)
        for (int j = 0; j < nc; ++j) y[r * N + c + j] = tl[codes[r * N + c + j] * DQC_SLICE + j];
}

size_t dynamic_quantize_codes_table_bytes(int Np) { return (size_t)256 * (size_t)Np; }

hipError_t launch_dynamic_quantize_codes(const uint8_t* codes, long long rows, int N, int Np, const float* bias,
                                         float dq_scale, int q_zp, int gelu, const float* parts, int nparts,
                                         uint8_t* table, uint8_t* y, float* y_scale, uint8_t* y_zp,
                                         hipStream_t s) {
    hipLaunchKernelGGL(dynq_codes_table_kernel, dim3((unsigned)(Np / 64), 4), dim3(1024), 0, s, parts, nparts,
                       bias, dq_scale, q_zp, gelu, Np, table, y_scale, y_zp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || rows == 0) return e;
    // rows a block: the fewest (a multiple of 8, at most 256) that keep the
    // grid within the resident blocks, else 256
    const long long slices = (Np + DQC_SLICE - 1) / DQC_SLICE;
    const long long per = (rows * slices + DQC_RESIDENT - 1) / DQC_RESIDENT;
    long long R = (per + 7) / 8 * 8;
    R = R < 8 ? 8 : R > 8 * DQC_RPT ? 8 * DQC_RPT : R;
    while (R < 8 * DQC_RPT && ((rows + R - 1) / R) * slices > DQC_RESIDENT) R += 8;
    hipLaunchKernelGGL(dynq_codes_gather_kernel, dim3((unsigned)slices, (unsigned)((rows + R - 1) / R)),
                       dim3(DQC_THREADS), 0, s, codes, rows, N, Np, (int)R, table, y);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// QLinearAdd. kind: 0 same shape, 1 B scalar, 2 A scalar, 3 per-channel B[C].
__global__ __launch_bounds__(256) void qadd_kernel(QAddArgs p) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (; i < p.n; i += stride) {
        int q;
        if (p.kind == 0) {
            const long long body = p.tail_all ? 0 : p.n - p.n % 16;
            int a = ld_q(p.a, p.dt, i), b = ld_q(p.b, p.dt, i);
            if (i < body) {
                // v = fma(fa, sa, fma(fb, sb, fixed)); cvtps2dq; saturating pack
                float v = __builtin_fmaf((float)b, p.sb, p.fixed);
                v = __builtin_fmaf((float)a, p.sa, v);
                q = clampi(x86_f2i(__builtin_rintf(v)), p.lo, p.hi);
            } else {
                float t1 = p.sa * (float)(a - p.a_zp);
                float t2 = p.sb * (float)(b - p.b_zp);
                float v = (t1 + t2) + (float)p.y_zp;
                q = clampi(x86_f2i(__builtin_rintf(v)), p.lo, p.hi);
            }
        } else if (p.kind == 1 || p.kind == 2) {
            // scalar loops (QLinearAdd.cpp:108-119); the scalar operand's
            // term c = s * (q - zp) is formed from the device byte, as the
            // reference forms it from the host one
            float v;
            if (p.kind == 1) {
                const float cval = p.sb * (float)(ld_q(p.b, p.dt, 0) - p.b_zp);
                float t = p.sa * (float)(ld_q(p.a, p.dt, i) - p.a_zp);
                v = (t + cval) + (float)p.y_zp;
            } else {
                const float cval = p.sa * (float)(ld_q(p.a, p.dt, 0) - p.a_zp);
                float t = p.sb * (float)(ld_q(p.b, p.dt, i) - p.b_zp);
                v = (cval + t) + (float)p.y_zp;
            }
            q = clampi(x86_f2i(__builtin_rintf(v)), p.lo, p.hi);
        } else {
            // per-channel: a full, b[C] (QLinearAdd.cpp:120-226)
            int c;
            long long inner;
            if (p.y_nhwc) { c = (int)(i % p.C); inner = c; }
            else { c = (int)((i / p.HW) % p.C); inner = i % p.HW; }
            const long long body = p.y_nhwc ? (p.C - p.C % 16) : (p.HW - p.HW % 16);
            int a = ld_q(p.a, p.dt, i);
            int bc = ld_q(p.b, p.dt, c) - p.b_zp;
            if (p.y_nhwc) {
                float t0 = p.sb * (float)bc;
                float off = t0 + (float)p.y_zp;     // ch_off[c]
                if (inner < body) {
                    float v = __builtin_fmaf((float)a - (float)p.a_zp, p.sa, off);
                    v = clamp_minmax(__builtin_rintf(v), (float)p.lo, (float)p.hi);
                    q = (int)v;
                } else {
                    float t = p.sa * (float)(a - p.a_zp);
                    q = clampi(x86_f2i(__builtin_rintf(t + off)), p.lo, p.hi);
                }
            } else {
                float chv = p.sb * (float)bc;
                if (inner < body) {
                    float voff = chv + (float)p.y_zp;
                    float v = __builtin_fmaf((float)a - (float)p.a_zp, p.sa, voff);
                    v = clamp_minmax(__builtin_rintf(v), (float)p.lo, (float)p.hi);
                    q = (int)v;
                } else {
                    float t = p.sa * (float)(a - p.a_zp);
                    float v = (t + chv) + (float)p.y_zp;
                    q = clampi(x86_f2i(__builtin_rintf(v)), p.lo, p.hi);
                }
            }
        }
        st_q(p.y, p.dt, i, q);
    }
}

// Same-shape fast path: 16 elements per thread with 16-byte loads/stores.
// Chunks never straddle the body/tail boundary (body = n - n%16).
__global__ __launch_bounds__(256) void qadd_same16_kernel(QAddArgs p) {
    const long long nchunk = p.n >> 4;
    for (long long c = (long long)blockIdx.x * blockDim.x + threadIdx.x; c < nchunk;
         c += (long long)gridDim.x * blockDim.x) {
        uint4 av = ((const uint4*)p.a)[c];
        uint4 bv = ((const uint4*)p.b)[c];
        uint32_t aw[4] = {av.x, av.y, av.z, av.w}, bw[4] = {bv.x, bv.y, bv.z, bv.w}, yw[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t w = 0;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                int a = (int)((aw[q] >> (8 * r)) & 0xff), b = (int)((bw[q] >> (8 * r)) & 0xff);
                if (p.dt) { a = (int)(int8_t)a; b = (int)(int8_t)b; }
                float v = __builtin_fmaf((float)b, p.sb, p.fixed);
                v = __builtin_fmaf((float)a, p.sa, v);
                int qv = clampi(x86_f2i(__builtin_rintf(v)), p.lo, p.hi);
                w |= (uint32_t)(qv & 0xff) << (8 * r);
            }
            yw[q] = w;
        }
        ((uint4*)p.y)[c] = make_uint4(yw[0], yw[1], yw[2], yw[3]);
    }
}

hipError_t launch_qadd(const QAddArgs& p, hipStream_t s) {
    if (p.n <= 0) return hipSuccess;
    const bool vec = p.kind == 0 && (((uintptr_t)p.a | (uintptr_t)p.b | (uintptr_t)p.y) & 15) == 0;
    if (vec && p.n >= 16) {
        long long chunks = p.n >> 4;
        long long blocks = (chunks + 255) / 256;
        if (blocks > 8192) blocks = 8192;
        hipLaunchKernelGGL(qadd_same16_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess || p.n % 16 == 0) return e;
        // the scalar tail: reuse the generic kernel on the last n%16 elements
        QAddArgs t = p;
        const long long off = p.n - p.n % 16;
        t.a = (const uint8_t*)p.a + off;
        t.b = (const uint8_t*)p.b + off;
        t.y = (uint8_t*)p.y + off;
        t.n = p.n % 16;
        t.tail_all = 1;
        hipLaunchKernelGGL(qadd_kernel, dim3(1), dim3(64), 0, s, t);
        return hipGetLastError();
    }
    long long blocks = (p.n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(qadd_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// MaxPool uint8 NHWC: max over the in-image window, starting from 0.
__global__ __launch_bounds__(256) void maxpool_u8_kernel(const uint8_t* __restrict x,
                                                         uint8_t* __restrict y, int N, int C,
                                                         int iH, int iW, int oH, int oW, int kH,
                                                         int kW, int sH, int sW, int pH,
                                                         int pW) {
    const int C4 = (C + 3) >> 2;
    long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long total = (long long)N * oH * oW * C4;
    if (idx >= total) return;
    const int cg = (int)(idx % C4);
    const long long pix = idx / C4;
    const int ow = (int)(pix % oW), oh = (int)((pix / oW) % oH), n = (int)(pix / ((long long)oW * oH));
    const int c0 = cg * 4;
    const int ih0 = oh * sH - pH, iw0 = ow * sW - pW;
    const int kh0 = ih0 < 0 ? -ih0 : 0, kh1 = kH < iH - ih0 ? kH : iH - ih0;
    const int kw0 = iw0 < 0 ? -iw0 : 0, kw1 = kW < iW - iw0 ? kW : iW - iw0;
    const bool vec_ok = (C & 3) == 0;
    uint32_t m[4] = {0, 0, 0, 0};
    for (int a = kh0; a < kh1; ++a)
        for (int b = kw0; b < kw1; ++b) {
            const uint8_t* xp = x + (((long long)n * iH + ih0 + a) * iW + iw0 + b) * C + c0;
            if (vec_ok) {
                uint32_t w = *(const uint32_t*)xp;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint32_t v = (w >> (8 * i)) & 0xff;
                    m[i] = v > m[i] ? v : m[i];
                }
            } else {
                for (int i = 0; i < 4 && c0 + i < C; ++i) m[i] = xp[i] > m[i] ? xp[i] : m[i];
            }
        }
    uint8_t* yp = y + pix * C + c0;
    if (vec_ok) *(uint32_t*)yp = m[0] | (m[1] << 8) | (m[2] << 16) | (m[3] << 24);
    else
        for (int i = 0; i < 4 && c0 + i < C; ++i) yp[i] = (uint8_t)m[i];
}

__device__ __forceinline__ uint32_t bytemax4(uint32_t a, uint32_t b) {
    uint32_t r = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t x = (a >> (8 * i)) & 0xff, y = (b >> (8 * i)) & 0xff;
        r |= (x > y ? x : y) << (8 * i);
    }
    return r;
}

// grid: x over (ow, 16-channel group) of one output row, y = oh, z = image
__global__ __launch_bounds__(256) void maxpool_u8_16_kernel(const uint8_t* __restrict x,
                                                            uint8_t* __restrict y, int N, int C,
                                                            int iH, int iW, int oH, int oW, int kH,
                                                            int kW, int sH, int sW, int pH, int pW) {
    const int C16 = C >> 4;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= oW * C16) return;
    const int ow = t / C16, cg = t - ow * C16;
    const int oh = blockIdx.y, n = blockIdx.z;
    const int ih0 = oh * sH - pH, iw0 = ow * sW - pW;
    const int kh0 = ih0 < 0 ? -ih0 : 0, kh1 = kH < iH - ih0 ? kH : iH - ih0;
    const int kw0 = iw0 < 0 ? -iw0 : 0, kw1 = kW < iW - iw0 ? kW : iW - iw0;
    const uint8_t* xi = x + (long long)n * iH * iW * C + cg * 16;
    uint32_t m[4] = {0, 0, 0, 0};
    for (int a = kh0; a < kh1; ++a)
        for (int b = kw0; b < kw1; ++b) {
            uint4 v = *(const uint4*)(xi + ((long long)(ih0 + a) * iW + iw0 + b) * C);
            m[0] = bytemax4(m[0], v.x);
            m[1] = bytemax4(m[1], v.y);
            m[2] = bytemax4(m[2], v.z);
            m[3] = bytemax4(m[3], v.w);
        }
    const long long pix = ((long long)n * oH + oh) * oW + ow;
    *(uint4*)(y + pix * C + cg * 16) = make_uint4(m[0], m[1], m[2], m[3]);
}

// the same with a compile-time window: every tap's load is issued before the
// first max (out-of-image taps are skipped by predicate, not by loop bounds)
template <int KH, int KW>
__global__ __launch_bounds__(256) void maxpool_u8_16_fixed_kernel(const uint8_t* __restrict x,
                                                                  uint8_t* __restrict y, int N, int C,
                                                                  int iH, int iW, int oH, int oW, int sH,
                                                                  int sW, int pH, int pW) {
    const int C16 = C >> 4;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= oW * C16) return;
    const int ow = t / C16, cg = t - ow * C16;
    const int oh = blockIdx.y, n = blockIdx.z;
    const int ih0 = oh * sH - pH, iw0 = ow * sW - pW;
    const uint8_t* xi = x + (long long)n * iH * iW * C + cg * 16;
    uint4 v[KH][KW];
#pragma unroll
    for (int a = 0; a < KH; ++a)
#pragma unroll
        for (int b = 0; b < KW; ++b) {
            const int ih = ih0 + a, iw = iw0 + b;
            v[a][b] = ((unsigned)ih < (unsigned)iH && (unsigned)iw < (unsigned)iW)
                          ? *(const uint4*)(xi + ((long long)ih * iW + iw) * C)
                          : make_uint4(0u, 0u, 0u, 0u);
        }
    uint32_t m[4] = {0, 0, 0, 0};
#pragma unroll
    for (int a = 0; a < KH; ++a)
#pragma unroll
        for (int b = 0; b < KW; ++b) {
            m[0] = bytemax4(m[0], v[a][b].x);
            m[1] = bytemax4(m[1], v[a][b].y);
            m[2] = bytemax4(m[2], v[a][b].z);
            m[3] = bytemax4(m[3], v[a][b].w);
        }
    const long long pix = ((long long)n * oH + oh) * oW + ow;
    *(uint4*)(y + pix * C + cg * 16) = make_uint4(m[0], m[1], m[2], m[3]);
}

hipError_t launch_maxpool_u8_nhwc(const uint8_t* x, uint8_t* y, int N, int C, int iH, int iW,
                                  int oH, int oW, int kH, int kW, int sH, int sW, int pH, int pW,
                                  hipStream_t s) {
    if ((C & 15) == 0 && (((uintptr_t)x | (uintptr_t)y) & 15) == 0 && N <= 65535 && oH <= 65535) {
        const long long row = (long long)oW * (C / 16);
        if (row <= 0 || N <= 0 || oH <= 0) return hipSuccess;
        const dim3 grid((unsigned)((row + 255) / 256), (unsigned)oH, (unsigned)N);
        if (kH == 3 && kW == 3)
            hipLaunchKernelGGL((maxpool_u8_16_fixed_kernel<3, 3>), grid, dim3(256), 0, s, x, y, N, C, iH, iW, oH,
                               oW, sH, sW, pH, pW);
        else if (kH == 2 && kW == 2)
            hipLaunchKernelGGL((maxpool_u8_16_fixed_kernel<2, 2>), grid, dim3(256), 0, s, x, y, N, C, iH, iW, oH,
                               oW, sH, sW, pH, pW);
        else
            hipLaunchKernelGGL(maxpool_u8_16_kernel, grid, dim3(256), 0, s, x, y, N, C, iH, iW, oH, oW, kH, kW,
                               sH, sW, pH, pW);
        return hipGetLastError();
    }
    long long total = (long long)N * oH * oW * ((C + 3) / 4);
    if (total <= 0) return hipSuccess;
    hipLaunchKernelGGL(maxpool_u8_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, x,
                       y, N, C, iH, iW, oH, oW, kH, kW, sH, sW, pH, pW);
    return hipGetLastError();
}

}  // namespace nnrh

namespace nnrh {

// ---------------------------------------------------------------------------
// The rest of the QLinear family (QOperator models). Every kernel restates the
// reference expression element by element, including its 16-wide body /
// scalar tail split, so results are bit-identical.

// byte k of a word as the quantized type (0 u8, 1 s8)
__device__ __forceinline__ int byte_q(uint32_t w, int k, int dt) {
    const uint32_t b = (w >> (8 * k)) & 0xffu;
    return dt == 0 ? (int)b : (int)(int8_t)b;
}

// QLinearMul (QLinearMul.cpp:25-231). kind as QLinearAdd: 0 same shape, 1 B
// scalar, 2 A scalar, 3 per channel (a full, b [C]); cs = fl(fl(a_s*b_s)/y_s).
// One element: `a` and `b` are the element's operands (b: B's element for
// kind 0, B's channel value for kind 3); `body` marks the 16-wide body.
__device__ __forceinline__ int qmul_elem(const QMulArgs& p, int a, int b, bool body) {
    if (p.kind == 0) {
        if (body) {
            // fma(fl(fl(a - a_zp) * fl(b - b_zp)), cs, y_zp), roundscale, min / max
            const float va = (float)a - (float)p.a_zp, vb = (float)b - (float)p.b_zp;
            const float v = __builtin_fmaf(va * vb, p.cs, (float)p.y_zp);
            return (int)clamp_minmax(__builtin_rintf(v), (float)p.lo, (float)p.hi);
        }
        const float t1 = p.cs * (float)(a - p.a_zp);
        const float v = t1 * (float)(b - p.b_zp) + (float)p.y_zp;
        return clampi(x86_f2i(__builtin_rintf(v)), p.lo, p.hi);
    }
    if (p.kind == 1 || p.kind == 2) {
        // a: the full operand's element, b: the scalar operand's value
        const bool b_sc = p.kind == 1;
        const float cval = b_sc ? p.cs * (float)(b - p.b_zp) : p.cs * (float)(b - p.a_zp);
        const float d = b_sc ? (float)(a - p.a_zp) : (float)(a - p.b_zp);
        return clampi(x86_f2i(__builtin_rintf(cval * d + (float)p.y_zp)), p.lo, p.hi);
    }
    const float chv = p.cs * (float)(b - p.b_zp);
    if (body) {
        const float v = __builtin_fmaf((float)a - (float)p.a_zp, chv, (float)p.y_zp);
        return (int)clamp_minmax(__builtin_rintf(v), (float)p.lo, (float)p.hi);
    }
    return clampi(x86_f2i(__builtin_rintf(chv * (float)(a - p.a_zp) + (float)p.y_zp)), p.lo, p.hi);
}

// one element per thread: any shape, type or alignment
__global__ __launch_bounds__(256) void qmul_kernel(QMulArgs p) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    const bool b_sc = p.kind == 1, a_sc = p.kind == 2;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < p.n; i += stride) {
        int a, b;
        bool body = false;
        if (p.kind == 0) {
            a = ld_q(p.a, p.dt, i);
            b = ld_q(p.b, p.dt, i);
            body = i < p.n - p.n % 16;
        } else if (b_sc || a_sc) {
            a = b_sc ? ld_q(p.a, p.dt, i) : ld_q(p.b, p.dt, i);
            b = b_sc ? ld_q(p.b, p.dt, 0) : ld_q(p.a, p.dt, 0);
        } else {
            int c;
            long long inner;
            if (p.y_nhwc) { c = (int)(i % p.C); inner = c; }
            else { c = (int)((i / p.HW) % p.C); inner = i % p.HW; }
            a = ld_q(p.a, p.dt, i);
            b = ld_q(p.b, p.dt, c);
            body = inner < (p.y_nhwc ? (p.C - p.C % 16) : (p.HW - p.HW % 16));
        }
        st_q(p.y, p.dt, i, qmul_elem(p, a, b, body));
    }
}

// 16 elements per thread (one 16-byte load per operand, one store): n % 16
// == 0, every streamed operand 16-byte aligned and, per channel, C % 16 == 0
// (NHWC) or HW % 16 == 0 (NCHW). Then every element is in the 16-wide body
// (kind 0: n - n%16 = n; kind 3: the body bound is C or HW itself).
__global__ __launch_bounds__(256) void qmul16_kernel(QMulArgs p) {
    const long long nv = p.n / 16;
    const long long stride = (long long)gridDim.x * blockDim.x;
    const bool b_sc = p.kind == 1, a_sc = p.kind == 2;
    const void* full = a_sc ? p.b : p.a;
    const int sval = b_sc ? ld_q(p.b, p.dt, 0) : (a_sc ? ld_q(p.a, p.dt, 0) : 0);
    for (long long v = (long long)blockIdx.x * blockDim.x + threadIdx.x; v < nv; v += stride) {
        const uint4 av = ((const uint4*)full)[v];
        uint4 bv = make_uint4(0, 0, 0, 0);
        int bc = 0;
        if (p.kind == 0) {
            bv = ((const uint4*)p.b)[v];
        } else if (p.kind == 3) {
            const long long i0 = v * 16;
            if (p.y_nhwc) bv = *(const uint4*)((const uint8_t*)p.b + (i0 % p.C));
            else bc = ld_q(p.b, p.dt, (i0 / p.HW) % p.C);
        }
        const uint32_t aw[4] = {av.x, av.y, av.z, av.w}, bw[4] = {bv.x, bv.y, bv.z, bv.w};
        uint32_t ow[4];
        if (p.dt == 0 && (p.kind == 0 || p.kind == 3) && __builtin_isfinite(p.cs)) {
            // uint8 body: clamp to [0, 255] then nearest even is one
            // v_cvt_pk_u8_f32 per byte (finite inputs; +-inf saturate alike)
            const float az = (float)p.a_zp, bz = (float)p.b_zp, yz = (float)p.y_zp;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                uint32_t o = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float va = (float)((aw[k] >> (8 * j)) & 0xffu) - az;
                    float v;
                    if (p.kind == 0) {
                        const float vb = (float)((bw[k] >> (8 * j)) & 0xffu) - bz;
                        v = __builtin_fmaf(va * vb, p.cs, yz);
                    } else {
                        const int b = p.y_nhwc ? (int)((bw[k] >> (8 * j)) & 0xffu) : bc;
                        v = __builtin_fmaf(va, p.cs * (float)(b - p.b_zp), yz);
                    }
                    o = __builtin_amdgcn_cvt_pk_u8_f32(v, j, o);
                }
                ow[k] = o;
            }
            ((uint4*)p.y)[v] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
            continue;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t o = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int a = byte_q(aw[k], j, p.dt);
                int b;
                if (p.kind == 0 || (p.kind == 3 && p.y_nhwc)) b = byte_q(bw[k], j, p.dt);
                else if (p.kind == 3) b = bc;
                else b = sval;
                o |= ((uint32_t)qmul_elem(p, a, b, true) & 0xffu) << (8 * j);
            }
            ow[k] = o;
        }
        ((uint4*)p.y)[v] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    }
}

hipError_t launch_qmul(const QMulArgs& p, hipStream_t s) {
    if (p.n <= 0) return hipSuccess;
    const auto al = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
    bool vec = p.n % 16 == 0 && al(p.y) && al(p.kind == 2 ? p.b : p.a);
    if (p.kind == 0) vec = vec && al(p.b);
    if (p.kind == 3) vec = vec && (p.y_nhwc ? (p.C % 16 == 0 && al(p.b)) : p.HW % 16 == 0);
    const long long work = vec ? p.n / 16 : p.n;
    long long blocks = (work + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (vec) hipLaunchKernelGGL(qmul16_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p);
    else hipLaunchKernelGGL(qmul_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p);
    return hipGetLastError();
}

// QLinearGlobalAveragePool (QLinearGlobalAveragePool.cpp:38-60), RQ-F: the
// int32 sum of a (n, c) plane (exact in any order), minus x_zp * spatial,
// times rs = fl(x_s / fl(y_s * spatial)), nearbyint, + y_zp, clamp.
__device__ __forceinline__ int qgap_out(uint32_t sum, int spatial, float rs, int x_zp, int y_zp, int lo, int hi) {
    sum -= (uint32_t)x_zp * (uint32_t)spatial;
    int32_t q = x86_f2i(__builtin_rintf((float)(int32_t)sum * rs));
    q = (int32_t)((uint32_t)q + (uint32_t)y_zp);
    return clampi(q, lo, hi);
}

// Any layout / alignment. NCHW: one wave per plane; NHWC: one thread per
// (n, c), channels coalesced.
__global__ __launch_bounds__(256) void qgap_kernel(const void* __restrict x, void* __restrict y, int N, int C,
                                                   int spatial, int nhwc, int dt, float rs, int x_zp, int y_zp,
                                                   int lo, int hi) {
    long long nc;
    uint32_t sum = 0;
    if (nhwc) {
        nc = (long long)blockIdx.x * 256 + threadIdx.x;
        if (nc >= (long long)N * C) return;
        const long long n = nc / C, c = nc - n * C;
        for (int s = 0; s < spatial; ++s) sum += (uint32_t)ld_q(x, dt, (n * spatial + s) * C + c);
    } else {
        nc = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
        const int lane = threadIdx.x & 63;
        if (nc >= (long long)N * C) return;
        for (int s = lane; s < spatial; s += 64) sum += (uint32_t)ld_q(x, dt, nc * spatial + s);
        for (int off = 32; off > 0; off >>= 1) sum += (uint32_t)__shfl_xor((int)sum, off, 64);
        if (lane) return;
    }
    st_q(y, dt, nc, qgap_out(sum, spatial, rs, x_zp, y_zp, lo, hi));
}

// NCHW, spatial % 16 == 0, x 16-byte aligned: one wave per plane, 16 bytes
// per lane per load, byte sums by v_sad_u8 (int8 is biased to uint8 by
// flipping the sign bit, then 128 * spatial is taken off)
__global__ __launch_bounds__(256) void qgap_nchw16_kernel(const void* __restrict x, void* __restrict y, int N, int C,
                                                          int spatial, int dt, float rs, int x_zp, int y_zp, int lo,
                                                          int hi) {
    const long long nc = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (nc >= (long long)N * C) return;
    const uint4* p = (const uint4*)((const uint8_t*)x + nc * spatial);
    const uint32_t flip = dt ? 0x80808080u : 0u;
    uint32_t sum = 0;
    const int nv = spatial / 16;
    for (int v = lane; v < nv; v += 64) {
        const uint4 q = p[v];
        sum = __builtin_amdgcn_sad_u8(q.x ^ flip, 0u, sum);
        sum = __builtin_amdgcn_sad_u8(q.y ^ flip, 0u, sum);
        sum = __builtin_amdgcn_sad_u8(q.z ^ flip, 0u, sum);
        sum = __builtin_amdgcn_sad_u8(q.w ^ flip, 0u, sum);
    }
    for (int off = 32; off > 0; off >>= 1) sum += (uint32_t)__shfl_xor((int)sum, off, 64);
    if (lane) return;
    if (dt) sum -= 128u * (uint32_t)spatial;
    st_q(y, dt, nc, qgap_out(sum, spatial, rs, x_zp, y_zp, lo, hi));
}

// NHWC, C % 16 == 0, x 16-byte aligned. Block (n, channel slice): each
// thread owns one 16-channel group and every P-th pixel of image n, loads
// 16 bytes per pixel (a wave reads whole pixel rows) and keeps the 16 sums
// as pairs of 16-bit lanes (bytes 0/2 and 1/3 of each word), flushed to
// 32-bit totals every 256 pixels (256 * 255 < 2^16). The P partial sums of a
// channel are added in LDS.
constexpr int QGAP_NT = 512;
constexpr int QGAP_UNROLL = 8;
__global__ __launch_bounds__(QGAP_NT) void qgap_nhwc16_kernel(const void* __restrict x, void* __restrict y, int C,
                                                              int spatial, int dt, float rs, int x_zp, int y_zp,
                                                              int lo, int hi) {
    __shared__ uint32_t red[QGAP_NT * 16];
    const int G = C / 16;
    const int n = blockIdx.x;
    const int t = threadIdx.x;
    int P, g, pl;
    if (G >= QGAP_NT) { P = 1; g = blockIdx.y * QGAP_NT + t; pl = 0; }
    else { P = QGAP_NT / G; g = t % G; pl = t / G; }
    const bool active = g < G && pl < P;
    const uint32_t flip = dt ? 0x80808080u : 0u;
    uint32_t tot[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) tot[j] = 0;
    if (active) {
        const uint4* base = (const uint4*)((const uint8_t*)x + (size_t)n * spatial * C) + g;
        long long s = pl;
        while (s < spatial) {
            // one run: at most 256 pixels of this thread before a flush
            const long long run_end = s + 256LL * P < spatial ? s + 256LL * P : spatial;
            uint32_t acc[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[k] = 0;
            for (; s + (QGAP_UNROLL - 1) * (long long)P < run_end; s += QGAP_UNROLL * (long long)P) {
                uint4 v[QGAP_UNROLL];
#pragma unroll
                for (int u = 0; u < QGAP_UNROLL; ++u) v[u] = base[(size_t)(s + u * (long long)P) * G];
#pragma unroll
                for (int u = 0; u < QGAP_UNROLL; ++u) {
                    const uint32_t w[4] = {v[u].x ^ flip, v[u].y ^ flip, v[u].z ^ flip, v[u].w ^ flip};
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        acc[2 * k] += w[k] & 0x00ff00ffu;
                        acc[2 * k + 1] += (w[k] >> 8) & 0x00ff00ffu;
                    }
                }
            }
            for (; s < run_end; s += P) {
                const uint4 v = base[(size_t)s * G];
                const uint32_t w[4] = {v.x ^ flip, v.y ^ flip, v.z ^ flip, v.w ^ flip};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    acc[2 * k] += w[k] & 0x00ff00ffu;
                    acc[2 * k + 1] += (w[k] >> 8) & 0x00ff00ffu;
                }
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                tot[4 * k + 0] += acc[2 * k] & 0xffffu;
                tot[4 * k + 2] += acc[2 * k] >> 16;
                tot[4 * k + 1] += acc[2 * k + 1] & 0xffffu;
                tot[4 * k + 3] += acc[2 * k + 1] >> 16;
            }
        }
    }
    const uint32_t bias = dt ? 128u * (uint32_t)spatial : 0u;
    if (P == 1) {
        if (!active) return;
        uint32_t ow[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t o = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                o |= ((uint32_t)qgap_out(tot[4 * k + j] - bias, spatial, rs, x_zp, y_zp, lo, hi) & 0xffu) << (8 * j);
            ow[k] = o;
        }
        uint8_t* yp = (uint8_t*)y + (size_t)n * C + (size_t)g * 16;
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int j = 0; j < 4; ++j) yp[4 * k + j] = (uint8_t)(ow[k] >> (8 * j));
        return;
    }
    // partials: red[pl * C + c]
    if (active) {
#pragma unroll
        for (int j = 0; j < 16; ++j) red[pl * C + g * 16 + j] = tot[j];
    }
    __syncthreads();
    // with few channels, two levels: thread (c, q) adds partials q, q + Q,
    // ...; then each channel adds its Q values. R rows of partials are left.
    const int Q = QGAP_NT / C;
    int R = P;
    if (Q >= 2) {
        uint32_t part = 0;
        const int c = t % C, q = t / C;
        if (q < Q)
            for (int p2 = q; p2 < P; p2 += Q) part += red[p2 * C + c];
        __syncthreads();
        if (q < Q) red[q * C + c] = part;
        __syncthreads();
        R = Q;
    }
    for (int cc = t; cc < C; cc += QGAP_NT) {
        uint32_t sum = 0;
        for (int r = 0; r < R; ++r) sum += red[r * C + cc];
        st_q(y, dt, (long long)n * C + cc, qgap_out(sum - bias, spatial, rs, x_zp, y_zp, lo, hi));
    }
}

hipError_t launch_qgap(const void* x, void* y, int N, int C, int spatial, int nhwc, int dt, float rs, int x_zp,
                       int y_zp, int lo, int hi, hipStream_t s) {
    const long long rows = (long long)N * C;
    if (rows <= 0) return hipSuccess;
    const bool al = ((uintptr_t)x & 15) == 0;
    if (nhwc && al && C % 16 == 0 && spatial > 0) {
        const int G = C / 16;
        const unsigned slices = G >= QGAP_NT ? (unsigned)((G + QGAP_NT - 1) / QGAP_NT) : 1u;
        if (slices <= 65535u) {
            hipLaunchKernelGGL(qgap_nhwc16_kernel, dim3((unsigned)N, slices), dim3(QGAP_NT), 0, s, x, y, C, spatial,
                               dt, rs, x_zp, y_zp, lo, hi);
            return hipGetLastError();
        }
    }
    if (!nhwc && al && spatial % 16 == 0) {
        hipLaunchKernelGGL(qgap_nchw16_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, x, y, N, C,
                           spatial, dt, rs, x_zp, y_zp, lo, hi);
        return hipGetLastError();
    }
    const long long blocks = nhwc ? (rows + 255) / 256 : (rows + 3) / 4;
    hipLaunchKernelGGL(qgap_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, y, N, C, spatial, nhwc, dt, rs,
                       x_zp, y_zp, lo, hi);
    return hipGetLastError();
}

// QLinearAveragePool (QLinearAveragePool.cpp:67-115): in-image taps only,
// avg = fl(fl(sum * x_s) / count), q = nearbyint(fl(avg / y_s)) + y_zp, clamp.
__device__ __forceinline__ int qavg_out(int32_t sum, int count, float x_s, float y_s, int y_zp, int lo, int hi) {
    if (count == 0) count = 1;
    const float t = (float)sum * x_s;
    const float avg = t / (float)count;
    int32_t q = x86_f2i(__builtin_rintf(avg / y_s));
    q = (int32_t)((uint32_t)q + (uint32_t)y_zp);
    return clampi(q, lo, hi);
}

// One thread per output element, NCHW or NHWC, any alignment.
__global__ __launch_bounds__(256) void qavgpool_kernel(const void* __restrict x, void* __restrict y, int N, int C,
                                                       int iH, int iW, int oH, int oW, int kH, int kW, int sH,
                                                       int sW, int pH, int pW, int nhwc, int dt, float x_s,
                                                       int x_zp, float y_s, int y_zp, int lo, int hi) {
    const long long total = (long long)N * C * oH * oW;
    for (long long o = (long long)blockIdx.x * 256 + threadIdx.x; o < total; o += (long long)gridDim.x * 256) {
        int n, c, oh, ow;
        if (nhwc) {
            c = (int)(o % C); long long r = o / C;
            ow = (int)(r % oW); r /= oW;
            oh = (int)(r % oH); n = (int)(r / oH);
        } else {
            ow = (int)(o % oW); long long r = o / oW;
            oh = (int)(r % oH); r /= oH;
            c = (int)(r % C); n = (int)(r / C);
        }
        int32_t sum = 0;
        int count = 0;
        for (int kh = 0; kh < kH; ++kh) {
            const int ih = oh * sH - pH + kh;
            if (ih < 0 || ih >= iH) continue;
            for (int kw = 0; kw < kW; ++kw) {
                const int iw = ow * sW - pW + kw;
                if (iw < 0 || iw >= iW) continue;
                const long long i = nhwc ? (((long long)n * iH + ih) * iW + iw) * C + c
                                         : (((long long)n * C + c) * iH + ih) * iW + iw;
                sum += ld_q(x, dt, i) - x_zp;
                ++count;
            }
        }
        st_q(y, dt, o, qavg_out(sum, count, x_s, y_s, y_zp, lo, hi));
    }
}

// NHWC, C % 16 == 0, x and y 16-byte aligned, kH * kW <= 256: one thread per
// (output pixel, 16-channel group), one 16-byte load per in-image tap, the 16
// sums kept as 16-bit lane pairs (at most 256 taps of 255). The int32 sum of
// (x - x_zp) over the taps is sum(x) - count * x_zp exactly.
__global__ __launch_bounds__(256) void qavgpool_nhwc16_kernel(const void* __restrict x, void* __restrict y, int N,
                                                              int C, int iH, int iW, int oH, int oW, int kH, int kW,
                                                              int sH, int sW, int pH, int pW, int dt, float x_s,
                                                              int x_zp, float y_s, int y_zp, int lo, int hi) {
    const int G = C / 16;
    const long long total = (long long)N * oH * oW * G;
    const uint32_t flip = dt ? 0x80808080u : 0u;
    for (long long o = (long long)blockIdx.x * 256 + threadIdx.x; o < total; o += (long long)gridDim.x * 256) {
        const int g = (int)(o % G);
        long long r = o / G;
        const int ow = (int)(r % oW);
        r /= oW;
        const int oh = (int)(r % oH);
        const int n = (int)(r / oH);
        uint32_t acc[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] = 0;
        int count = 0;
        const int h0 = oh * sH - pH, w0 = ow * sW - pW;
        for (int kh = 0; kh < kH; ++kh) {
            const int ih = h0 + kh;
            if (ih < 0 || ih >= iH) continue;
            const uint4* row = (const uint4*)((const uint8_t*)x + (((long long)n * iH + ih) * iW) * C) + g;
            for (int kw = 0; kw < kW; ++kw) {
                const int iw = w0 + kw;
                if (iw < 0 || iw >= iW) continue;
                const uint4 v = row[(long long)iw * G];
                const uint32_t w[4] = {v.x ^ flip, v.y ^ flip, v.z ^ flip, v.w ^ flip};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    acc[2 * k] += w[k] & 0x00ff00ffu;
                    acc[2 * k + 1] += (w[k] >> 8) & 0x00ff00ffu;
                }
                ++count;
            }
        }
        // channel 4k+j: pair word 2k holds bytes 0 / 2, word 2k+1 bytes 1 / 3
        const int32_t off = (dt ? 128 : 0) * count + count * x_zp;
        uint32_t ow_[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int32_t s0 = (int32_t)(acc[2 * k] & 0xffffu), s2 = (int32_t)(acc[2 * k] >> 16);
            const int32_t s1 = (int32_t)(acc[2 * k + 1] & 0xffffu), s3 = (int32_t)(acc[2 * k + 1] >> 16);
            ow_[k] = ((uint32_t)qavg_out(s0 - off, count, x_s, y_s, y_zp, lo, hi) & 0xffu) |
                     (((uint32_t)qavg_out(s1 - off, count, x_s, y_s, y_zp, lo, hi) & 0xffu) << 8) |
                     (((uint32_t)qavg_out(s2 - off, count, x_s, y_s, y_zp, lo, hi) & 0xffu) << 16) |
                     (((uint32_t)qavg_out(s3 - off, count, x_s, y_s, y_zp, lo, hi) & 0xffu) << 24);
        }
        ((uint4*)y)[o] = make_uint4(ow_[0], ow_[1], ow_[2], ow_[3]);
    }
}

// the same for a fixed window: every tap's 16-byte load (predicated on the
// tap lying in the image) is issued before the first sum
template <int KH, int KW>
__global__ __launch_bounds__(256) void qavgpool_nhwc16_fixed_kernel(const void* __restrict x, void* __restrict y,
                                                                    int N, int C, int iH, int iW, int oH, int oW,
                                                                    int sH, int sW, int pH, int pW, int dt, float x_s,
                                                                    int x_zp, float y_s, int y_zp, int lo, int hi) {
    const int G = C / 16;
    const long long total = (long long)N * oH * oW * G;
    const uint32_t flip = dt ? 0x80808080u : 0u;
    for (long long o = (long long)blockIdx.x * 256 + threadIdx.x; o < total; o += (long long)gridDim.x * 256) {
        const int g = (int)(o % G);
        long long r = o / G;
        const int ow = (int)(r % oW);
        r /= oW;
        const int oh = (int)(r % oH);
        const int n = (int)(r / oH);
        const int h0 = oh * sH - pH, w0 = ow * sW - pW;
        const uint4* img = (const uint4*)((const uint8_t*)x + (long long)n * iH * iW * C) + g;
        uint4 v[KH * KW];
        bool ok[KH * KW];
#pragma unroll
        for (int kh = 0; kh < KH; ++kh)
#pragma unroll
            for (int kw = 0; kw < KW; ++kw) {
                const int ih = h0 + kh, iw = w0 + kw;
                const bool in = ih >= 0 && ih < iH && iw >= 0 && iw < iW;
                ok[kh * KW + kw] = in;
                v[kh * KW + kw] = in ? img[((long long)ih * iW + iw) * G] : make_uint4(0, 0, 0, 0);
            }
        uint32_t acc[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] = 0;
        int count = 0;
#pragma unroll
        for (int t = 0; t < KH * KW; ++t) {
            if (!ok[t]) continue;
            ++count;
            const uint32_t w[4] = {v[t].x ^ flip, v[t].y ^ flip, v[t].z ^ flip, v[t].w ^ flip};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                acc[2 * k] += w[k] & 0x00ff00ffu;
                acc[2 * k + 1] += (w[k] >> 8) & 0x00ff00ffu;
            }
        }
        const int32_t off = (dt ? 128 : 0) * count + count * x_zp;
        uint32_t ow_[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int32_t s0 = (int32_t)(acc[2 * k] & 0xffffu), s2 = (int32_t)(acc[2 * k] >> 16);
            const int32_t s1 = (int32_t)(acc[2 * k + 1] & 0xffffu), s3 = (int32_t)(acc[2 * k + 1] >> 16);
            ow_[k] = ((uint32_t)qavg_out(s0 - off, count, x_s, y_s, y_zp, lo, hi) & 0xffu) |
                     (((uint32_t)qavg_out(s1 - off, count, x_s, y_s, y_zp, lo, hi) & 0xffu) << 8) |
                     (((uint32_t)qavg_out(s2 - off, count, x_s, y_s, y_zp, lo, hi) & 0xffu) << 16) |
                     (((uint32_t)qavg_out(s3 - off, count, x_s, y_s, y_zp, lo, hi) & 0xffu) << 24);
        }
        ((uint4*)y)[o] = make_uint4(ow_[0], ow_[1], ow_[2], ow_[3]);
    }
}

hipError_t launch_qavgpool(const void* x, void* y, int N, int C, int iH, int iW, int oH, int oW, int kH, int kW,
                           int sH, int sW, int pH, int pW, int nhwc, int dt, float x_s, int x_zp, float y_s,
                           int y_zp, int lo, int hi, hipStream_t s) {
    const long long total = (long long)N * C * oH * oW;
    if (total <= 0) return hipSuccess;
    const bool vec = nhwc && C % 16 == 0 && (((uintptr_t)x | (uintptr_t)y) & 15) == 0 && kH * kW <= 256;
    long long blocks = ((vec ? total / 16 : total) + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (vec && kH == 3 && kW == 3)
        hipLaunchKernelGGL((qavgpool_nhwc16_fixed_kernel<3, 3>), dim3((unsigned)blocks), dim3(256), 0, s, x, y, N, C,
                           iH, iW, oH, oW, sH, sW, pH, pW, dt, x_s, x_zp, y_s, y_zp, lo, hi);
    else if (vec && kH == 2 && kW == 2)
        hipLaunchKernelGGL((qavgpool_nhwc16_fixed_kernel<2, 2>), dim3((unsigned)blocks), dim3(256), 0, s, x, y, N, C,
                           iH, iW, oH, oW, sH, sW, pH, pW, dt, x_s, x_zp, y_s, y_zp, lo, hi);
    else if (vec)
        hipLaunchKernelGGL(qavgpool_nhwc16_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, y, N, C, iH, iW, oH,
                           oW, kH, kW, sH, sW, pH, pW, dt, x_s, x_zp, y_s, y_zp, lo, hi);
    else
        hipLaunchKernelGGL(qavgpool_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, y, N, C, iH, iW, oH, oW, kH,
                           kW, sH, sW, pH, pW, nhwc, dt, x_s, x_zp, y_s, y_zp, lo, hi);
    return hipGetLastError();
}

// One input of QLinearConcat (QLinearConcat.cpp:70-104, :119-236): `outer`
// chunks of `count` elements go to y at o * y_row + y_off. Matching scale and
// zero point copy; otherwise the first count - count % 16 elements of a chunk
// (count >= 16) take the 16-wide body rne(clamp(fma(rs, x - x_zp, y_zp))),
// the rest the scalar nearbyint(fl(rs * (x - x_zp)) + y_zp), clamped.
__device__ __forceinline__ int qconcat_elem(int xv, bool body, float rs, int x_zp, int y_zp, int lo, int hi) {
    if (body) {
        float v = __builtin_fmaf(rs, (float)xv - (float)x_zp, (float)y_zp);
        v = v > (float)lo ? v : (float)lo;
        v = v < (float)hi ? v : (float)hi;
        return (int)__builtin_rintf(v);
    }
    const float v = rs * (float)(xv - x_zp) + (float)y_zp;
    return clampi(x86_f2i(__builtin_rintf(v)), lo, hi);
}

// W bytes per thread (W = 1, 4, 8 or 16, dividing count, y_row and y_off, both
// pointers W-aligned). W divides 16, so a unit lies wholly in a chunk's body
// or wholly in its tail.
template <int W>
__global__ __launch_bounds__(256) void qconcat_kernel(const void* __restrict x, void* __restrict y, long long outer,
                                                      long long count, long long y_row, long long y_off, int dt,
                                                      int copy, float rs, int x_zp, int y_zp, int lo, int hi) {
    const long long units = outer * count / W;
    const long long body = count >= 16 ? count - count % 16 : 0;
    for (long long u = (long long)blockIdx.x * 256 + threadIdx.x; u < units; u += (long long)gridDim.x * 256) {
        const long long e = u * W;
        const long long o = e / count, i = e - o * count;
        uint8_t* dst = (uint8_t*)y + o * y_row + y_off + i;
        if constexpr (W == 1) {
            const int xv = ld_q(x, dt, e);
            *dst = (uint8_t)(copy ? xv : qconcat_elem(xv, i < body, rs, x_zp, y_zp, lo, hi));
        } else {
            constexpr int NW = W / 4;
            uint32_t w[NW];
            if constexpr (W == 16) {
                const uint4 v = ((const uint4*)x)[u];
                w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
            } else if constexpr (W == 8) {
                const uint2 v = ((const uint2*)x)[u];
                w[0] = v.x; w[1] = v.y;
            } else {
                w[0] = ((const uint32_t*)x)[u];
            }
            if (!copy) {
                const bool bd = i < body;
#pragma unroll
                for (int k = 0; k < NW; ++k) {
                    uint32_t r = 0;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        r |= ((uint32_t)qconcat_elem(byte_q(w[k], j, dt), bd, rs, x_zp, y_zp, lo, hi) & 0xffu)
                             << (8 * j);
                    w[k] = r;
                }
            }
            if constexpr (W == 16) *(uint4*)dst = make_uint4(w[0], w[1], w[2], w[3]);
            else if constexpr (W == 8) *(uint2*)dst = make_uint2(w[0], w[1]);
            else *(uint32_t*)dst = w[0];
        }
    }
}

hipError_t launch_qconcat_part(const void* x, void* y, long long outer, long long count, long long y_row,
                               long long y_off, int dt, int copy, float rs, int x_zp, int y_zp, int lo, int hi,
                               hipStream_t s) {
    const long long total = outer * count;
    if (total <= 0) return hipSuccess;
    const uintptr_t al = (uintptr_t)x | (uintptr_t)y | (uintptr_t)count | (uintptr_t)y_row | (uintptr_t)y_off;
    const int W = (al & 15) == 0 ? 16 : (al & 7) == 0 ? 8 : (al & 3) == 0 ? 4 : 1;
    long long blocks = (total / W + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    const dim3 grid((unsigned)blocks), block(256);
    if (W == 16)
        hipLaunchKernelGGL((qconcat_kernel<16>), grid, block, 0, s, x, y, outer, count, y_row, y_off, dt, copy, rs,
                           x_zp, y_zp, lo, hi);
    else if (W == 8)
        hipLaunchKernelGGL((qconcat_kernel<8>), grid, block, 0, s, x, y, outer, count, y_row, y_off, dt, copy, rs,
                           x_zp, y_zp, lo, hi);
    else if (W == 4)
        hipLaunchKernelGGL((qconcat_kernel<4>), grid, block, 0, s, x, y, outer, count, y_row, y_off, dt, copy, rs,
                           x_zp, y_zp, lo, hi);
    else
        hipLaunchKernelGGL((qconcat_kernel<1>), grid, block, 0, s, x, y, outer, count, y_row, y_off, dt, copy, rs,
                           x_zp, y_zp, lo, hi);
    return hipGetLastError();
}

// BatchNormalization after fold_bn_qdq (BatchNormalization.cpp:246-376): per
// channel y = A[c] * x + B[c] into uint8, x uint8 (DQ -> BN -> Q folded) or
// fp32 (BN -> Q folded), NCHW or NHWC, with the reference's per-layout
// 16-wide body / scalar tail:
//   NCHW, body of each plane: fma(x, A, B), clamp [0, 255], round to nearest
//         even; tail: fl(x * A) + B, clamp, roundf (ties away from zero)
//   NHWC, body of each pixel's channels: fma(x, A, B), round to nearest even
//         (x86 cvtps: INT32_MIN out of range), then an UNSIGNED saturation to
//         255 -- a negative value becomes 255 -- with no clamp before it for
//         uint8 input (ops_x64.h:110-129) and a [0, 255] clamp for fp32 input
//         (:135-155); tail: fl(A * x) + B, clamp, lrintf (nearest even)
// The scalar clamps are std::max(0, std::min(255, v)).
__device__ __forceinline__ float std_clamp255(float v) {
    const float m = v < 255.0f ? v : 255.0f;    // std::min(255.0f, v)
    return 0.0f < m ? m : 0.0f;                 // std::max(0.0f, m)
}
__device__ __forceinline__ float simd_clamp255(float v) {
    // _mm512_max_ps(_mm512_min_ps(v, 255), 0): NaN takes the second operand
    const float m = v < 255.0f ? v : 255.0f;
    return m > 0.0f ? m : 0.0f;
}

template <bool F32_IN>
__global__ __launch_bounds__(256) void bn_affine_u8_kernel(const void* __restrict x, uint8_t* __restrict y,
                                                           const float* __restrict A, const float* __restrict B,
                                                           long long total, int C, long long HW, int nhwc) {
    const long long body_hw = HW - HW % 16;
    const int body_c = C - C % 16;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long long)gridDim.x * 256) {
        const float xf = F32_IN ? ((const float*)x)[i] : (float)((const uint8_t*)x)[i];
        int c;
        bool body;
        if (nhwc) {
            c = (int)(i % C);
            body = c < body_c;
        } else {
            const long long pix = i % HW;
            c = (int)((i / HW) % C);
            body = pix < body_hw;
        }
        const float a = A[c], b = B[c];
        uint32_t q;
        if (body) {
            float v = __builtin_fmaf(xf, a, b);
            if (!nhwc || F32_IN) v = simd_clamp255(v);
            const uint32_t r = (uint32_t)x86_f2i(__builtin_rintf(v));
            q = r > 255u ? 255u : r;               // unsigned saturation
        } else if (nhwc) {
            const float v = std_clamp255(a * xf + b);
            q = (uint32_t)__builtin_rintf(v);
        } else {
            const float v = std_clamp255(xf * a + b);
            q = (uint32_t)roundf(v);
        }
        y[i] = (uint8_t)q;
    }
}

// 16 elements per thread: NHWC with C % 16 == 0 (16 channels of one pixel)
// or NCHW with HW % 16 == 0 (16 pixels of one plane), 16-byte aligned
// operands. Every element is then in a 16-wide body.
// the 16 channels' A / B of the vector starting at element i0
template <bool NHWC>
__device__ __forceinline__ void bn_coeffs_16(float* a, float* b, const float* __restrict A, const float* __restrict B,
                                             long long i0, int C, long long HW) {
    if (NHWC) {
        const int c0 = (int)(i0 % C);
#pragma unroll
        for (int k = 0; k < 16; ++k) { a[k] = A[c0 + k]; b[k] = B[c0 + k]; }
    } else {
        const int c = (int)((i0 / HW) % C);
        const float ac = A[c], bc = B[c];
#pragma unroll
        for (int k = 0; k < 16; ++k) { a[k] = ac; b[k] = bc; }
    }
}

// NHWC uint8 input with finite A / B: t = fma(x, A, B) is never NaN (an
// infinite A with x = 0, or A*x = +inf with B = -inf, would make it NaN), and
// round-to-nearest-even + unsigned saturation (negative -> 255) is
// t < -0.5 ? 255 : v_cvt_pk_u8_f32(t) (t = -0.5 rounds to -0, i.e. 0)
__device__ __forceinline__ uint4 bn_affine_16_u8q(const float* xf, const float* a, const float* b) {
    uint32_t o[4] = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const float t = __builtin_fmaf(xf[k], a[k], b[k]);
        o[k >> 2] = t < -0.5f ? (o[k >> 2] | (0xffu << (8 * (k & 3))))
                              : __builtin_amdgcn_cvt_pk_u8_f32(t, k & 3, o[k >> 2]);
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

template <bool F32_IN, bool NHWC>
__device__ __forceinline__ uint4 bn_affine_16(const float* xf, const float* a, const float* b) {
    uint32_t o[4] = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        float t = __builtin_fmaf(xf[k], a[k], b[k]);
        if (!NHWC || F32_IN) t = simd_clamp255(t);
        const uint32_t r = (uint32_t)x86_f2i(__builtin_rintf(t));
        o[k >> 2] |= (r > 255u ? 255u : r) << (8 * (k & 3));
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// 16 elements per vector: NHWC with C % 16 == 0 (16 channels of one pixel)
// or NCHW with HW % 16 == 0 (16 pixels of one plane), 16-byte aligned
// operands; every element is then in a 16-wide body. uint8 input: each
// thread has BN_U8_VECS vectors' loads in flight (block-strided, coalesced).
// NHWC with 256 % (C / 16) == 0: a thread's vectors all start at the same
// channel (strides are multiples of 256 vectors), so its A / B are loaded
// once.
constexpr int BN_U8_VECS = 4;
template <bool F32_IN, bool NHWC>
__global__ __launch_bounds__(256) void bn_affine_u8_16_kernel(const void* __restrict x, uint8_t* __restrict y,
                                                              const float* __restrict A, const float* __restrict B,
                                                              long long nv, int C, long long HW) {
    constexpr int U = F32_IN ? 1 : BN_U8_VECS;
    const bool fixed = NHWC && 256 % (C / 16) == 0;
    float a[16], b[16];
    bool fast_u8q = false;   // NHWC uint8 body through bn_affine_16_u8q
    if (fixed) {
        bn_coeffs_16<NHWC>(a, b, A, B, (long long)(threadIdx.x % (C / 16)) * 16, C, HW);
        if (NHWC && !F32_IN) {
            fast_u8q = true;
#pragma unroll
            for (int k = 0; k < 16; ++k) fast_u8q &= __builtin_isfinite(a[k]) && __builtin_isfinite(b[k]);
        }
    }
    for (long long base = (long long)blockIdx.x * 256 * U; base < nv; base += (long long)gridDim.x * 256 * U) {
        if (F32_IN) {
            const long long v = base + threadIdx.x;
            if (v >= nv) continue;
            float xf[16];
            const float4* p = (const float4*)x + v * 4;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 q = p[k];
                xf[4 * k] = q.x; xf[4 * k + 1] = q.y; xf[4 * k + 2] = q.z; xf[4 * k + 3] = q.w;
            }
            if (!fixed) bn_coeffs_16<NHWC>(a, b, A, B, v * 16, C, HW);
            ((uint4*)y)[v] = bn_affine_16<F32_IN, NHWC>(xf, a, b);
        } else {
            uint4 q[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const long long v = base + u * 256 + threadIdx.x;
                q[u] = v < nv ? ((const uint4*)x)[v] : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const long long v = base + u * 256 + threadIdx.x;
                if (v >= nv) continue;
                const uint32_t w[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
                float xf[16];
#pragma unroll
                for (int k = 0; k < 16; ++k) xf[k] = (float)((w[k >> 2] >> (8 * (k & 3))) & 0xffu);
                if (!fixed) bn_coeffs_16<NHWC>(a, b, A, B, v * 16, C, HW);
                ((uint4*)y)[v] = fast_u8q ? bn_affine_16_u8q(xf, a, b) : bn_affine_16<F32_IN, NHWC>(xf, a, b);
            }
        }
    }
}

hipError_t launch_bn_affine_u8(const void* x, int x_f32, uint8_t* y, const float* A, const float* B, long long N,
                               int C, long long HW, int nhwc, hipStream_t s) {
    const long long total = N * C * HW;
    if (total <= 0) return hipSuccess;
    const bool al = (((uintptr_t)x | (uintptr_t)y) & 15) == 0;
    if (al && (nhwc ? C % 16 == 0 : HW % 16 == 0)) {
        const long long nv = total / 16;
        const long long per_block = 256LL * (x_f32 ? 1 : BN_U8_VECS);
        long long blocks = (nv + per_block - 1) / per_block;
        if (blocks > 65536) blocks = 65536;
        const dim3 g((unsigned)blocks), b(256);
        if (x_f32 && nhwc)
            hipLaunchKernelGGL((bn_affine_u8_16_kernel<true, true>), g, b, 0, s, x, y, A, B, nv, C, HW);
        else if (x_f32)
            hipLaunchKernelGGL((bn_affine_u8_16_kernel<true, false>), g, b, 0, s, x, y, A, B, nv, C, HW);
        else if (nhwc)
            hipLaunchKernelGGL((bn_affine_u8_16_kernel<false, true>), g, b, 0, s, x, y, A, B, nv, C, HW);
        else
            hipLaunchKernelGGL((bn_affine_u8_16_kernel<false, false>), g, b, 0, s, x, y, A, B, nv, C, HW);
        return hipGetLastError();
    }
    long long blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (x_f32)
        hipLaunchKernelGGL((bn_affine_u8_kernel<true>), dim3((unsigned)blocks), dim3(256), 0, s, x, y, A, B, total,
                           C, HW, nhwc);
    else
        hipLaunchKernelGGL((bn_affine_u8_kernel<false>), dim3((unsigned)blocks), dim3(256), 0, s, x, y, A, B, total,
                           C, HW, nhwc);
    return hipGetLastError();
}

// inference BatchNormalization in fp32: y = alpha[c] * x + beta[c]
// (BatchNormalization.cpp:126-160; alpha / beta precomputed on the host)
__global__ __launch_bounds__(256) void bn_f32_kernel(const float* __restrict x, float* __restrict y,
                                                     const float* __restrict A, const float* __restrict B,
                                                     long long total, int C, long long HW, int nhwc) {
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long long)gridDim.x * 256) {
        const int c = nhwc ? (int)(i % C) : (int)((i / HW) % C);
        y[i] = A[c] * x[i] + B[c];
    }
}

hipError_t launch_bn_f32(const float* x, float* y, const float* A, const float* B, long long N, int C, long long HW,
                         int nhwc, hipStream_t s) {
    const long long total = N * C * HW;
    if (total <= 0) return hipSuccess;
    long long blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(bn_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, y, A, B, total, C, HW, nhwc);
    return hipGetLastError();
}

// QLinearConcat in one launch (QLinearConcat.cpp:70-236): every output row of
// `row` bytes is the concatenation of the parts' chunks; a thread writes one
// W-byte cell of a row (W divides every chunk length, the row and every
// pointer's alignment, and 16, so a cell lies in one part and wholly in its
// 16-wide body or its tail) and reads it from that part.
// One cell: output bytes [j, j + W) of row o, from part t at offset i.
template <int W>
__device__ __forceinline__ void qconcat_cell(const QConcatRows& a, long long o, long long j, int t, long long i) {
    {
        const uint8_t* src = (const uint8_t*)a.x[t] + o * a.cnt[t] + i;
        uint8_t* dst = (uint8_t*)a.y + o * a.row + j;
        constexpr int NW = W >= 4 ? W / 4 : 1;
        uint32_t w[NW];
        if constexpr (W == 16) {
            const uint4 v = *(const uint4*)src;
            w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
        } else if constexpr (W == 8) {
            const uint2 v = *(const uint2*)src;
            w[0] = v.x; w[1] = v.y;
        } else if constexpr (W == 4) {
            w[0] = *(const uint32_t*)src;
        } else {
            w[0] = *src;
        }
        if (!a.copy[t] && W >= 4 && a.dt == 0 && i < a.body[t] && __builtin_isfinite(a.rs[t])) {
            // uint8 body: clamp to [0, 255] then nearest even is one
            // v_cvt_pk_u8_f32 per byte
            const float zp = (float)a.zp[t], yz = (float)a.y_zp, rs = a.rs[t];
#pragma unroll
            for (int k = 0; k < NW; ++k) {
                uint32_t r = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    r = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_fmaf(rs, (float)((w[k] >> (8 * b)) & 0xffu) - zp, yz),
                                                       b, r);
                w[k] = r;
            }
        } else if (!a.copy[t]) {
            const bool bd = i < a.body[t];
#pragma unroll
            for (int k = 0; k < NW; ++k) {
                uint32_t r = 0;
#pragma unroll
                for (int b = 0; b < (W >= 4 ? 4 : 1); ++b)
                    r |= ((uint32_t)qconcat_elem(byte_q(w[k], b, a.dt), bd, a.rs[t], a.zp[t], a.y_zp, a.lo, a.hi) &
                          0xffu) << (8 * b);
                w[k] = r;
            }
        }
        if constexpr (W == 16) *(uint4*)dst = make_uint4(w[0], w[1], w[2], w[3]);
        else if constexpr (W == 8) *(uint2*)dst = make_uint2(w[0], w[1]);
        else if constexpr (W == 4) *(uint32_t*)dst = w[0];
        else *dst = (uint8_t)w[0];
    }
}

// a thread per cell (long rows)
template <int W>
__global__ __launch_bounds__(256) void qconcat_rows_kernel(QConcatRows a) {
    const long long cpr = a.row / W;
    const long long cells = a.outer * cpr;
    for (long long e = (long long)blockIdx.x * 256 + threadIdx.x; e < cells; e += (long long)gridDim.x * 256) {
        const long long o = e / cpr;
        const long long j = (e - o * cpr) * W;
        int t = 0;
        while (t + 1 < a.n && j >= a.off[t + 1]) ++t;
        qconcat_cell<W>(a, o, j, t, j - a.off[t]);
    }
}

// a thread per output row (short rows: an NHWC pixel's channels), walking the
// parts in order with no division per cell
template <int W>
__global__ __launch_bounds__(256) void qconcat_row_thread_kernel(QConcatRows a) {
    for (long long o = (long long)blockIdx.x * 256 + threadIdx.x; o < a.outer; o += (long long)gridDim.x * 256) {
        for (int t = 0; t < a.n; ++t)
            for (long long i = 0; i < a.cnt[t]; i += W) qconcat_cell<W>(a, o, a.off[t] + i, t, i);
    }
}

hipError_t launch_qconcat_rows(const QConcatRows& a, hipStream_t s) {
    uintptr_t al = (uintptr_t)a.y | (uintptr_t)a.row;
    for (int t = 0; t < a.n; ++t) al |= (uintptr_t)a.x[t] | (uintptr_t)a.cnt[t];
    const int W = (al & 15) == 0 ? 16 : (al & 7) == 0 ? 8 : (al & 3) == 0 ? 4 : 1;
    const long long cells = a.outer * (a.row / W);
    if (cells <= 0) return hipSuccess;
    if (a.row / W <= 8) {   // short rows: a thread per row
        long long blocks = (a.outer + 255) / 256;
        if (blocks > 65536) blocks = 65536;
        const dim3 g((unsigned)blocks), b(256);
        if (W == 16) hipLaunchKernelGGL((qconcat_row_thread_kernel<16>), g, b, 0, s, a);
        else if (W == 8) hipLaunchKernelGGL((qconcat_row_thread_kernel<8>), g, b, 0, s, a);
        else if (W == 4) hipLaunchKernelGGL((qconcat_row_thread_kernel<4>), g, b, 0, s, a);
        else hipLaunchKernelGGL((qconcat_row_thread_kernel<1>), g, b, 0, s, a);
        return hipGetLastError();
    }
    long long blocks = (cells + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    const dim3 g((unsigned)blocks), b(256);
    if (W == 16) hipLaunchKernelGGL((qconcat_rows_kernel<16>), g, b, 0, s, a);
    else if (W == 8) hipLaunchKernelGGL((qconcat_rows_kernel<8>), g, b, 0, s, a);
    else if (W == 4) hipLaunchKernelGGL((qconcat_rows_kernel<4>), g, b, 0, s, a);
    else hipLaunchKernelGGL((qconcat_rows_kernel<1>), g, b, 0, s, a);
    return hipGetLastError();
}

}  // namespace nnrh
