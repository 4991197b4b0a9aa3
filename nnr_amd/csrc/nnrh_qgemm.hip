// nnrh_qgemm.hip -- int8 GEMM / implicit-GEMM convolution on gfx950 i8 MFMA.
//
// C[m][n] = sum_k A[m][k] * B[n][k] with exact int32 accumulation
// (v_mfma_i32_16x16x64_i8), followed by the zero-point correction and one of
// NNR's requantize epilogues. This single kernel replaces the reference's
// VNNI GEMM drivers and JIT micro-kernels:
//   gemm_int8_nr48 / gemm_int8 (src/backend/x64/gemm_int8_avx512.h:1000-1106)
//   conv_int8_packed_nr48      (gemm_int8_avx512.h:1232-1518)
//   conv_int8_nhwc_direct_nr16 (src/backend/x64/conv_int8_nhwc_direct.h:35-198)
//   conv_int8_fused_gemm       (gemm_int8_avx512.h:540-895)
//   conv_int8_direct_avx512    (src/backend/x64/conv_int8_direct_avx512.h:82-210)
//   first-layer direct conv    (src/backend/x64/conv_first_layer_int8_avx512.h)
//
// Signedness: MFMA i8 is signed x signed. uint8 activations are fed as
// x' = x ^ 0x80 = x - 128 and the shift is folded into the zero-point term
//   sum (x - x_zp)(w - w_zp) = sum x'w' - alpha*colsum(w') - beta*rowsum(x - x_zp)
// with alpha = x_zp - 128 (0 shift for int8), beta = w_zp - (128 for uint8 w).
// Everything is int32 arithmetic modulo 2^32, so the result is bit-identical
// to the reference's accumulators whatever the tiling.
//
// Block: 256 threads = 4 waves; each wave owns a 64x64 tile of C as 4x4
// MFMA 16x16 tiles. K advances 64 per step through an LDS double buffer.
// The MFMA "A" operand is the weight tile (rows = output channels) and the
// "B" operand the activation tile (columns = output pixels), so lane l holds
// D[4*(l/16)+r][l%16]. Packed weights permute rows inside each 64-column
// group (packed_row_of_col) so that each lane ends with 16 consecutive output
// channels of one pixel: one 16-byte store per lane and MFMA tile row.
#include "nnrh_internal.h"
#include "nnrh_rq.h"

namespace nnrh {

typedef int v4i __attribute__((ext_vector_type(4)));

// byte offset of 16-byte chunk c of tile row `row` in LDS (XOR swizzle keeps
// the ds_read_b128 fragment reads and the 16-byte stores conflict-free)
__device__ __forceinline__ int lds_off(int row, int c) {
    return row * 64 + ((c ^ ((row >> 1) & 3)) << 4);
}

template <int VEC>
struct SubLoad;
template <> struct SubLoad<8> {
    __device__ static void ld(const uint8_t* p, uint32_t* w) {
        uint2 v = *(const uint2*)p; w[0] = v.x; w[1] = v.y;
    }
};
template <> struct SubLoad<4> {
    __device__ static void ld(const uint8_t* p, uint32_t* w) { w[0] = *(const uint32_t*)p; }
};
template <> struct SubLoad<16> {
    __device__ static void ld(const uint8_t* p, uint32_t* w) {
        uint4 v = *(const uint4*)p; w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    }
};

// byte-granular gather for channel counts / K that are not multiples of 4
template <int AMODE>
__device__ __forceinline__ void load_bytes(const GemmArgs& g, const uint8_t* abase,
                                           long long base, int ih0, int iw0, bool ok, int kk,
                                           uint32_t* w) {
    uint32_t padb = (uint32_t)(g.pad_byte & 0xff);
#pragma unroll
    for (int q = 0; q < 4; ++q) w[q] = 0u;
#pragma unroll
    for (int sb = 0; sb < 16; ++sb) {
        int k = kk + sb;
        uint32_t b = 0u;
        if (ok && k < g.K) {
            if constexpr (AMODE == A_DENSE) {
                b = abase[base + k];
            } else {
                int kp = k / g.C;
                int ic = k - kp * g.C;
                int kh = kp / g.kW;
                int kw = kp - kh * g.kW;
                int ih = ih0 + kh * g.dH;
                int iw = iw0 + kw * g.dW;
                if ((unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W)
                    b = abase[base + (long long)(ih * g.W + iw) * g.Cs + ic];
                else
                    b = padb;
            }
        }
        w[sb >> 2] |= b << (8 * (sb & 3));
    }
}

template <int BM, int BN, int VEC, int AMODE>
__global__ __launch_bounds__(256, 2) void qgemm_kernel(GemmArgs g) {
    constexpr int WAVES_N = BN / 64;
    constexpr int WAVES_M = BM / 64;
    static_assert(WAVES_N * WAVES_M == 4, "4 waves of 64x64");
    constexpr int A_CH = BM / 64;   // 16-byte A chunks per thread per K step
    constexpr int B_CH = BN / 64;

    __shared__ __attribute__((aligned(16))) uint8_t lds_a[2][BM * 64];
    __shared__ __attribute__((aligned(16))) uint8_t lds_b[2][BN * 64];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;

    // ---- persistent tiles, XCD-aware: blocks on XCD x (blockIdx % 8 == x)
    // walk the x-th contiguous eighth of the tile list (m-major), so the N
    // tiles of one A row block meet in the same L2.
    const int nbn = (g.N + BN - 1) / BN;
    const int nbm = (g.M + BM - 1) / BM;
    const int total = nbm * nbn;
    const int G = gridDim.x;
    const int z = blockIdx.z;
    int t_cur, t_end, t_step;
    if (G >= 8 && (G & 7) == 0) {
        const int per = G >> 3, xcd = blockIdx.x & 7, local = blockIdx.x >> 3;
        const int chunk = (total + 7) >> 3;
        t_cur = xcd * chunk + local;
        t_end = min(total, (xcd + 1) * chunk);
        t_step = per;
    } else {
        t_cur = blockIdx.x;
        t_end = total;
        t_step = G;
    }
    if (t_cur >= t_end) return;

    const uint8_t* abase = g.a + (long long)z * g.a_bstride;
    const int8_t* bbase = g.b + (long long)z * g.b_bstride;
    const uint32_t xmask = (uint32_t)g.a_xor * 0x01010101u;
    const int c16 = tid & 3;          // this thread's 16-byte chunk in a row
    const int sp_out = g.oH * g.oW;

    // ---- per-thread A rows of the tile being loaded
    int a_row[A_CH];
    bool a_ok[A_CH];
    long long a_base[A_CH];   // dense: row offset; conv: image offset
    int a_ih0[A_CH], a_iw0[A_CH];
    int ld_m0 = 0, ld_n0 = 0;
    int kc_ic = 0, kc_kh = 0, kc_kw = 0;   // conv K decode of k = k0 + c16*16 (VEC 16)
    auto setup_tile = [&](int t) {
        ld_m0 = (t / nbn) * BM;
        ld_n0 = (t % nbn) * BN;
#pragma unroll
        for (int j = 0; j < A_CH; ++j) {
            a_row[j] = (tid >> 2) + 64 * j;
            int m = ld_m0 + a_row[j];
            a_ok[j] = m < g.M;
            if constexpr (AMODE == A_DENSE) {
                a_base[j] = (long long)m * g.lda;
                a_ih0[j] = 0; a_iw0[j] = 0;
            } else {
                int mm = a_ok[j] ? m : 0;
                int img = mm / sp_out, s = mm - img * sp_out;
                int oh = s / g.oW, ow = s - oh * g.oW;
                a_base[j] = (long long)img * g.H * g.W * g.Cs;
                a_ih0[j] = oh * g.sH - g.pad_t;
                a_iw0[j] = ow * g.sW - g.pad_l;
            }
        }
        if constexpr (AMODE == A_CONV && VEC == 16) {
            int k = c16 * 16;
            int kp = k / g.C;
            kc_ic = k - kp * g.C;
            kc_kh = kp / g.kW;
            kc_kw = kp - kc_kh * g.kW;
        }
    };
    const uint32_t padw = (uint32_t)(g.pad_byte & 0xff) * 0x01010101u;

    v4i ra[A_CH], rb[B_CH];

    auto load_tiles = [&](int k0) {
        // ---- A
#pragma unroll
        for (int j = 0; j < A_CH; ++j) {
            uint32_t w[4] = {0u, 0u, 0u, 0u};
            const int kk = k0 + c16 * 16;
            if constexpr (AMODE == A_CONV4) {
                // first-layer layout: K = (kh, kw < kWp, c < 4); a 16-byte chunk
                // holds 4 consecutive taps of one input row (4 channels each)
                const int cpr = g.kWp >> 2;
                const int q = kk >> 4;
                const int kh = q / cpr;
                const int kw0 = (q - kh * cpr) << 2;
                if (a_ok[j] && kh < g.kH) {
                    const int ih = a_ih0[j] + kh;
                    if ((unsigned)ih < (unsigned)g.H) {
                        const uint8_t* rowp = abase + a_base[j] + (long long)ih * g.W * 4;
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            const int iw = a_iw0[j] + kw0 + t;
                            w[t] = ((unsigned)iw < (unsigned)g.W) ? *(const uint32_t*)(rowp + (long long)iw * 4)
                                                                  : padw;
                        }
                    } else {
                        w[0] = w[1] = w[2] = w[3] = padw;
                    }
                }
            } else if constexpr (VEC == 1) {
                load_bytes<AMODE>(g, abase, a_base[j], a_ih0[j], a_iw0[j], a_ok[j], kk, w);
            } else if constexpr (AMODE == A_DENSE) {
                if (a_ok[j]) {
                    if constexpr (VEC == 16) {
                        if (kk < g.K) {
                            v4i v = *(const v4i*)(abase + a_base[j] + kk);
                            w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
                        }
                    } else {
#pragma unroll
                        for (int sb = 0; sb < 16 / VEC; ++sb) {
                            int k = kk + sb * VEC;
                            if (k < g.K) SubLoad<VEC>::ld(abase + a_base[j] + k, &w[sb * VEC / 4]);
                        }
                    }
                }
            } else {
                if constexpr (VEC == 16) {
                    if (a_ok[j] && kc_kh < g.kH) {
                        int ih = a_ih0[j] + kc_kh * g.dH;
                        int iw = a_iw0[j] + kc_kw * g.dW;
                        if ((unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W) {
                            v4i v = *(const v4i*)(abase + a_base[j] +
                                                  ((long long)(ih * g.W + iw) * g.Cs + kc_ic));
                            w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
                        } else {
                            w[0] = w[1] = w[2] = w[3] = padw;
                        }
                    }
                } else {
#pragma unroll
                    for (int sb = 0; sb < 16 / VEC; ++sb) {
                        int k = kk + sb * VEC;
                        if (a_ok[j] && k < g.K) {
                            int kp = k / g.C;
                            int ic = k - kp * g.C;
                            int kh = kp / g.kW;
                            int kw = kp - kh * g.kW;
                            int ih = a_ih0[j] + kh * g.dH;
                            int iw = a_iw0[j] + kw * g.dW;
                            if ((unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W) {
                                SubLoad<VEC>::ld(abase + a_base[j] +
                                                 ((long long)(ih * g.W + iw) * g.Cs + ic),
                                                 &w[sb * VEC / 4]);
                            } else {
#pragma unroll
                                for (int q = 0; q < VEC / 4; ++q) w[sb * VEC / 4 + q] = padw;
                            }
                        }
                    }
                }
            }
            ra[j].x = (int)(w[0] ^ xmask);
            ra[j].y = (int)(w[1] ^ xmask);
            ra[j].z = (int)(w[2] ^ xmask);
            ra[j].w = (int)(w[3] ^ xmask);
        }
        // ---- B (packed [Np][Kp], always in bounds below Np)
#pragma unroll
        for (int j = 0; j < B_CH; ++j) {
            int n = ld_n0 + (tid >> 2) + 64 * j;
            if (n < g.Np) {
                rb[j] = *(const v4i*)(bbase + (long long)n * g.Kp + k0 + c16 * 16);
            } else {
                rb[j] = v4i{0, 0, 0, 0};
            }
        }
    };
    auto advance_k = [&]() {
        if constexpr (AMODE == A_CONV && VEC == 16) {
            kc_ic += 64;
            while (kc_ic >= g.C) {
                kc_ic -= g.C;
                if (++kc_kw == g.kW) { kc_kw = 0; ++kc_kh; }
            }
        }
    };
    auto store_tiles = [&](int buf) {
#pragma unroll
        for (int j = 0; j < A_CH; ++j)
            *(v4i*)(&lds_a[buf][lds_off(a_row[j], c16)]) = ra[j];
#pragma unroll
        for (int j = 0; j < B_CH; ++j)
            *(v4i*)(&lds_b[buf][lds_off((tid >> 2) + 64 * j, c16)]) = rb[j];
    };

    v4i acc[4][4];
    const int nk = g.Kp >> 6;
    const int frow = lane & 15;
    const int fchunk = lane >> 4;
    auto epilogue = [&](const int m0, const int n0) {
        // ---- epilogue: lane owns columns nb..nb+15 of rows m0 + wm*64 + 16*tm + frow.
        // Per-column constants are padded to Np, so the vector loads need no
        // guard. c0[n] folds the zero-point column term (and, for RQ-B, the int32
        // bias): v = acc' + c0[n] - beta*rowsum[m] is the reference's value.
        const int nb = n0 + wn * 64 + 16 * fchunk;
        if (nb >= g.N) return;
        const long long po = (long long)z * g.param_bstride;
        int alpha = g.alpha;
        if (g.alpha_zp_dev) {
            int zp = g.a_xor ? (int)*(const uint8_t*)g.alpha_zp_dev
                             : (int)*(const int8_t*)g.alpha_zp_dev;
            alpha = zp - g.a_sub;
        }
        float cm = g.cm;
        if (g.epi == EPI_RQD && g.cm_a_scale_dev) {
            float t1 = *g.cm_a_scale_dev * g.cm_b;
            cm = t1 / g.cm_y;
        }
        const int sp = g.oH * g.oW;
        const bool full16 = (nb + 16 <= g.N);
        // per-row terms
        int rs[4];
        bool tail[4];
        bool any_tail = false;
    #pragma unroll
        for (int tm = 0; tm < 4; ++tm) {
            const int m = m0 + wm * 64 + tm * 16 + frow;
            rs[tm] = (g.rowsum && m < g.M) ? g.rowsum[(long long)z * g.rowsum_bstride + m] : 0;
            bool tl = false;
            if (g.tail != TAIL_NONE && m < g.M) {
                int s = m % sp;
                if (g.tail == TAIL_SPATIAL) {
                    tl = s >= sp - sp % 16;
                } else if (g.tail == TAIL_OW) {
                    int ow = s % g.oW;
                    tl = ow >= g.oW - g.oW % 16;
                } else {
                    int oh = s / g.oW;
                    int oh0 = (oh / g.tile_h) * g.tile_h;
                    int th = g.oH - oh0 < g.tile_h ? g.oH - oh0 : g.tile_h;
                    int tsp = th * g.oW;
                    int ts = s - oh0 * g.oW;
                    tl = ts >= tsp - tsp % 16;
                }
            }
            tail[tm] = tl;
            any_tail |= tl;
        }
        const bool use_rows = g.rowsum != nullptr;
        // slow (reference-expression) path: scalar tails and RQ-B' columns
        const bool slow = any_tail || (g.epi == EPI_RQB && nb + 16 > g.bprime_from);
        uint32_t packed[4][4];
    #pragma unroll
        for (int tn = 0; tn < 4; ++tn) {
            const int n4 = nb + 4 * tn;
            int cc[4];
            if (g.c0 && !g.alpha_zp_dev) {
                int4 c = *(const int4*)(g.c0 + po + n4);
                cc[0] = c.x; cc[1] = c.y; cc[2] = c.z; cc[3] = c.w;
            } else {
    #pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int32_t cs_ = g.colsum ? g.colsum[po + n4 + r] : 0;
                    int32_t b_ = (g.epi == EPI_RQB && g.bias) ? g.bias[po + n4 + r] : 0;
                    cc[r] = wrap_add(b_, -wrap_mul(alpha, cs_));
                }
            }
            int bc[4] = {g.beta, g.beta, g.beta, g.beta};
            if (use_rows && g.beta_col) {
                int4 b4 = *(const int4*)(g.beta_col + po + n4);
                bc[0] = b4.x; bc[1] = b4.y; bc[2] = b4.z; bc[3] = b4.w;
            }
            float p0[4] = {0.f, 0.f, 0.f, 0.f}, p1[4] = {0.f, 0.f, 0.f, 0.f};
            if (g.epi == EPI_RQB) {
                float4 s4 = *(const float4*)(g.os + po + n4);
                p0[0] = s4.x; p0[1] = s4.y; p0[2] = s4.z; p0[3] = s4.w;
            } else if (g.epi == EPI_RQA || g.epi == EPI_RQC) {
                float4 s4 = *(const float4*)(g.cs + po + n4);
                float4 b4 = *(const float4*)(g.bf + po + n4);
                p0[0] = s4.x; p0[1] = s4.y; p0[2] = s4.z; p0[3] = s4.w;
                p1[0] = b4.x; p1[1] = b4.y; p1[2] = b4.z; p1[3] = b4.w;
            }
    #pragma unroll
            for (int tm = 0; tm < 4; ++tm) {
                int32_t v[4] = {acc[tm][tn].x, acc[tm][tn].y, acc[tm][tn].z, acc[tm][tn].w};
    #pragma unroll
                for (int r = 0; r < 4; ++r) {
                    v[r] = wrap_add(v[r], cc[r]);
                    if (use_rows) v[r] = wrap_add(v[r], -wrap_mul(bc[r], rs[tm]));
                }
                if (g.epi == EPI_I32) {
                    packed[tm][tn] = 0;
                    acc[tm][tn] = v4i{v[0], v[1], v[2], v[3]};
                    continue;
                }
                uint32_t w = 0;
                if (!slow) {
    #pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        uint32_t b;
                        if (g.epi == EPI_RQB) b = rqb_fast(v[r], p0[r], g.y_zp, g.lo, g.hi);
                        else if (g.epi == EPI_RQA) b = rqa_fast(v[r], p0[r], p1[r], g.inv_y, g.y_zp, g.L, g.hi);
                        else if (g.epi == EPI_RQC) b = rqc_fast(v[r], p0[r], p1[r], g.inv_y, g.y_zp, g.L, g.hi);
                        else b = rqd_fast(v[r], cm, g.y_zp, g.lo, g.hi);
                        w |= (b & 0xffu) << (8 * r);
                    }
                } else {
    #pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        int q;
                        if (g.epi == EPI_RQB) {
                            q = (n4 + r >= g.bprime_from) ? rq_b_roundf(v[r], p0[r], g.y_zp, g.lo, g.hi)
                                                          : rq_b(v[r], p0[r], g.y_zp, g.lo, g.hi);
                        } else if (g.epi == EPI_RQA) {
                            q = tail[tm] ? rq_a_tail(v[r], p0[r], p1[r], g.inv_y, g.y_zp, g.L, g.hi)
                                         : rq_a(v[r], p0[r], p1[r], g.inv_y, g.y_zp, g.L, g.hi);
                        } else if (g.epi == EPI_RQC) {
                            q = tail[tm] ? rq_a_tail(v[r], p0[r], p1[r], g.inv_y, g.y_zp, g.L, g.hi)
                                         : rq_c(v[r], p0[r], p1[r], g.inv_y, g.y_zp, g.L, g.hi);
                        } else {
                            q = rq_d(v[r], cm, g.y_zp, g.lo, g.hi);
                        }
                        w |= (uint32_t)(q & 0xff) << (8 * r);
                    }
                }
                packed[tm][tn] = w;
            }
        }
    #pragma unroll
        for (int tm = 0; tm < 4; ++tm) {
            const int m = m0 + wm * 64 + tm * 16 + frow;
            if (m >= g.M) continue;
            if (g.epi == EPI_I32) {
                int32_t* yrow = (int32_t*)g.y + (long long)z * g.y_bstride + (long long)m * g.ldy + nb;
                if (full16 && ((((uintptr_t)yrow) & 15) == 0)) {
    #pragma unroll
                    for (int tn = 0; tn < 4; ++tn) *(v4i*)(yrow + 4 * tn) = acc[tm][tn];
                } else {
    #pragma unroll
                    for (int tn = 0; tn < 4; ++tn) {
                        int32_t vv[4] = {acc[tm][tn].x, acc[tm][tn].y, acc[tm][tn].z, acc[tm][tn].w};
    #pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (nb + 4 * tn + r < g.N) yrow[4 * tn + r] = vv[r];
                    }
                }
                continue;
            }
            if (g.y_nchw) {
                uint8_t* yb = (uint8_t*)g.y + (long long)z * g.y_bstride;
                int img = m / sp, s = m - img * sp;
    #pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (nb + i < g.N)
                        yb[((long long)img * g.ldy + nb + i) * sp + s] = (uint8_t)(packed[tm][i >> 2] >> (8 * (i & 3)));
            } else {
                uint8_t* yrow = (uint8_t*)g.y + (long long)z * g.y_bstride + (long long)m * g.ldy + nb;
                if (full16 && ((((uintptr_t)yrow) & 15) == 0)) {
                    *(v4i*)yrow = v4i{(int)packed[tm][0], (int)packed[tm][1], (int)packed[tm][2], (int)packed[tm][3]};
                } else {
    #pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (nb + i < g.N) yrow[i] = (uint8_t)(packed[tm][i >> 2] >> (8 * (i & 3)));
                }
            }
        }
    };

    setup_tile(t_cur);
    load_tiles(0);
    advance_k();
    for (;;) {
        const int m0 = ld_m0, n0 = ld_n0;
        const int t_next = t_cur + t_step;
        const bool has_next = t_next < t_end;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = v4i{0, 0, 0, 0};
        store_tiles(0);
        __syncthreads();
        for (int kt = 0; kt < nk; ++kt) {
            const int cur = kt & 1;
            if (kt + 1 < nk) {
                load_tiles((kt + 1) << 6);
                advance_k();
            } else if (has_next) {
                // first K step of the next tile: in flight during the epilogue
                setup_tile(t_next);
                load_tiles(0);
                advance_k();
            }
            v4i xf[4], wf[4];
#pragma unroll
            for (int tm = 0; tm < 4; ++tm)
                xf[tm] = *(const v4i*)(&lds_a[cur][lds_off(wm * 64 + tm * 16 + frow, fchunk)]);
#pragma unroll
            for (int tn = 0; tn < 4; ++tn)
                wf[tn] = *(const v4i*)(&lds_b[cur][lds_off(wn * 64 + tn * 16 + frow, fchunk)]);
#pragma unroll
            for (int tm = 0; tm < 4; ++tm)
#pragma unroll
                for (int tn = 0; tn < 4; ++tn)
                    acc[tm][tn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[tn], xf[tm], acc[tm][tn], 0, 0, 0);
            if (kt + 1 < nk) store_tiles(cur ^ 1);
            __syncthreads();
        }
        epilogue(m0, n0);
        if (!has_next) break;
        t_cur = t_next;
    }
}

template <int BM, int BN, int VEC, int AMODE>
static hipError_t launch_one(const GemmArgs& g, int batch, hipStream_t s) {
    // one tile per block: this kernel keeps its next-tile prefetch in VGPRs,
    // and hardware block dispatch overlaps tiles better than a persistent loop
    const int tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
    auto kern = qgemm_kernel<BM, BN, VEC, AMODE>;
    hipLaunchKernelGGL(kern, dim3(tiles, 1, batch), dim3(256), 0, s, g);
    return hipGetLastError();
}

template <int BM, int BN, int AMODE>
static hipError_t launch_vec(const GemmArgs& g, int batch, int vec, hipStream_t s) {
    if (g.kWp > 0) return launch_one<BM, BN, 4, A_CONV4>(g, batch, s);
    switch (vec) {
    case 16: return launch_one<BM, BN, 16, AMODE>(g, batch, s);
    case 8: return launch_one<BM, BN, 8, AMODE>(g, batch, s);
    case 4: return launch_one<BM, BN, 4, AMODE>(g, batch, s);
    case 1: return launch_one<BM, BN, 1, AMODE>(g, batch, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_qgemm(const GemmArgs& g, int batch, int tile, int vec, hipStream_t s) {
    if (g.M <= 0 || g.N <= 0 || batch <= 0) return hipSuccess;
    if (g.Kp <= 0 || (g.Kp & 63) || g.Kp < g.K) return hipErrorInvalidValue;
    if (g.a == nullptr || g.b == nullptr || g.y == nullptr) return hipErrorInvalidValue;
    const bool conv = (g.H > 0);
    if (qgemm_direct_eligible(g, batch)) return launch_qgemm_direct(g, s);
    if (qgemm_dma_eligible(g, vec)) return launch_qgemm_dma(g, batch, tile, s);
    if (g.add_other || g.dq_bias) return hipErrorNotSupported;   // fusions: pipelined kernel only
    prof_count("variant:qgemm_reg");
    switch (tile) {
    case TILE_128x128:
    case TILE_256x128:
        return conv ? launch_vec<128, 128, A_CONV>(g, batch, vec, s)
                    : launch_vec<128, 128, A_DENSE>(g, batch, vec, s);
    case TILE_256x64:
        return conv ? launch_vec<256, 64, A_CONV>(g, batch, vec, s)
                    : launch_vec<256, 64, A_DENSE>(g, batch, vec, s);
    case TILE_64x256:
        return conv ? launch_vec<64, 256, A_CONV>(g, batch, vec, s)
                    : launch_vec<64, 256, A_DENSE>(g, batch, vec, s);
    default:
        return hipErrorInvalidValue;
    }
}

}  // namespace nnrh
