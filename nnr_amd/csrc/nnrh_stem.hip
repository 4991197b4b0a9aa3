// nnrh_stem.hip -- the first convolution of an image network in one kernel:
// input quantization (or the raw uint8 image), implicit im2col, i8 MFMA and
// the RQ-C epilogue of NNR's first-layer driver.
//
// The reference runs QuantizeLinear over the fp32 image (QuantizeLinear.cpp:
// 15-301), then exec_first_layer_int8 (QLinearConv.cpp:665-700) over the
// uint8 NCHW tensor with 3-4 input channels, requantizing with RQ-C
// (conv_first_layer_int8_avx512.h:262-273). Here one block walks a strip of
// output rows of one image:
//  * the input rows it needs are read from HBM once (fp32 NCHW or uint8
//    NCHW), quantized with the QuantizeLinear body / tail expressions of the
//    whole tensor, and written into an LDS ring as zero-point padded
//    4-channel pixels (one dword: channels 0..C-1, then the zero point),
//    already shifted to int8 (x ^ 0x80);
//  * the rows of the next group of output rows load while the current group
//    runs its MFMAs, so the image streams in once at HBM rate;
//  * the weights stay in registers ([Np = 64][Kp] packed as for the GEMM
//    kernels, K order (kh, kw < kWp, c < 4)), each lane holding its 16-byte
//    K chunks of its 16 output channels;
//  * every 16 output pixels take Kp / 64 x 4 MFMAs 16x16x64 and go straight
//    through the epilogue: RQ-C, 16 consecutive channels per lane, 16-byte
//    stores into the NHWC uint8 output.
// The accumulators start at c0[n] = -(x_zp - 128) * colsum[n], so
// acc = sum (x - x_zp) w exactly, as in the GEMM kernels.
//
// With the MaxPool after the conv fused (POOL; 3x3, stride 2, padding 1 on
// the uint8 NHWC conv output, MaxPool.cpp / pool_x64.h:396-436), a block
// walks a strip of pooled rows [pa, pb): it computes conv row 2 pa - 1
// first, then conv rows in groups of 4 from 2 pa, writes them into an LDS
// tile of 5 conv rows (the group's 4 and the previous group's last; a zero
// column either side) instead of HBM, and after each group writes the two
// pooled rows it completes. The pooled
// bytes are the max of the conv's requantized bytes, exactly as when the two
// operators run apart; out-of-image taps are skipped (a uint8 max with the
// zero columns changes nothing).
#include "nnrh_internal.h"
#include "nnrh_rq.h"

#include <type_traits>

namespace nnrh {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int STEM_MGW = 7;    // 16-pixel groups per wave per row group (x 4 waves)
constexpr int STEM_RING_DW = 10240;    // LDS ring: dwords (staged pixels, mapped twice)
constexpr int STEM_STAGE_B = 36 * 1024; // LDS staging: raw input bytes of one row group's span
constexpr int STEM_DMA = 2;    // 16-byte DMA chunks one thread issues per input row (x 256 threads)
// with the MaxPool fused: a ring of exactly one group's span, staging for
// one group's new rows, the 5-row conv tile; 81,904 bytes, two blocks per CU
constexpr int STEM_P_RING_DW = 5980;
constexpr int STEM_P_STAGE_B = 21504;
constexpr int STEM_P_TILE_B = 36480;
#define LDS_AS __attribute__((address_space(3)))

__device__ __forceinline__ uint32_t stem_quant(float xv, bool body, const StemArgs& a) {
    int q;
    if (body) {
        // QuantizeLinear's 16-wide body: rint(x * (1/s)) + zp, clamped in float
        float v = xv * a.q_inv;
        v = __builtin_rintf(v) + (float)a.q_zp;
        v = clamp_minmax(v, 0.0f, 255.0f);
        q = (int)v;
    } else {
        // scalar tail: rint(x / s) through the x86 convert, + zp, clamped
        q = clampi(wrap_add(x86_f2i(__builtin_rintf(xv / a.q_scale)), a.q_zp), 0, 255);
    }
    return (uint32_t)q;
}

// running byte-wise max of 4 uint8 lanes, kept as the even bytes (lo) and
// the odd bytes (hi) in 16-bit lanes: two packed max instructions a dword
typedef unsigned short stem_us2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void bytemax_acc(uint32_t x, uint32_t& lo, uint32_t& hi) {
    const stem_us2 xl = __builtin_bit_cast(stem_us2, x & 0x00ff00ffu);
    const stem_us2 xh = __builtin_bit_cast(stem_us2, (x >> 8) & 0x00ff00ffu);
    lo = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(stem_us2, lo), xl));
    hi = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(stem_us2, hi), xh));
}

// every wave's LDS writes done, then a plain s_barrier: __syncthreads'
// workgroup fence would also wait for this wave's output stores, which the
// kernel leaves in flight (the memory clobber keeps the compiler from moving
// LDS accesses across)
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
}

}  // namespace

// CC: input channels (3 or 4); KS: MFMA K-steps (Kp / 64); POOL: the 3x3 /
// stride 2 / padding 1 MaxPool after the conv fused (strip = pooled rows)
// NT: 16-column MFMA blocks computed (OC = 16 NT, or 64 with NT = 4): lane
// (fch, frow) holds output channels 4 NT fch .. 4 NT fch + 4 NT - 1 of its
// pixel, so a 16- or 32-channel layer issues NT MFMAs a K-step and its
// epilogue touches only real channels
template <bool F32, int CC, int KS, bool POOL, int NT = 4>
__global__ __launch_bounds__(256, 2) void stem_conv_kernel(StemArgs a) {
    static_assert(NT == 4 || NT == 2 || NT == 1, "16, 32 or 64 output channels");
    static_assert(!POOL || NT == 4, "the fused MaxPool takes 64 channels");
    // separate static arrays: the compiler then tells the ring's reads from
    // the staging area's in-flight DMA writes and waits for neither
    __shared__ __attribute__((aligned(16))) uint32_t ring[POOL ? STEM_P_RING_DW : STEM_RING_DW];   // WR rows x L
    __shared__ __attribute__((aligned(16))) uint8_t stage[POOL ? STEM_P_STAGE_B : STEM_STAGE_B];   // raw rows
    __shared__ __attribute__((aligned(16))) uint8_t tile[POOL ? STEM_P_TILE_B : 16];   // 5 conv rows
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int frow = lane & 15, fch = lane >> 4;
    const int n = blockIdx.y;
    // conv rows of the block's groups [oh_begin, oh_end); POOL: pooled rows
    // [pa, pb), conv rows 2 pa - 1 (computed first, alone) to 2 pb - 1
    int oh_begin, oh_end, pa = 0, pb = 0;
    if constexpr (POOL) {
        pa = blockIdx.x * a.strip;
        pb = min(a.pH, pa + a.strip);
        if (pa >= pb) return;
        oh_begin = 2 * pa;
        oh_end = min(a.oH, 2 * pb);
    } else {
        oh_begin = blockIdx.x * a.strip;
        oh_end = min(a.oH, oh_begin + a.strip);
        if (oh_begin >= oh_end) return;
    }
    const long long HW = (long long)a.H * a.W;
    const long long img = (long long)n * a.C * HW;

    // ---- weights (B fragments) and per-column constants in registers
    // MFMA block tn's row frow is output channel (frow / 4) * 4 NT + 4 tn +
    // frow % 4 (with NT = 4 the packed weight row tn * 16 + frow itself)
    v4i wf[KS][NT];   // [K-step][tn]
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int tn = 0; tn < NT; ++tn) {
            const int row = packed_row_of_col((frow >> 2) * 4 * NT + 4 * tn + (frow & 3));
            wf[ks][tn] = *(const v4i*)(a.w + (long long)row * a.Kp + ks * 64 + fch * 16);
        }
    // per-column constants of this lane's 4 NT columns
    v4i c0v[NT], csv[NT], bfv[NT];
#pragma unroll
    for (int tn = 0; tn < NT; ++tn) {
        c0v[tn] = *(const v4i*)(a.c0 + 4 * NT * fch + 4 * tn);
        csv[tn] = *(const v4i*)(a.cs + 4 * NT * fch + 4 * tn);
        bfv[tn] = *(const v4i*)(a.bf + 4 * NT * fch + 4 * tn);
    }
    // the weights have landed before the row groups start: the compiler
    // then has no load outstanding from outside the pixel-group loop that
    // the loop uses, and keeps the row prefetch in flight across it
    __builtin_amdgcn_s_waitcnt(0);

    // ---- index maps fixed for the whole strip (no divisions in the loop)
    constexpr int ES = F32 ? 4 : 1;          // input element bytes
    constexpr int CE = 16 / ES;              // elements per 16-byte DMA chunk
    const int row_chunks = CC * (a.W / CE);  // DMA chunks of one padded row (all channels)
    const int row_bytes = CC * a.W * ES;     // staged bytes of one padded row
    // this thread's DMA chunks of a row (k = 0, 1): element offset c * H * W
    // + w within the image, -1 past the row
    int d_off[STEM_DMA];
#pragma unroll
    for (int k = 0; k < STEM_DMA; ++k) {
        const int u = tid + 256 * k;
        const int c = u / (a.W / CE), w4 = u - c * (a.W / CE);
        d_off[k] = u < row_chunks ? (int)(c * HW) + w4 * CE : -1;
    }
    // this lane's pixel p = r * oW + ow of 16-pixel group i (output pixel
    // oh0 * oW + p of the image), as a dword offset in the ring from the
    // group's first row: (r * sH) * L + ow * sW
    int m_off[STEM_MGW];
    // POOL: the pixel's LDS tile offset from its row's slot, (ow + 1) * OC +
    // 16 fch (below 2^24), with its row in the group, r, in bits 24..
    int m_tile[POOL ? STEM_MGW : 1];
#pragma unroll
    for (int i = 0; i < STEM_MGW; ++i) {
        const int p = (wave + 4 * i) * 16 + frow;
        const int r = p / a.oW, ow = p - (p / a.oW) * a.oW;
        m_off[i] = r * a.sH * a.L + ow * a.sW;
        if constexpr (POOL) m_tile[i] = ((ow + 1) * a.OC + 16 * fch) | (r << 24);
    }
    // the image's output (NHWC, OC bytes a pixel; offsets within it fit 32 bits)
    uint8_t* const y_img = a.y + (long long)n * a.oH * a.oW * a.OC;
    // K chunk of K-step ks: kernel row (clamped into the kernel: past it the
    // weights are zero) and first tap
    int k_kh[KS], k_kw[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int q = ks * 4 + fch;
        const int kh = q / a.cpr;
        k_kh[ks] = min(kh, a.kH - 1);
        k_kw[ks] = (q - kh * a.cpr) * 4;
    }
    // QuantizeLinear's scalar tail lies in the last image's last channel
    const bool all_body = img + (long long)CC * HW <= a.qbody;

    const uint8_t* xb = (const uint8_t*)a.x + img * ES;

    // raw padded rows [r0, r0 + nr) into the staging area (rows outside the
    // image load row 0: never read)
    auto dma_rows = [&](int r0, int nr) {
        for (int r = 0; r < nr; ++r) {
            const int ih = r0 + r - a.pad_t;
            const long long rowe = (long long)((unsigned)ih < (unsigned)a.H ? ih : 0) * a.W;
#pragma unroll
            for (int k = 0; k < STEM_DMA; ++k) {
                if (k * 256 + wave * 64 >= row_chunks) break;
                if (d_off[k] >= 0)
                    __builtin_amdgcn_global_load_lds(xb + (rowe + d_off[k]) * ES,
                                                     (LDS_AS void*)(stage + r * row_bytes + (k * 256 + wave * 64) * 16),
                                                     16, 0, 0);
            }
        }
    };
    // staged rows [r0, r0 + nr) quantized into their ring slots, one thread
    // per padded column; slot0 = slot of row r0. Bytes go in with
    // v_cvt_pk_u8_f32, exact for the integral values in [0, 255] QuantizeLinear
    // produces; the pad channels / pixels are the zero point; then ^ 0x80.
    uint32_t fill4 = 0;
#pragma unroll
    for (int c = CC; c < 4; ++c) fill4 |= a.fill << (8 * c);
    const uint32_t fill_all = a.fill * 0x01010101u;
    // (BODY: every element of the block's image takes QuantizeLinear's body
    // expression, fixed at compile time like the epilogue's variants)
    auto quantize_rows = [&](int r0, int nr, int slot0, auto body_t) {
        constexpr bool BODY = decltype(body_t)::value;
        for (int r = 0; r < nr; ++r) {
            const int ih = r0 + r - a.pad_t;
            const bool row_in = (unsigned)ih < (unsigned)a.H;
            int slot = slot0 + r;
            slot -= slot >= a.WR ? a.WR : 0;
            const uint8_t* srow = stage + r * row_bytes;
            for (int pc = tid; pc < a.L; pc += 256) {
                const int iw = pc - a.pad_l;
                uint32_t w = fill_all;
                if (row_in && (unsigned)iw < (unsigned)a.W) {
                    if constexpr (F32) {
                        const float* sp = (const float*)srow + iw;
                        if constexpr (BODY) {
                            w = fill4;
#pragma unroll
                            for (int c = 0; c < CC; ++c) {
                                // QuantizeLinear's 16-wide body
                                float v = __builtin_rintf(sp[c * a.W] * a.q_inv) + (float)a.q_zp;
                                v = clamp_minmax(v, 0.0f, 255.0f);
                                w = __builtin_amdgcn_cvt_pk_u8_f32(v, c, w);
                            }
                        } else {
                            w = fill4;
#pragma unroll
                            for (int c = 0; c < CC; ++c) {
                                const long long idx = img + (long long)c * HW + (long long)ih * a.W + iw;
                                w |= stem_quant(sp[c * a.W], idx < a.qbody, a) << (8 * c);
                            }
                        }
                    } else {
                        w = fill4;
#pragma unroll
                        for (int c = 0; c < CC; ++c) w |= (uint32_t)srow[c * a.W + iw] << (8 * c);
                    }
                }
                // the ring is mapped twice (rows slot and slot + WR): a
                // group's rows are then contiguous from its first slot
                ring[slot * a.L + pc] = w ^ 0x80808080u;
                ring[(slot + a.WR) * a.L + pc] = w ^ 0x80808080u;
            }
        }
    };

    // ---- the strip's first rows, from ring slot 0: a group's span (or,
    // POOL, the kH rows of the lone conv row 2 pa - 1)
    const int span = (a.R - 1) * a.sH + a.kH;   // padded input rows of one row group
    const int step = a.R * a.sH;                // new rows per group
    auto quantize = [&](int r0, int nr, int slot0) {
        if (!F32 || all_body) quantize_rows(r0, nr, slot0, std::true_type{});
        else quantize_rows(r0, nr, slot0, std::false_type{});
    };
    const int c_pro = oh_begin - 1;             // POOL: the lone first conv row
    const int first_r0 = (POOL ? c_pro : oh_begin) * a.sH;
    const int first_n = POOL ? a.kH : span;
    int g_slot = 0;                             // ring slot of the group's first row
    dma_rows(first_r0, first_n);
    if constexpr (POOL) {
        // the tile's zero columns (conv columns -1 and oW) of its 5 rows
        const int C16 = a.OC >> 4, TW = a.oW + 2;
        if (tid < 10 * C16) {
            const int row = tid / (2 * C16), u = tid - row * 2 * C16;
            const int col = u < C16 ? 0 : TW - 1;
            *(v4i*)(tile + (row * TW + col) * a.OC + 16 * (u % C16)) = v4i{0, 0, 0, 0};
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
    quantize(first_r0, first_n, g_slot);
    lds_barrier();
    const uint8_t* const yq_img = a.y + (long long)n * a.pH * a.pW * a.OC;   // POOL output
    // gi = -1 (POOL): the lone conv row c_pro, whose span is kH rows and after
    // which the ring advances sH rows; the next step rows follow it as they
    // follow a group, so the first group's span is complete after them
    for (int gi = POOL ? -1 : 0;; ++gi) {
        const bool pro = POOL && gi < 0;
        const int oh0 = pro ? c_pro : oh_begin + a.R * gi;
        if (!pro && oh0 >= oh_end) break;
        const int span_g = pro ? a.kH : span;
        const bool more = pro || oh0 + a.R < oh_end;
        // the next group's new rows: raw input into the staging area
        const int pre_r0 = oh0 * a.sH + span_g;
        if (more) dma_rows(pre_r0, step);

        // MFMAs + epilogue, 16 pixels at a time; ks_base: dword offset of
        // this lane's kernel row and first tap of K-step ks from the group's
        // first ring row (the second mapping keeps a group's span contiguous)
        int ks_base[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) ks_base[ks] = (g_slot + k_kh[ks]) * a.L + k_kw[ks];
        const int P_here = (pro ? 1 : min(a.R, oh_end - oh0)) * a.oW;
        // outputs of this wave's pixel groups, stored after the ring refill so
        // that they stay in flight across the next group's DMA and MFMAs
        uint32_t outv[STEM_MGW][NT];
        // the pixel groups with the saturating epilogue (SAT) and the 8-byte
        // fragment reads (A8) fixed at compile time: a run-time test inside
        // puts a branch around every element and fragment read, and then no
        // MFMA, LDS read or epilogue instruction overlaps another
        auto run_groups = [&](auto sat_t, auto a8_t) {
            constexpr bool SAT = decltype(sat_t)::value;
            constexpr bool A8 = decltype(a8_t)::value;
#pragma unroll
            for (int i = 0; i < STEM_MGW; ++i) {
                const int mg = wave + 4 * i;
                if (mg * 16 < P_here) {
                    // this lane's 16-byte chunks: kernel row kh, taps kw0..kw0+3
                    v4i xf[KS];
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) {
                        const uint32_t* px = ring + ks_base[ks] + m_off[i];
                        if constexpr (A8) {
                            const uint2 lo = *(const uint2*)px, hi = *(const uint2*)(px + 2);
                            xf[ks] = v4i{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
                        } else {
                            xf[ks] = v4i{(int)px[0], (int)px[1], (int)px[2], (int)px[3]};
                        }
                    }
                    v4i acc[NT];
#pragma unroll
                    for (int tn = 0; tn < NT; ++tn) acc[tn] = c0v[tn];
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                        for (int tn = 0; tn < NT; ++tn)
                            acc[tn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[ks][tn], xf[ks], acc[tn], 0, 0, 0);
                    // RQ-C: rne(clamp(fma(fma(acc, cs, bf), 1/y_s, zp), qmin, qmax))
#pragma unroll
                    for (int tn = 0; tn < NT; ++tn) {
                        const v4i csq = csv[tn], bfq = bfv[tn];
                        uint32_t w = 0;
#pragma unroll
                        for (int qq = 0; qq < 4; ++qq) {
                            const float csf = __int_as_float(csq[qq]), bff = __int_as_float(bfq[qq]);
                            if constexpr (SAT) {
                                const float t = __builtin_fmaf((float)acc[tn][qq], csf, bff);
                                const float f = __builtin_fmaf(t, a.inv_y, (float)a.y_zp);
                                w = __builtin_amdgcn_cvt_pk_u8_f32(f, qq, w);
                            } else {
                                const uint32_t b = rqc_fast(acc[tn][qq], csf, bff, a.inv_y, a.y_zp, a.qmin, a.qmax);
                                w |= (b & 0xffu) << (8 * qq);
                            }
                        }
                        outv[i][tn] = w;
                    }
                }
            }
        };
        using T = std::true_type;
        using Fa = std::false_type;
        if (a.sat) {
            if (a.align8) run_groups(T{}, T{});
            else run_groups(T{}, Fa{});
        } else {
            if (a.align8) run_groups(Fa{}, T{});
            else run_groups(Fa{}, Fa{});
        }
        if constexpr (POOL) {
            // conv row c goes to tile row (c - c_pro) mod 5: the group's rows
            // take the slots after the previous group's last row, which stays
            const int TW = a.oW + 2;
            int base = (oh0 - c_pro) % 5;
#pragma unroll
            for (int i = 0; i < STEM_MGW; ++i) {
                const int p = (wave + 4 * i) * 16 + frow;
                if ((wave + 4 * i) * 16 < P_here && p < P_here && 16 * fch < a.OC) {
                    int slot = base + (m_tile[i] >> 24);
                    slot -= slot >= 5 ? 5 : 0;
                    *(v4i*)(tile + slot * TW * a.OC + (m_tile[i] & 0xffffff)) =
                        v4i{(int)outv[i][0], (int)outv[i][1], (int)outv[i][2], (int)outv[i][3]};
                }
            }
        }

        if (more) {
            // every wave's DMA has landed and no wave reads this group's ring
            // slots past its span: quantize the staged rows into the ring
            __builtin_amdgcn_s_waitcnt(0);
            lds_barrier();
            int p_slot = g_slot + span_g;
            p_slot -= p_slot >= a.WR ? a.WR : 0;
            quantize(pre_r0, step, p_slot);
        } else if constexpr (POOL) {
            lds_barrier();   // the tile rows are written
        }
        if constexpr (POOL) {
            if (!pro) {
                // pooled rows pa + 2 gi (conv rows oh0 - 1 .. oh0 + 1) and
                // pa + 2 gi + 1 (oh0 + 1 .. oh0 + 3), one (pixel, 16 channels)
                // a task; conv rows outside the image are skipped
                const int C16 = a.OC >> 4, TW = a.oW + 2;
                const int per_row = a.pW * C16;
                const int ph0 = pa + 2 * gi;
                for (int t = tid; t < 2 * per_row; t += 256) {
                    const int pr = t >= per_row ? 1 : 0;
                    const int u = t - pr * per_row;
                    const int pc = u / C16, ch = u - pc * C16;
                    const int ph = ph0 + pr;
                    if (ph >= pb) continue;
                    uint32_t lo[4] = {0, 0, 0, 0}, hi[4] = {0, 0, 0, 0};
#pragma unroll
                    for (int dr = 0; dr < 3; ++dr) {
                        const int c = 2 * ph - 1 + dr;
                        if ((unsigned)c >= (unsigned)a.oH) continue;
                        const int slot = (c - c_pro) % 5;
                        // tile column 2 pc holds conv column 2 pc - 1
                        const uint8_t* tp = tile + (slot * TW + 2 * pc) * a.OC + 16 * ch;
#pragma unroll
                        for (int dc = 0; dc < 3; ++dc) {
                            const v4i v = *(const v4i*)(tp + dc * a.OC);
#pragma unroll
                            for (int q = 0; q < 4; ++q) bytemax_acc((uint32_t)v[q], lo[q], hi[q]);
                        }
                    }
                    uint8_t* yp = (uint8_t*)yq_img + (uint32_t)((ph * a.pW + pc) * a.OC + 16 * ch);
                    *(v4i*)yp = v4i{(int)(lo[0] | (hi[0] << 8)), (int)(lo[1] | (hi[1] << 8)),
                                    (int)(lo[2] | (hi[2] << 8)), (int)(lo[3] | (hi[3] << 8))};
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < STEM_MGW; ++i) {
                const int p = (wave + 4 * i) * 16 + frow;
                if ((wave + 4 * i) * 16 < P_here && p < P_here && 4 * NT * fch < a.OC) {
                    uint8_t* yp = y_img + (uint32_t)((oh0 * a.oW + p) * a.OC + 4 * NT * fch);
                    if constexpr (NT == 4)
                        *(v4i*)yp = v4i{(int)outv[i][0], (int)outv[i][1], (int)outv[i][2], (int)outv[i][3]};
                    else if constexpr (NT == 2)
                        *(uint2*)yp = make_uint2(outv[i][0], outv[i][1]);
                    else
                        *(uint32_t*)yp = outv[i][0];
                }
            }
        }
        g_slot += pro ? a.sH : step;
        g_slot -= g_slot >= a.WR ? a.WR : 0;
        lds_barrier();
    }
}

bool stem_eligible(const StemArgs& a, bool f32) {
    if (a.C < 3 || a.C > 4 || a.cpr < 1 || a.KS < 1 || a.KS > 4 || a.kH < 1) return false;
    if (a.Kp != a.KS * 64 || a.kH * a.cpr * 16 > a.Kp) return false;
    if (a.OC < 16 || a.OC > 64 || (a.OC & 15)) return false;
    if (a.R < 1 || a.R * a.oW > 4 * 16 * STEM_MGW) return false;
    // raw rows in 16-byte chunks (4 fp32 or 16 uint8 elements), a row's
    // chunks over at most STEM_DMA rounds of the 256 threads
    if (a.W % (f32 ? 4 : 16) || (long long)a.C * a.W > 256LL * STEM_DMA * (f32 ? 4 : 16)) return false;
    if ((long long)a.C * a.H * a.W >= (1LL << 26)) return false;
    if ((long long)a.oH * a.oW * a.OC >= (1LL << 31)) return false;   // 32-bit output offsets
    const long long span = (long long)(a.R - 1) * a.sH + a.kH;
    const long long row_b = (long long)a.C * a.W * (f32 ? 4 : 1);   // raw bytes of one input row
    if (a.pool) {
        // groups of 4 conv rows (2 pooled rows); the ring holds one group's
        // span (the next rows are quantized after the group's MFMAs), the
        // staging area the kH rows of the lone first row or a group's new
        // rows; the conv tile 5 rows of oW + 2 pixels
        // a group's R * sH new rows overwrite the slots of rows no longer
        // read; more new rows than ring slots would overwrite each other
        if (a.R != 4 || a.KS != 4 || a.WR < span || (long long)a.R * a.sH > a.WR) return false;
        if (2LL * a.WR * a.L > STEM_P_RING_DW) return false;
        if ((long long)(a.kH > a.R * a.sH ? a.kH : a.R * a.sH) * row_b > STEM_P_STAGE_B) return false;
        if (5LL * (a.oW + 2) * a.OC > STEM_P_TILE_B) return false;
        if (a.pH != (a.oH - 1) / 2 + 1 || a.pW != (a.oW - 1) / 2 + 1 || (a.strip & 1)) return false;
        if ((long long)a.pH * a.pW * a.OC >= (1LL << 31)) return false;
    } else {
        // the ring holds the rows in use plus the next group's
        if (a.WR < span + a.R * a.sH) return false;
        // LDS: the ring, and the raw rows staged at once: the first group's
        // span, then each later group's R * sH new rows (more than a span
        // when sH > kH)
        const long long staged = span > (long long)a.R * a.sH ? span : (long long)a.R * a.sH;
        if (2LL * a.WR * a.L > STEM_RING_DW || staged * row_b > STEM_STAGE_B) return false;
    }
    if (a.L < (a.oW - 1) * a.sW + 4 * a.cpr || a.L > 4096) return false;
    if (a.align8 && ((a.sW & 1) || (a.L & 1))) return false;
    if (((uintptr_t)a.w & 15) || ((uintptr_t)a.c0 & 15) || ((uintptr_t)a.y & 15)) return false;
    return a.N >= 1 && a.N <= 65535 && a.strip >= 1;
}

hipError_t launch_stem_conv(const StemArgs& a, bool f32, hipStream_t s) {
    if (!stem_eligible(a, f32)) return hipErrorInvalidValue;
    const int rows = a.pool ? a.pH : a.oH;
    const dim3 grid((unsigned)((rows + a.strip - 1) / a.strip), (unsigned)a.N);
    if (((uintptr_t)a.x & 15)) return hipErrorInvalidValue;
    const size_t lds = 0;
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(256), lds, s, a); };
    auto by_ks = [&](auto f32c, auto ccc) {
        constexpr bool F = decltype(f32c)::value;
        constexpr int C = decltype(ccc)::value;
        if (a.pool) {
            go(stem_conv_kernel<F, C, 4, true>);   // (KS == 4: checked above)
            return;
        }
        switch (a.KS) {
        case 1:
            // 16 or 32 output channels: only their MFMA blocks
            if (a.OC == 16) go(stem_conv_kernel<F, C, 1, false, 1>);
            else if (a.OC == 32) go(stem_conv_kernel<F, C, 1, false, 2>);
            else go(stem_conv_kernel<F, C, 1, false>);
            break;
        case 2: go(stem_conv_kernel<F, C, 2, false>); break;
        case 3: go(stem_conv_kernel<F, C, 3, false>); break;
        default: go(stem_conv_kernel<F, C, 4, false>); break;
        }
    };
    using T = std::true_type;
    using Fa = std::false_type;
    if (a.C == 3) {
        if (f32) by_ks(T{}, std::integral_constant<int, 3>{});
        else by_ks(Fa{}, std::integral_constant<int, 3>{});
    } else {
        if (f32) by_ks(T{}, std::integral_constant<int, 4>{});
        else by_ks(Fa{}, std::integral_constant<int, 4>{});
    }
    return hipGetLastError();
}

}  // namespace nnrh
