// nnrh_qgemm_dma.hip -- pipelined int8 GEMM / implicit-GEMM convolution for
// gfx950: persistent blocks, direct global->LDS loads, S-stage LDS ring.
//
// Same arithmetic as qgemm_kernel (nnrh_qgemm.hip): i8 MFMA 16x16x64 with
// exact int32 accumulation, uint8 activations fed as x ^ 0x80 and the
// zero-point shift folded into the per-column constant c0[n], then one of
// NNR's requantize epilogues (RQ-B for the packed / NR16 conv drivers,
// jit_conv_int8_ukernel.cpp:906-967 and :1857-1918; RQ-D for QLinearMatMul,
// QLinearMatMul.cpp:188-198; RQ-A body for im2col, QLinearConv.cpp:1171-1179).
// Results are bit-identical to the register-staged kernel; only the data
// movement differs:
//  * every 16-byte chunk of the A and B tiles goes straight from global
//    memory into LDS (global_load_lds_dwordx4). No VGPR staging, so S
//    K-steps are in flight per block and HBM latency is hidden behind the
//    MFMA work of the steps before them;
//  * blocks are persistent: one block walks a list of output tiles and the
//    load stream runs across tile boundaries, so the next tile's first
//    K-steps load while the current tile's epilogue runs;
//  * out-of-image taps, rows past M and K padding load from a constant
//    16-byte pattern of the pad byte instead of branching around the load;
//  * the per-column requantize constants of a tile (c0 and the scales) ride
//    the same DMA stream into a small LDS ring slot, read back in the
//    epilogue without touching the vector-memory counter.
// The u8 -> s8 shift is applied to the activation fragments after they are
// read from LDS (4 v_xor per fragment).
//
// The first layer (3-4 input channels, RQ-C, first-layer driver of
// conv_first_layer_int8_avx512.h:262-273) runs here on a zero-point padded,
// multi-copy NHWC4 image (launch_first_layer_copies): every 16-byte chunk of
// its K order (kh, kw < kWp, c < 4) is then 4 aligned, in-bounds taps.
//
// Eligibility (checked by the launcher): A rows in 16-byte chunks (conv:
// channels % 16 == 0; dense: K % 16 == 0), no per-row zero-point term
// (beta == 0), zero points known on the host, NHWC / row-major output and
// no scalar-tail or RQ-B' columns. Everything else takes qgemm_kernel.
#include <type_traits>

#include <cstdio>

#include "nnrh_internal.h"
#include "nnrh_rq.h"

namespace nnrh {

typedef int v4i __attribute__((ext_vector_type(4)));
#define NNRH_LDS __attribute__((address_space(3)))

namespace {

// LDS image of a K-step: one row of BK bytes per A / B row, its 16-byte
// chunks XOR-swizzled by (row >> 1) so that the 16 rows one ds_read_b128
// touches spread over the banks
template <int BK>
__device__ __forceinline__ int dma_swz(int row) { return (row >> 1) & (BK / 16 - 1); }
template <int BK>
__device__ __forceinline__ int dma_lds_off(int row, int c) {
    return row * BK + ((c ^ dma_swz<BK>(row)) << 4);
}

// 256 x 16 bytes: chunk b holds 16 copies of byte b (pad source for the DMA)
struct PadTable {
    uint32_t w[256 * 4];
    constexpr PadTable() : w() {
        for (int i = 0; i < 256 * 4; ++i) w[i] = (uint32_t)(i >> 2) * 0x01010101u;
    }
};
__device__ const PadTable kPadTable{};

// s_waitcnt with vmcnt = n and no wait on expcnt / lgkmcnt (gfx9 encoding)
#define NNRH_VMCNT(n) ((((n) & 0xF)) | 0x70 | 0xF00 | ((((n) >> 4) & 3) << 14))
// lgkmcnt(0) alone (vmcnt and expcnt at their maxima)
#define NNRH_LGKMCNT0 0xC07F

__device__ __forceinline__ void dma16(const void* src, uint8_t* lds_dst) {
    __builtin_amdgcn_global_load_lds(src, (NNRH_LDS void*)lds_dst, 16, 0, 0);
}

// bytes 0 of a, b, c, d -> one dword (a lowest). v_perm_b32 selects bytes
// of {S0, S1} with S1 as bytes 0-3 and S0 as bytes 4-7; selector 0x0c is 0.
// the first `valid` (1..16) output bytes of {w0, w1, w2, w3} to p: 8- and
// 4-byte stores where p is 8-byte aligned, single bytes for the rest (a
// ragged last column chunk: 24 output channels take one 16-byte and one
// 8-byte store a row, or two 8-byte stores, instead of byte stores). The
// words stay in registers: every index is a constant.
__device__ __forceinline__ void store_bytes_prefix(uint8_t* p, uint32_t w0, uint32_t w1, uint32_t w2,
                                                   uint32_t w3, int valid) {
    auto bytes_of = [&](int from, uint32_t w, int n) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < n) p[from + i] = (uint8_t)(w >> (8 * i));
    };
    if ((((uintptr_t)p) & 7) == 0 && valid >= 8) {
        *(uint2*)p = make_uint2(w0, w1);
        if (valid == 16) {
            *(uint2*)(p + 8) = make_uint2(w2, w3);
        } else if (valid >= 12) {
            *(uint32_t*)(p + 8) = w2;
            bytes_of(12, w3, valid - 12);
        } else {
            bytes_of(8, w2, valid - 8);
        }
        return;
    }
    bytes_of(0, w0, valid);
    if (valid > 4) bytes_of(4, w1, valid - 4);
    if (valid > 8) bytes_of(8, w2, valid - 8);
    if (valid > 12) bytes_of(12, w3, valid - 12);
}

__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);   // [a0, b0, 0, 0]
    const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x0c0c0400u);   // [c0, d0, 0, 0]
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);              // [a0, b0, c0, d0]
}

__device__ __forceinline__ void block_barrier() {
    // plain s_barrier: the waits this kernel needs are explicit s_waitcnt;
    // the memory clobber keeps the compiler from moving LDS accesses across
    asm volatile("s_barrier" ::: "memory");
}

// epilogue fusions: none, QLinearAdd of a residual (RQ-B), DequantizeLinear
// of the output plus a per-column fp32 bias (RQ-D), or a per-row term
// row_coef[n] * (sum_k (a[m][k] - a_zp)) added to the int32 accumulator
// (EPI_I32), the row sums taken from the A fragments on the way. FUSE_DQC:
// the dequantize chain stores the uint8 RQ-D bytes (GemmArgs::dq_codes); its
// values are formed only for the (min, max) pairs, when those are written
// FUSE_ADD1: the fused add with one residual buffer for the block instead of
// one per slot (tiles of at least S K-steps; the residual then loads with the
// tile's step S - 1, after every wave's epilogue of the tile before)
enum { FUSE_NONE = 0, FUSE_ADD = 1, FUSE_DQB = 2, FUSE_ROW = 3, FUSE_DQC = 4, FUSE_ADD1 = 5 };
constexpr bool fuse_dq(int f) { return f == FUSE_DQB || f == FUSE_DQC; }
constexpr bool fuse_add(int f) { return f == FUSE_ADD || f == FUSE_ADD1; }

template <int EPI>
struct EpiParams;
// number of per-column 32-bit arrays staged per tile
template <> struct EpiParams<EPI_RQB> { static constexpr int NP = 2; };   // c0, os
template <> struct EpiParams<EPI_RQA> { static constexpr int NP = 3; };   // c0, cs, bf
template <> struct EpiParams<EPI_RQC> { static constexpr int NP = 3; };   // c0, cs, bf
template <> struct EpiParams<EPI_RQD> { static constexpr int NP = 1; };   // c0
template <> struct EpiParams<EPI_I32> { static constexpr int NP = 1; };   // c0
template <> struct EpiParams<EPI_I32S> { static constexpr int NP = 2; };  // c0, per-column scale

}  // namespace

// RQ-E of QLinearAdd (QLinearAdd.cpp:79-104) on one element: body is the
// 16-wide SIMD expression, tail the scalar one
__device__ __forceinline__ int qadd_elem(int a, int b, const GemmArgs& g, bool tail) {
    float v;
    if (!tail) {
        v = __builtin_fmaf((float)b, g.add_sb, g.add_fixed);
        v = __builtin_fmaf((float)a, g.add_sa, v);
    } else {
        const float t1 = g.add_sa * (float)(a - g.add_a_zp);
        const float t2 = g.add_sb * (float)(b - g.add_b_zp);
        v = (t1 + t2) + (float)g.add_y_zp;
    }
    return clampi(x86_f2i(__builtin_rintf(v)), g.lo, g.hi);
}

// LDS bytes of one block: S stages of A and B rows plus S per-tile slots,
// each NPX per-column arrays (1 KB granules) and, with a fused add, the
// tile's residual bytes
template <int BM, int BN, int S, int NPX, int FUSE>
constexpr int dma_pslot_bytes() {
    return ((NPX * BN * 4 + 1023) / 1024) * 1024 + (FUSE == FUSE_ADD ? BM * BN : 0);
}
// per-column arrays staged per tile: the epilogue's, + the fp32 bias of a
// fused dequantize, + the row-term coefficient
template <int EPI, int FUSE>
constexpr int dma_npx() { return EpiParams<EPI>::NP + (fuse_dq(FUSE) || FUSE == FUSE_ROW ? 1 : 0); }
// (KR > 0: the weights stay in registers, so a stage holds A rows only)
template <int BM, int BN, int S, int NPX, int FUSE, int BK, int KR>
constexpr int dma_lds_bytes() {
    return S * (BM + (KR ? 0 : BN)) * BK + S * dma_pslot_bytes<BM, BN, S, NPX, FUSE>() +
           (FUSE == FUSE_ADD1 ? BM * BN : 0);
}
// blocks per CU the kernel is compiled for: LDS and registers must fit them
// (4-wave blocks: 3 per CU when the LDS fits them, else 2; 8-wave blocks: 2)
template <int BM, int BN, int S, int NPX, int FUSE, int BK, int KR, int KSPLIT>
constexpr int dma_min_blocks() {
    return (BM / 64) * (BN / 64) * KSPLIT == 8 ? 2
                                               : (dma_lds_bytes<BM, BN, S, NPX, FUSE, BK, KR>() * 3 <= 160 * 1024 ? 3 : 2);
}
// threads of a block: a wave per 64 x 64 sub-tile (and per K half)
template <int BM, int BN, int KSPLIT = 1>
constexpr int dma_threads() { return (BM / 64) * (BN / 64) * KSPLIT * 64; }
// __launch_bounds__'s second argument in HIP is the minimum number of waves
// per SIMD (it sets the register budget): blocks per CU x waves per block / 4.
// 8-wave blocks get 128 VGPRs (2 blocks per CU) where the variant fits them;
// the general im2col producer, RQ-A and the row term do not without spills
// and keep 256 (one block per CU)
template <int BM, int BN, int S, int AMODE, int EPI, int FUSE, int BK, int KR, int KSPLIT>
constexpr int dma_min_waves_per_simd() {
    constexpr int waves = dma_threads<BM, BN, KSPLIT>() / 64;
    if (waves == 8 && (AMODE == A_CONV || EPI == EPI_RQA || FUSE == FUSE_ROW)) return 2;
    return dma_min_blocks<BM, BN, S, dma_npx<EPI, FUSE>(), FUSE, BK, KR, KSPLIT>() * waves / 4;
}

// BK: K bytes per pipeline stage, 64 (one MFMA K-step) or 128 (two). A
// 128-byte stage fetches whole 128-byte rows with each DMA instruction (8
// rows x 8 lanes instead of 16 rows x 4 lanes: twice the rate out of L2)
// and halves the barriers per K.
// KR: 0, or the packed K in 64-byte steps (1 or 2) when every tile of a block
// lies in one column block (the launcher sizes the grid for that, batch 1):
// each wave then loads its weight fragments once into registers and the
// stages carry A rows only, which leaves room for another stage or block.
// KSPLIT 2: two waves per 64 x 64 sub-tile, one per MFMA K-step of each
// 128-byte stage (twice the waves on a grid with few tiles); at the tile's
// end the halves exchange half-tiles of partial sums through the stage just
// consumed, and each half finishes two of the four 16-row blocks.
template <int BM, int BN, int S, int AMODE, int EPI, int FUSE, int BK, int KR = 0, int KSPLIT = 1>
__global__ __launch_bounds__((dma_threads<BM, BN, KSPLIT>()),
                             (dma_min_waves_per_simd<BM, BN, S, AMODE, EPI, FUSE, BK, KR, KSPLIT>()))
void qgemm_dma_kernel(GemmArgs g) {
    constexpr int WAVES_N = BN / 64;
    constexpr int WAVES_T = (BM / 64) * WAVES_N;   // waves of a tile's 64 x 64 sub-tiles
    constexpr int WAVES = WAVES_T * KSPLIT;
    constexpr int NT = 64 * WAVES;           // threads
    static_assert(WAVES == 4 || WAVES == 8, "4 or 8 waves of 64x64");
    static_assert(KSPLIT == 1 || (KSPLIT == 2 && BK == 128 && WAVES_T == 4 && KR == 0 && FUSE == FUSE_NONE),
                  "K split: 128-byte stages, 4 sub-tiles, no fusion");
    static_assert(BK == 64 || BK == 128, "stage width");
    static_assert(BK == 64 || AMODE != A_CONV4, "first layer: 64-byte stages");
    static_assert(KR == 0 || (KR <= 2 && BK == 64), "register weights: Kp = 64 or 128, 64-byte stages");
    constexpr int B_ROWS = KR ? 0 : BN;      // weight rows a stage carries
    constexpr int CPR = BK / 16;             // 16-byte chunks per LDS row
    constexpr int RND = NT * 16;             // bytes one DMA round of the block fills
    constexpr int RPR = RND / BK;            // rows one DMA round fills
    constexpr int A_CH = BM / RPR;           // DMA chunks per thread per step (A)
    constexpr int B_CH = BN / RPR;           // (B)
    constexpr int KK = BK / 64;              // MFMA K-steps per stage
    constexpr int LPS = A_CH + (KR ? 0 : B_CH);   // DMA instructions per thread per step
    constexpr int STAGE = (BM + B_ROWS) * BK;     // bytes per K-step
    constexpr int NP = EpiParams<EPI>::NP;
    constexpr int NPX = dma_npx<EPI, FUSE>();
    constexpr int PBYTES = NPX * BN * 4;
    constexpr int PWAVES = (PBYTES + 1023) / 1024;   // waves issuing the param DMA
    static_assert(PWAVES <= WAVES, "param slot");
    // per-tile slot: the per-column arrays, then (fused add) the residual tile
    // as BM rows of BN bytes, 16-byte chunks XOR-swizzled by row
    constexpr int PPAR = PWAVES * 1024;
    constexpr int PSLOT = dma_pslot_bytes<BM, BN, S, NPX, FUSE>();
    constexpr int RCPR = BN / 16;                    // residual chunks per row
    constexpr int RCH = fuse_add(FUSE) ? BM * BN / RND : 0;   // residual DMAs per thread
    // FUSE_ADD1: the one residual buffer, after the slots
    constexpr int RES1 = S * STAGE + S * PSLOT;

    __shared__ __attribute__((aligned(1024))) uint8_t lds[S * STAGE + S * PSLOT + (FUSE == FUSE_ADD1 ? BM * BN : 0)];
    static_assert(!fuse_add(FUSE) || (BM * BN) % RND == 0, "residual DMA granule");
    static_assert(BM % RPR == 0 && BN % RPR == 0, "DMA rounds per tile");
    static_assert(FUSE != FUSE_ROW || EPI == EPI_I32, "row term: int32 epilogue");

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // the wave index as a uniform value, so LDS destinations stay scalar
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // KSPLIT 2: K half kg of sub-tile sub
    const int kg = KSPLIT > 1 ? wave / WAVES_T : 0;
    const int sub = wave - kg * WAVES_T;
    const int wm = sub / WAVES_N, wn = sub % WAVES_N;
    const int frow = lane & 15, fchunk = lane >> 4;

    // ---- tile list: (z, m-block, n-block), n fastest; XCD-aware split
    const int nbn = (g.N + BN - 1) / BN;
    const int nbm = (g.M + BM - 1) / BM;
    const int per_z = nbm * nbn;
    const int total = per_z * g.nbatch;
    const int G = gridDim.x;
    int t_first, t_end, t_step;
    if ((G & 7) == 0) {
        const int chunk = (total + 7) >> 3;
        const int xcd = blockIdx.x & 7;
        t_first = xcd * chunk + (blockIdx.x >> 3);
        t_end = min(total, (xcd + 1) * chunk);
        t_step = G >> 3;
    } else {
        t_first = blockIdx.x;
        t_end = total;
        t_step = G;
    }
    if (t_first >= t_end) return;
    // tile index -> batch z, first row m0, first column n0
    auto decode = [&](int t, int& z, int& m0, int& n0) {
        z = g.nbatch == 1 ? 0 : (int)fast_div((uint32_t)t, g.div_pz_mul, g.div_pz_shift);
        const int r = t - z * per_z;
        const int mb = (int)fast_div((uint32_t)r, g.div_nbn_mul, g.div_nbn_shift);
        m0 = mb * BM;
        n0 = (r - mb * nbn) * BN;
    };

    const int nk = g.Kp / BK;
    const uint32_t xmask = (uint32_t)g.a_xor * 0x01010101u;
    // KR > 0: this wave's weight fragments of the block's column block, for
    // every K step of the tile (rows past Np repeat the last packed row; their
    // outputs are never stored)
    v4i wreg[KR ? KR : 1][4];
    if constexpr (KR > 0) {
        int zb, mb0, nb0;
        decode(t_first, zb, mb0, nb0);
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) {
            int n = nb0 + wn * 64 + tn * 16 + frow;
            n = n < g.Np ? n : g.Np - 1;
#pragma unroll
            for (int ks = 0; ks < KR; ++ks)
                wreg[ks][tn] = *(const v4i*)(g.b + (long long)n * g.Kp + ks * 64 + fchunk * 16);
        }
    }
    // zero-point column term from the activation zero point (host value or,
    // after DynamicQuantizeLinear, one byte in device memory)
    int alpha = g.alpha;
    if (g.alpha_zp_dev)
        alpha = (g.a_xor ? (int)*(const uint8_t*)g.alpha_zp_dev : (int)*(const int8_t*)g.alpha_zp_dev) - g.a_sub;
    const uint32_t neg_alpha = 0u - (uint32_t)alpha;
    // RQ-D combined scale, fl(fl(a_s * b_s) / y_s), with a device a_scale
    float cm = g.cm;
    const float a_scale_dev = ((EPI == EPI_RQD || EPI == EPI_I32S) && g.cm_a_scale_dev) ? *g.cm_a_scale_dev : 0.0f;
    if (EPI == EPI_RQD && g.cm_a_scale_dev) {
        const float t1 = a_scale_dev * g.cm_b;
        cm = t1 / g.cm_y;
    }
    // uint8 output whose clamp is exactly the [0, 255] saturation of
    // v_cvt_pk_u8_f32 (round to nearest even, saturate, insert one byte):
    // RQ-B with zero point 0 (clamp [0, 255] then rne) and RQ-D (rne of
    // acc*cm + zp, clamp [0, 255]) take one instruction for round + clamp + pack
    const bool sat_u8 = g.y_type == 0 && g.lo == 0 && g.hi == 255 && (EPI == EPI_RQD || g.y_zp == 0);
    // RQ-A adds the zero point after rounding (exact with the saturating
    // convert only for zero point 0); RQ-C rounds after adding it and clamps
    // to [L, hi] = [qmin, qmax]
    const bool sat_ac = g.y_type == 0 && g.L == 0 && g.hi == 255 && (EPI == EPI_RQC || g.y_zp == 0);
    const float zp_c = (float)g.y_zp;
    const uint8_t* pad16 = (const uint8_t*)&kPadTable.w[(g.pad_byte & 0xff) * 4];
    const int sp_out = g.oH * g.oW;
    // this thread's 16-byte chunk of a 64-byte row (pre-swizzled so the LDS
    // image matches dma_lds_off)
    const int cdma = (tid % CPR) ^ dma_swz<BK>(tid / CPR);

    // ---- producer (DMA issue) state
    int p_t = t_first, p_kt = 0, p_gs = 0;
    int p_stage = 0, p_pslot = 0;   // byte offsets of the stage / param slot being filled
    const uint8_t* p_a = nullptr;   // batch base of A
    int p_n0 = 0;
    long long p_pbase = 0;          // batch offset of the per-column arrays
    uint64_t a_addr[A_CH];          // A_DENSE / A_CONVU: address of this thread's chunk of row j
    uint32_t a_tmask[A_CH];         // A_CONVU: bit t set when tap t of row j is inside the image
    uint64_t b_addr[B_CH];          // this thread's chunk of weight row j
    long long a_base[A_CH];         // A_CONV / A_CONV4
    int a_ih0[A_CH], a_iw0[A_CH];
    bool a_ok[A_CH];
    int kc_ic = 0, kc_kh = 0, kc_kw = 0;   // A_CONV: tap of this thread's chunk
    int u_tap = 0, u_ic = 0, u_kh = 0, u_kw = 0, u_off = 0;   // A_CONVU: the step's tap

    int p_setup_m0 = 0;
    auto p_setup = [&](int t) {
        int z, m0;
        decode(t, z, m0, p_n0);
        p_setup_m0 = m0;
        p_a = g.a + (long long)z * g.a_bstride;
        const int8_t* pb = g.b + (long long)z * g.b_bstride;
        p_pbase = (long long)z * g.param_bstride;
#pragma unroll
        for (int j = 0; j < A_CH; ++j) {
            const int m = m0 + tid / CPR + RPR * j;
            a_ok[j] = m < g.M;
            const int mm = a_ok[j] ? m : 0;
            if constexpr (AMODE == A_DENSE) {
                a_addr[j] = (uint64_t)(p_a + (long long)mm * g.lda + cdma * 16);
            } else if constexpr (AMODE == A_CONVU) {
                const int img = (int)fast_div((uint32_t)mm, g.div_sp_mul, g.div_sp_shift);
                const int s = mm - img * sp_out;
                const int oh = (int)fast_div((uint32_t)s, g.div_ow_mul, g.div_ow_shift);
                const int ow = s - oh * g.oW;
                const int ih0 = oh * g.sH - g.pad_t, iw0 = ow * g.sW - g.pad_l;
                // (ih0, iw0) may lie in the padding: the address is only
                // dereferenced for taps inside the image
                a_addr[j] = (uint64_t)p_a +
                            (uint64_t)((((long long)img * g.H + ih0) * g.W + iw0) * g.Cs + cdma * 16);
                uint32_t hm = 0, wmk = 0, tm = 0;
                for (int kh = 0; kh < g.kH; ++kh)
                    hm |= (uint32_t)((unsigned)(ih0 + kh * g.dH) < (unsigned)g.H) << kh;
                for (int kw = 0; kw < g.kW; ++kw)
                    wmk |= (uint32_t)((unsigned)(iw0 + kw * g.dW) < (unsigned)g.W) << kw;
                for (int kh = 0; kh < g.kH; ++kh)
                    tm |= ((hm >> kh) & 1u) ? (wmk << (kh * g.kW)) : 0u;
                a_tmask[j] = a_ok[j] ? tm : 0u;
            } else if constexpr (AMODE == A_CONV4) {
                // padded multi-copy image: row start of this output pixel
                const int img = (int)fast_div((uint32_t)mm, g.div_sp_mul, g.div_sp_shift);
                const int s = mm - img * sp_out;
                const int oh = (int)fast_div((uint32_t)s, g.div_ow_mul, g.div_ow_shift);
                const int ow = s - oh * g.oW;
                const int pix0 = ow * g.sW;
                const int r = pix0 & 3;
                a_base[j] = (long long)(r >> g.copy_shift) * g.copy_stride +
                            (((long long)img * g.H + (long long)oh * g.sH) * g.W + (pix0 - r)) * 4;
                a_ih0[j] = 0; a_iw0[j] = 0;
            } else {
                const int img = (int)fast_div((uint32_t)mm, g.div_sp_mul, g.div_sp_shift);
                const int s = mm - img * sp_out;
                const int oh = (int)fast_div((uint32_t)s, g.div_ow_mul, g.div_ow_shift);
                const int ow = s - oh * g.oW;
                a_base[j] = (long long)img * g.H * g.W * g.Cs;
                a_ih0[j] = oh * g.sH - g.pad_t;
                a_iw0[j] = ow * g.sW - g.pad_l;
            }
        }
#pragma unroll
        for (int j = 0; j < B_CH; ++j) {
            int n = p_n0 + tid / CPR + RPR * j;
            n = n < g.Np ? n : g.Np - 1;
            b_addr[j] = (uint64_t)(pb + (long long)n * g.Kp + cdma * 16);
        }
        if constexpr (AMODE == A_CONV) {
            const int k = cdma * 16;
            const int kp = k / g.C;
            kc_ic = k - kp * g.C;
            kc_kh = kp / g.kW;
            kc_kw = kp - kc_kh * g.kW;
        }
        if constexpr (AMODE == A_CONVU) {
            u_tap = 0; u_ic = 0; u_kh = 0; u_kw = 0; u_off = 0;
        }
    };

    // issue the DMA of producer step (p_t, p_kt) into the stage at p_stage
    auto p_issue = [&]() {
        uint8_t* st = lds + p_stage;
        const int k0 = p_kt * BK;
#pragma unroll
        for (int j = 0; j < A_CH; ++j) {
            const uint8_t* src = pad16;
            if constexpr (AMODE == A_DENSE) {
                bool ok = a_ok[j];
                if (k0 + BK > g.K) ok = ok && (k0 + cdma * 16 < g.K);   // K padding
                if (ok) src = (const uint8_t*)(a_addr[j] + (uint64_t)k0);
            } else if constexpr (AMODE == A_CONVU) {
                if ((a_tmask[j] >> u_tap) & 1u) src = (const uint8_t*)(a_addr[j] + (uint64_t)(long long)u_off);
            } else if constexpr (AMODE == A_CONV4) {
                // chunk = 4 taps (kw0..kw0+3) x 4 channels of kernel row kh
                const int q = (k0 + cdma * 16) >> 4;
                const int cpr = g.kWp >> 2;
                const int kh = q / cpr;
                const int kw0 = (q - kh * cpr) << 2;
                if (a_ok[j] && kh < g.kH) src = p_a + a_base[j] + ((long long)kh * g.W + kw0) * 4;
            } else {
                if (a_ok[j] && kc_kh < g.kH) {
                    const int ih = a_ih0[j] + kc_kh * g.dH;
                    const int iw = a_iw0[j] + kc_kw * g.dW;
                    if ((unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W)
                        src = p_a + a_base[j] + ((long long)(ih * g.W + iw) * g.Cs + kc_ic);
                }
            }
            dma16(src, st + wave * 1024 + j * RND);
        }
        if constexpr (KR == 0) {
#pragma unroll
            for (int j = 0; j < B_CH; ++j)
                dma16((const void*)(b_addr[j] + (uint64_t)k0), st + BM * BK + wave * 1024 + j * RND);
        }
        if (p_kt == 0 && wave < PWAVES) {
            // per-column constants of the tile: NP arrays of BN int32/float,
            // one 16-byte chunk per lane; chunks past the arrays reload the
            // last one (never read back)
            const int i = wave * 64 + lane;          // chunk index in the slot
            const int arr = i / (BN / 4);
            const int col4 = i - arr * (BN / 4);
            int c = p_n0 + col4 * 4;
            c = c + 4 <= g.Np ? c : g.Np - 4;
            // array 0 is c0, or colsum when the zero point arrives with the
            // call; lanes past the last array reload array 0 (never read back)
            const void* base0 = g.c0 ? (const void*)g.c0 : (const void*)g.colsum;
            const void* base;
            if (fuse_dq(FUSE) && arr == NP) base = g.dq_bias;
            else if (FUSE == FUSE_ROW && arr == NP) base = g.row_coef;
            else if (arr == 0 || arr >= NP) base = base0;
            else if (EPI == EPI_RQB) base = g.os;
            else if (arr == 1) base = g.cs;
            else base = g.bf;
            const uint8_t* src = (const uint8_t*)base + (p_pbase + c) * 4;
            dma16(src, lds + S * STAGE + p_pslot + wave * 1024);
        }
        if constexpr (fuse_add(FUSE)) {
            if (p_kt == (FUSE == FUSE_ADD1 ? S - 1 : 0)) {
                // the residual tile of the fused QLinearAdd (batch 1, row stride
                // and base 16-byte aligned, N % 16 == 0: checked by the launcher);
                // it lands with the tile's first K step (FUSE_ADD1: step S - 1),
                // so the step waits cover it. FUSE_ADD1's one buffer: this step
                // issues after the barrier that follows the last wave's epilogue
                // of the tile before, whose residual it overwrites
                const int m0 = p_setup_m0;
#pragma unroll
                for (int j = 0; j < RCH; ++j) {
                    const int p = j * NT + wave * 64 + lane;   // chunk position in the slot
                    const int row = p / RCPR, pc = p - row * RCPR;
                    const int lc = pc ^ (row & (RCPR - 1));
                    const int m = m0 + row, n = p_n0 + lc * 16;
                    const uint8_t* src = pad16;
                    if (m < g.M && n < g.N) src = g.add_other + (long long)m * g.ldy + n;
                    dma16(src, lds + (FUSE == FUSE_ADD1 ? RES1 : S * STAGE + p_pslot + PPAR) + (j * NT + wave * 64) * 16);
                }
            }
        }
        // advance
        ++p_gs;
        p_stage = p_stage + STAGE == S * STAGE ? 0 : p_stage + STAGE;
        if constexpr (AMODE == A_CONV) {
            kc_ic += BK;
            while (kc_ic >= g.C) {
                kc_ic -= g.C;
                if (++kc_kw == g.kW) { kc_kw = 0; ++kc_kh; }
            }
        }
        if constexpr (AMODE == A_CONVU) {
            // C % BK == 0: the next step is the next BK channels of this tap,
            // or the first BK of the next tap (taps in (kh, kw) order)
            u_ic += BK;
            u_off += BK;
            if (u_ic == g.C) {
                u_ic = 0;
                ++u_tap;
                if (++u_kw == g.kW) { u_kw = 0; ++u_kh; }
                u_off = (u_kh * g.dH * g.W + u_kw * g.dW) * g.Cs;
            }
        }
        if (++p_kt == nk) {
            p_kt = 0;
            p_pslot = p_pslot + PSLOT == S * PSLOT ? 0 : p_pslot + PSLOT;
            p_t += t_step;
            if (p_t < t_end) p_setup(p_t);
        }
    };

    // ---- consumer state
    int c_t = t_first, c_kt = 0, c_gs = 0;
    int c_stage = 0, c_pslot = 0;
    v4i acc[4][4];   // started from c0 by the tile's first K-step
    // FUSE_ROW: this lane's partial sums of (a - a_sub) over its 16-byte
    // fragment chunks of rows tm * 16 + frow (the 4 lanes of a row hold the
    // 4 chunks of each 64-byte K step)
    int rsum[4] = {0, 0, 0, 0};

    // fused dequantize: running min / max of the fp32 outputs of the tile
    float mm_mn = 0.0f, mm_mx = 0.0f;

    // fp32 outputs of a fused epilogue (16 columns of one row): the Gelu
    // when fused, the running min / max for a DynamicQuantizeLinear that
    // reads them, then the store
    auto post_f32 = [&](float (&o)[16], bool full16, int nb) {
        if (g.dq_gelu) {
#pragma unroll
            for (int i = 0; i < 16; ++i) o[i] = gelu_erf(o[i]);
        }
        if (g.mm_parts) {
            // min / max of what this lane writes (0 stands in for nothing:
            // DynamicQuantizeLinear adds 0 anyway)
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (full16 || nb + i < g.N) {
                    mm_mn = fminf(mm_mn, o[i]);
                    mm_mx = fmaxf(mm_mx, o[i]);
                }
        }
    };
    auto store_f32 = [&](float (&o)[16], float* frow, bool full16, int nb) {
        post_f32(o, full16, nb);
        if (full16 && ((((uintptr_t)frow) & 15) == 0)) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *(float4*)(frow + 4 * q) = make_float4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (nb + i < g.N) frow[i] = o[i];
        }
    };

    // conv_is_a: the conv byte is input A of the fused QLinearAdd (else B)
    auto epilogue = [&](auto conv_is_a_t) {
        constexpr bool CONV_A = decltype(conv_is_a_t)::value;
        int z, m0, n0;
        decode(c_t, z, m0, n0);
        const int nl = wn * 64 + 16 * fchunk;   // first column of this lane in the tile
        const int nb = n0 + nl;
        if constexpr (FUSE == FUSE_ROW) {
            // row sums of the 4 lanes holding a row's chunks (lanes l, l ^ 16,
            // l ^ 32, l ^ 48), while every lane of the wave is active
#pragma unroll
            for (int tm = 0; tm < 4; ++tm) {
                rsum[tm] += __shfl_xor(rsum[tm], 16, 64);
                rsum[tm] += __shfl_xor(rsum[tm], 32, 64);
            }
        }
        if (nb >= g.N) return;
        // a grouped launch: member z's combined scale, zero point, output
        float cm_t = cm;
        int yzp_t = g.y_zp;
        if (fuse_dq(FUSE) && g.ngrp) {
            cm_t = g.grp_cm[z];
            if (g.cm_a_scale_dev) {
                const float t1 = a_scale_dev * g.grp_cm_b[z];
                cm_t = t1 / g.grp_cm_y[z];
            }
            yzp_t = g.grp_y_zp[z];
        }
        // the accumulators started at c0 (acc + c0 = the reference's value)
        const uint8_t* ps = lds + S * STAGE + c_pslot;
        // the tile's residual bytes (fused add)
        const uint8_t* rtile = FUSE == FUSE_ADD1 ? lds + RES1 : ps + PPAR;
        v4i p0[4], p1[4];
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) {
            if constexpr (NP >= 2) p0[tn] = *(const v4i*)(ps + BN * 4 + (nl + 4 * tn) * 4);
            if constexpr (NP >= 3) p1[tn] = *(const v4i*)(ps + 2 * BN * 4 + (nl + 4 * tn) * 4);
        }
        v4i rcoef[4];
        if constexpr (FUSE == FUSE_ROW) {
#pragma unroll
            for (int tn = 0; tn < 4; ++tn) rcoef[tn] = *(const v4i*)(ps + NP * BN * 4 + (nl + 4 * tn) * 4);
        }
        const bool full16 = nb + 16 <= g.N;
#pragma unroll
        for (int tm = 0; tm < 4; ++tm) {
            if (KSPLIT > 1 && (tm >> 1) != kg) continue;   // the other K half's rows
            const int m = m0 + wm * 64 + tm * 16 + frow;
            if (m >= g.M) continue;
            if constexpr (EPI == EPI_I32S) {
                // MatMulInteger -> Cast (float(acc), nearest even) -> Mul by
                // the scale product fl(a_s * w_s[n]) -> Add(bias[n]) (->
                // Gelu), each an IEEE binary32 operation in that order
                const float a_s = g.cm_a_scale_dev ? a_scale_dev : g.cm;
                const uint8_t* pb = ps + NP * BN * 4 + nl * 4;
                float* frow = (g.ngrp ? (float*)g.grp_y[z] : (float*)g.y + (long long)z * g.y_bstride) +
                              (long long)m * g.ldy + nb;
                float o[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float sp = a_s * __int_as_float(p0[i >> 2][i & 3]);
                    const float v = (float)acc[tm][i >> 2][i & 3] * sp;
                    o[i] = g.dq_nobias ? v : v + *(const float*)(pb + 4 * i);
                }
                store_f32(o, frow, full16, nb);
                continue;
            }
            if constexpr (EPI == EPI_I32) {
                v4i o[4];
#pragma unroll
                for (int tn = 0; tn < 4; ++tn) o[tn] = acc[tm][tn];
                if constexpr (FUSE == FUSE_ROW) {
                    // + row_coef[n] * sum_k (a - a_zp), int32 wrap-around: the
                    // Kp shifted bytes of the row (padding reads the zero
                    // point) sum to the row sum + Kp * alpha
                    const uint32_t r = (uint32_t)rsum[tm] - (uint32_t)g.Kp * (uint32_t)alpha;
#pragma unroll
                    for (int tn = 0; tn < 4; ++tn)
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            o[tn][q] = (int)((uint32_t)o[tn][q] + (uint32_t)rcoef[tn][q] * r);
                    if (g.y_nchw) {
                        // NCHW [img][n][s]: 16 lanes store 16 consecutive pixels
                        // of one channel plane
                        const int img = (int)fast_div((uint32_t)m, g.div_sp_mul, g.div_sp_shift);
                        const int sp = m - img * sp_out;
                        int32_t* yb = (int32_t*)g.y + (long long)z * g.y_bstride +
                                      ((long long)img * g.ldy + nb) * sp_out + sp;
#pragma unroll
                        for (int i = 0; i < 16; ++i)
                            if (nb + i < g.N) yb[(long long)i * sp_out] = o[i >> 2][i & 3];
                        continue;
                    }
                }
                int32_t* yrow = (int32_t*)g.y + (long long)z * g.y_bstride + (long long)m * g.ldy + nb;
                if (full16 && ((((uintptr_t)yrow) & 15) == 0)) {
#pragma unroll
                    for (int tn = 0; tn < 4; ++tn) *(v4i*)(yrow + 4 * tn) = o[tn];
                } else {
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (nb + i < g.N) yrow[i] = o[i >> 2][i & 3];
                }
            } else {
                uint32_t packed[4];
                // fused QLinearAdd, body rows: the conv byte enters RQ-E as
                // a float. rne(clamp(f, lo - zp, hi - zp)) + zp is exactly the
                // value of the byte RQ-B stores (an integer in [lo, hi]), so
                // it is used as it is, with no byte pack and unpack between
                // the two requantizations
                bool add_done = false;
                if constexpr (fuse_add(FUSE) && EPI == EPI_RQB) {
                    const long long i0 = (long long)m * g.ldy + nb;
                    if (i0 + 16 <= g.add_body) {
                        const int rrow = wm * 64 + tm * 16 + frow;
                        const int rpc = (wn * 4 + fchunk) ^ (rrow & (RCPR - 1));
                        const v4i rres = *(const v4i*)(rtile + (rrow * RCPR + rpc) * 16);
                        const float lo_f = (float)g.lo - (float)g.y_zp, hi_f = (float)g.hi - (float)g.y_zp;
                        auto add_body = [&](auto zp0_t) {
                            constexpr bool ZP0 = decltype(zp0_t)::value;
                            const float zp_f = (float)g.y_zp;
#pragma unroll
                            for (int tn = 0; tn < 4; ++tn) {
                                const uint32_t rw = (uint32_t)rres[tn];
                                uint32_t w = 0;
#pragma unroll
                                for (int q = 0; q < 4; ++q) {
                                    const float f = (float)acc[tm][tn][q] * __int_as_float(p0[tn][q]);
                                    float qf = __builtin_rintf(med3f(f, lo_f, hi_f));
                                    if constexpr (!ZP0) qf = qf + zp_f;
                                    const float rf = (float)((rw >> (8 * q)) & 0xffu);
                                    float v = __builtin_fmaf(CONV_A ? rf : qf, g.add_sb, g.add_fixed);
                                    v = __builtin_fmaf(CONV_A ? qf : rf, g.add_sa, v);
                                    w = __builtin_amdgcn_cvt_pk_u8_f32(v, q, w);
                                }
                                packed[tn] = w;
                            }
                        };
                        if (g.y_zp == 0) add_body(std::true_type{});
                        else add_body(std::false_type{});
                        add_done = true;
                    }
                }
                if (add_done) {
                } else if constexpr (EPI == EPI_RQB) {
                    if (sat_u8) {
                        // zero point 0: rne(clamp(f, 0, 255)) = sat(rne(f))
#pragma unroll
                        for (int tn = 0; tn < 4; ++tn) {
                            uint32_t w = 0;
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                const float f = (float)acc[tm][tn][q] * __int_as_float(p0[tn][q]);
                                w = __builtin_amdgcn_cvt_pk_u8_f32(f, q, w);
                            }
                            packed[tn] = w;
                        }
                    } else {
                        // RQ-B: with an even zero point, fl(f + 1.5*2^23 + zp)
                        // rounds to M + zp + rne(f) (the tie goes to the same
                        // even integer), so the low byte already holds
                        // rne(f) + zp; an odd zero point is added to the bit
                        // pattern
                        const float lo_f = (float)g.lo - (float)g.y_zp, hi_f = (float)g.hi - (float)g.y_zp;
                        auto rqb_row = [&](auto zp_even) {
                            constexpr bool EVEN = decltype(zp_even)::value;
                            const float magic = EVEN ? RNE_MAGIC + (float)g.y_zp : RNE_MAGIC;
#pragma unroll
                            for (int tn = 0; tn < 4; ++tn) {
                                uint32_t b[4];
#pragma unroll
                                for (int q = 0; q < 4; ++q) {
                                    float f = (float)acc[tm][tn][q] * __int_as_float(p0[tn][q]);
                                    f = med3f(f, lo_f, hi_f);
                                    b[q] = (uint32_t)__float_as_int(f + magic);
                                    if constexpr (!EVEN) b[q] += (uint32_t)g.y_zp;
                                }
                                packed[tn] = pack_low_bytes(b[0], b[1], b[2], b[3]);
                            }
                        };
                        if ((g.y_zp & 1) == 0) rqb_row(std::true_type{});
                        else rqb_row(std::false_type{});
                    }
                } else if (EPI == EPI_RQD && sat_u8) {
                    // RQ-D into uint8: sat(rne(acc*cm + zp)); a value >= 2^31
                    // (or NaN) converts to INT32_MIN on x86 and clamps to 0
                    const float zp_f = (float)yzp_t;
#pragma unroll
                    for (int tn = 0; tn < 4; ++tn) {
                        uint32_t w = 0;
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const float t = (float)acc[tm][tn][q] * cm_t;
                            float val = t + zp_f;
                            val = val < 2147483648.0f ? val : -1.0f;
                            w = __builtin_amdgcn_cvt_pk_u8_f32(val, q, w);
                        }
                        packed[tn] = w;
                    }
                } else if ((EPI == EPI_RQA || EPI == EPI_RQC) && sat_ac) {
                    // clamp [0, 255] into uint8 with zero point 0 (RQ-A) or
                    // bounds qmin = 0, qmax = 255 (RQ-C): the rounding,
                    // clamp and byte insert are one v_cvt_pk_u8_f32
#pragma unroll
                    for (int tn = 0; tn < 4; ++tn) {
                        uint32_t w = 0;
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const float t = __builtin_fmaf((float)acc[tm][tn][q], __int_as_float(p0[tn][q]),
                                                           __int_as_float(p1[tn][q]));
                            const float f = EPI == EPI_RQA ? t * g.inv_y : __builtin_fmaf(t, g.inv_y, zp_c);
                            w = __builtin_amdgcn_cvt_pk_u8_f32(f, q, w);
                        }
                        packed[tn] = w;
                    }
                } else {
#pragma unroll
                    for (int tn = 0; tn < 4; ++tn) {
                        uint32_t w = 0;
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const int32_t v = acc[tm][tn][q];
                            uint32_t b;
                            if constexpr (EPI == EPI_RQA)
                                b = rqa_fast(v, __int_as_float(p0[tn][q]), __int_as_float(p1[tn][q]),
                                             g.inv_y, g.y_zp, g.L, g.hi);
                            else if constexpr (EPI == EPI_RQC)
                                b = rqc_fast(v, __int_as_float(p0[tn][q]), __int_as_float(p1[tn][q]),
                                             g.inv_y, g.y_zp, g.L, g.hi);
                            else
                                b = rqd_fast(v, cm_t, yzp_t, g.lo, g.hi);
                            w |= (b & 0xffu) << (8 * q);
                        }
                        packed[tn] = w;
                    }
                }
                if constexpr (fuse_add(FUSE)) if (!add_done) {
                    // uint8 output (checked on the host)
                    const long long i0 = (long long)m * g.ldy + nb;
                    // this lane's 16 residual bytes (row m, columns nb..nb+15)
                    const int rrow = wm * 64 + tm * 16 + frow;
                    const int rpc = (wn * 4 + fchunk) ^ (rrow & (RCPR - 1));
                    const v4i rres = *(const v4i*)(rtile + (rrow * RCPR + rpc) * 16);
                    if (i0 + 16 <= g.add_body) {
                        // RQ-E body, fma(a, sa, fma(b, sb, fixed)); into uint8
                        // the reference's rint, cvt and saturation is
                        // v_cvt_pk_u8_f32 (round to nearest even, clamp [0,255])
#pragma unroll
                        for (int tn = 0; tn < 4; ++tn) {
                            const uint32_t qw = packed[tn], rw = (uint32_t)rres[tn];
                            uint32_t w = 0;
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                const float qf = (float)((qw >> (8 * q)) & 0xffu);
                                const float rf = (float)((rw >> (8 * q)) & 0xffu);
                                float v = __builtin_fmaf(CONV_A ? rf : qf, g.add_sb, g.add_fixed);
                                v = __builtin_fmaf(CONV_A ? qf : rf, g.add_sa, v);
                                w = __builtin_amdgcn_cvt_pk_u8_f32(v, q, w);
                            }
                            packed[tn] = w;
                        }
                    } else {
                        // the row segment reaches the scalar tail
#pragma unroll
                        for (int tn = 0; tn < 4; ++tn) {
                            uint32_t w = 0;
                            const uint32_t rw = (uint32_t)rres[tn];
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                const int qc = (int)((packed[tn] >> (8 * q)) & 0xffu);
                                const int rv = (int)((rw >> (8 * q)) & 0xffu);
                                const int a = CONV_A ? qc : rv;
                                const int b = CONV_A ? rv : qc;
                                const int o = qadd_elem(a, b, g, i0 + 4 * tn + q >= g.add_body);
                                w |= (uint32_t)(o & 0xff) << (8 * q);
                            }
                            packed[tn] = w;
                        }
                    }
                }
                if constexpr (fuse_dq(FUSE)) {
                    // DequantizeLinear fl((q - zp) * s) (DequantizeLinear.cpp:133-152),
                    // then the fp32 Add of the column bias, written as fp32
                    const float zp_f = (float)yzp_t;
                    const float dqs = g.ngrp ? g.grp_dq_scale[z] : g.dq_scale;
                    const uint8_t* pb = ps + NP * BN * 4 + nl * 4;
                    float o[16];
                    auto chain_values = [&]() {
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            // uint8 output (checked on the host)
                            const float qf = (float)((packed[i >> 2] >> (8 * (i & 3))) & 0xffu);
                            const float d = (qf - zp_f) * dqs;
                            o[i] = d + *(const float*)(pb + 4 * i);
                        }
                    };
                    if constexpr (FUSE == FUSE_DQC) {
                        // y gets the bytes; the values are formed only for
                        // the (min, max) pairs (the reader of the bytes
                        // forms them itself)
                        if (g.mm_parts) {
                            chain_values();
                            post_f32(o, full16, nb);
                        }
                        uint8_t* crow = (g.ngrp ? (uint8_t*)g.grp_y[z] : (uint8_t*)g.y + (long long)z * g.y_bstride) +
                                        (long long)m * g.ldy + nb;
                        if (full16 && ((((uintptr_t)crow) & 15) == 0))
                            *(v4i*)crow = v4i{(int)packed[0], (int)packed[1], (int)packed[2], (int)packed[3]};
                        else
                            store_bytes_prefix(crow, packed[0], packed[1], packed[2], packed[3],
                                               g.N - nb < 16 ? g.N - nb : 16);
                        continue;
                    }
                    chain_values();
                    float* frow = (g.ngrp ? (float*)g.grp_y[z] : (float*)g.y + (long long)z * g.y_bstride) +
                                  (long long)m * g.ldy + nb;
                    store_f32(o, frow, full16, nb);
                    continue;
                }
                uint8_t* yrow = (uint8_t*)g.y + (long long)z * g.y_bstride + (long long)m * g.ldy + nb;
                if (full16 && ((((uintptr_t)yrow) & 15) == 0)) {
                    // (a plain store: the next layer reads this output, and a
                    // streaming store would send it past the caches to HBM)
                    *(v4i*)yrow = v4i{(int)packed[0], (int)packed[1], (int)packed[2], (int)packed[3]};
                } else if constexpr (fuse_add(FUSE)) {
                    // (a fused add has output channels % 16 == 0: never ragged)
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (nb + i < g.N) yrow[i] = (uint8_t)(packed[i >> 2] >> (8 * (i & 3)));
                } else {
                    store_bytes_prefix(yrow, packed[0], packed[1], packed[2], packed[3], g.N - nb < 16 ? g.N - nb : 16);
                }
            }
        }
    };

    // ---- prologue: S-1 steps in flight
    p_setup(p_t);
#pragma unroll
    for (int s = 0; s < S - 1; ++s)
        if (p_t < t_end) p_issue();

    // wait until every wave's DMAs of consumer step cs have landed, then
    // refill the stage (and param slot) that no wave reads any more
    auto sync_step = [&](int cs) {
        // this thread's DMAs of step cs; later steps stay in flight
        const int ahead = p_gs - cs - 1;
        if (ahead >= S - 2) __builtin_amdgcn_s_waitcnt(NNRH_VMCNT((S - 2) * LPS));
        else if (S >= 4 && ahead == 1) __builtin_amdgcn_s_waitcnt(NNRH_VMCNT(LPS));
        else __builtin_amdgcn_s_waitcnt(NNRH_VMCNT(0));
        // (this wave's LDS reads of the stage being freed were consumed by
        // its MFMAs / epilogue before it got here)
        block_barrier();
        if (p_t < t_end) p_issue();
    };
    // fragments of MFMA K-step kk (of KK) of a stage
    auto read_frags = [&](int stage, int kk, v4i (&xf)[4], v4i (&wf)[4]) {
        const uint8_t* st = lds + stage;
        const int c = kk * 4 + fchunk;
#pragma unroll
        for (int tm = 0; tm < 4; ++tm) {
            v4i v = *(const v4i*)(st + dma_lds_off<BK>(wm * 64 + tm * 16 + frow, c));
            xf[tm] = v4i{(int)((uint32_t)v.x ^ xmask), (int)((uint32_t)v.y ^ xmask),
                         (int)((uint32_t)v.z ^ xmask), (int)((uint32_t)v.w ^ xmask)};
        }
        if constexpr (KR > 0) {
            // K step c_kt of the tile (64-byte stages)
#pragma unroll
            for (int tn = 0; tn < 4; ++tn) wf[tn] = (KR == 1 || c_kt == 0) ? wreg[0][tn] : wreg[KR - 1][tn];
        } else {
#pragma unroll
            for (int tn = 0; tn < 4; ++tn)
                wf[tn] = *(const v4i*)(st + BM * BK + dma_lds_off<BK>(wn * 64 + tn * 16 + frow, c));
        }
    };
    auto mma = [&](const v4i (&xf)[4], const v4i (&wf)[4], bool first) {
        if constexpr (FUSE == FUSE_ROW) {
#pragma unroll
            for (int tm = 0; tm < 4; ++tm) {
                int r = first ? 0 : rsum[tm];
                r = __builtin_amdgcn_sdot4(xf[tm].x, 0x01010101, r, false);
                r = __builtin_amdgcn_sdot4(xf[tm].y, 0x01010101, r, false);
                r = __builtin_amdgcn_sdot4(xf[tm].z, 0x01010101, r, false);
                r = __builtin_amdgcn_sdot4(xf[tm].w, 0x01010101, r, false);
                rsum[tm] = r;
            }
        }
        if (first) {
            // the tile's constants landed with its first K-step: the first
            // MFMAs start from c0[n] (this lane's 16 columns), or from
            // -alpha * colsum[n] when the zero point is only known now
            const uint8_t* ps = lds + S * STAGE + c_pslot;
            const int nl = wn * 64 + 16 * fchunk;
            v4i ci[4];
#pragma unroll
            for (int tn = 0; tn < 4; ++tn) {
                v4i c = *(const v4i*)(ps + (nl + 4 * tn) * 4);
                if (!g.c0) {
                    c.x = (int)(neg_alpha * (uint32_t)c.x); c.y = (int)(neg_alpha * (uint32_t)c.y);
                    c.z = (int)(neg_alpha * (uint32_t)c.z); c.w = (int)(neg_alpha * (uint32_t)c.w);
                }
                // (the second K half starts from zero: c0 enters the sum once)
                if (KSPLIT > 1 && kg != 0) c = v4i{0, 0, 0, 0};
                ci[tn] = c;
            }
#pragma unroll
            for (int tm = 0; tm < 4; ++tm)
#pragma unroll
                for (int tn = 0; tn < 4; ++tn)
                    acc[tm][tn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[tn], xf[tm], ci[tn], 0, 0, 0);
        } else {
#pragma unroll
            for (int tm = 0; tm < 4; ++tm)
#pragma unroll
                for (int tn = 0; tn < 4; ++tn)
                    acc[tm][tn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[tn], xf[tm], acc[tm][tn], 0, 0, 0);
        }
    };
    // after the MFMAs of a step: the epilogue when it was the tile's last;
    // false when the block has no tile left
    auto finish_step = [&]() -> bool {
        ++c_gs;
        const int done_stage = c_stage;
        c_stage = c_stage + STAGE == S * STAGE ? 0 : c_stage + STAGE;
        if (++c_kt == nk) {
            if constexpr (KSPLIT > 1) {
                // K halves -> sums, through the stage just consumed (no DMA
                // targets it before the next step's barrier): the second half
                // hands over its 16-row blocks 0-1 (8 KB per sub-tile), the
                // first adds them and hands over its blocks 2-3
                v4i* xb = (v4i*)(lds + done_stage + sub * 8192) + lane;
                block_barrier();   // every wave's fragment reads of the stage are done
                if (kg != 0) {
#pragma unroll
                    for (int tm = 0; tm < 2; ++tm)
#pragma unroll
                        for (int tn = 0; tn < 4; ++tn) xb[(tm * 4 + tn) * 64] = acc[tm][tn];
                }
                __builtin_amdgcn_s_waitcnt(NNRH_LGKMCNT0);
                block_barrier();
                if (kg == 0) {
#pragma unroll
                    for (int tm = 0; tm < 2; ++tm)
#pragma unroll
                        for (int tn = 0; tn < 4; ++tn) {
                            const v4i o = xb[(tm * 4 + tn) * 64];
                            acc[tm][tn] = v4i{(int)((uint32_t)acc[tm][tn].x + (uint32_t)o.x),
                                              (int)((uint32_t)acc[tm][tn].y + (uint32_t)o.y),
                                              (int)((uint32_t)acc[tm][tn].z + (uint32_t)o.z),
                                              (int)((uint32_t)acc[tm][tn].w + (uint32_t)o.w)};
                            xb[(tm * 4 + tn) * 64] = acc[tm + 2][tn];
                        }
                }
                __builtin_amdgcn_s_waitcnt(NNRH_LGKMCNT0);
                block_barrier();
                if (kg != 0) {
#pragma unroll
                    for (int tm = 2; tm < 4; ++tm)
#pragma unroll
                        for (int tn = 0; tn < 4; ++tn) {
                            const v4i o = xb[((tm - 2) * 4 + tn) * 64];
                            acc[tm][tn] = v4i{(int)((uint32_t)acc[tm][tn].x + (uint32_t)o.x),
                                              (int)((uint32_t)acc[tm][tn].y + (uint32_t)o.y),
                                              (int)((uint32_t)acc[tm][tn].z + (uint32_t)o.z),
                                              (int)((uint32_t)acc[tm][tn].w + (uint32_t)o.w)};
                        }
                }
            }
            if (fuse_add(FUSE) && g.add_conv_is_a) epilogue(std::true_type{});
            else epilogue(std::false_type{});
            if (fuse_dq(FUSE) && g.mm_parts) {
                // one (min, max) pair per (tile, wave), at 2 * (WAVES * tile + wave)
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) {
                    mm_mn = fminf(mm_mn, __shfl_xor(mm_mn, off, 64));
                    mm_mx = fmaxf(mm_mx, __shfl_xor(mm_mx, off, 64));
                }
                if (lane == 0)
                    *(float2*)(g.mm_parts + 2 * (WAVES * c_t + wave)) = make_float2(mm_mn, mm_mx);
                mm_mn = 0.0f;
                mm_mx = 0.0f;
            }
            c_kt = 0;
            c_pslot = c_pslot + PSLOT == S * PSLOT ? 0 : c_pslot + PSLOT;
            c_t += t_step;
            if (c_t >= t_end) return false;
        }
        return true;
    };

    for (;;) {
        sync_step(c_gs);
        if constexpr (KSPLIT > 1) {
            // this wave's K half of the stage
            v4i xf[4], wf[4];
            read_frags(c_stage, kg, xf, wf);
            mma(xf, wf, c_kt == 0);
        } else {
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) {
                v4i xf[4], wf[4];
                read_frags(c_stage, kk, xf, wf);
                mma(xf, wf, kk == 0 && c_kt == 0);
            }
        }
        if (!finish_step()) break;
    }
    // nothing may be left in flight into LDS when the block retires
    __builtin_amdgcn_s_waitcnt(NNRH_VMCNT(0));
}

// Dense GEMMs with a short K (KS 64-byte MFMA K steps, KS = 1 launched)
// and the RQ-B epilogue: the pointwise convolutions of MobileNetV2 with
// C <= 64 and the first of ResNet-50. There is
// little to stage: each wave keeps the weight fragments and per-column
// constants of one 64-column block in registers and walks 64-row tiles of
// A on its own -- fragments loaded straight from global memory (one tile
// ahead), 16 MFMAs a K step, the epilogue, 16-byte stores -- with no LDS
// and no barrier. A row whose K is not a multiple of 16 (24 channels) is
// read in 8-byte pieces up to K; the rest of its last chunk is 0, which
// meets zero weight columns.
template <int KS>
__global__ __launch_bounds__(256, 2) void qgemm_direct_kernel(GemmArgs g) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int frow = lane & 15, fchunk = lane >> 4;
    const int nbn = (g.N + 63) >> 6;
    const int gw = blockIdx.x * 4 + (tid >> 6), tw = gridDim.x * 4;
    // this wave's column block and first row tile; waves step over row tiles
    // by tw / nbn (waves past the last whole multiple of nbn have no work)
    const int cb = gw % nbn;
    const int rstep = tw / nbn;
    if (gw >= rstep * nbn) return;
    const int nrt = (g.M + 63) >> 6;
    int rt = gw / nbn;
    if (rt >= nrt) return;
    const int nb = cb * 64 + 16 * fchunk;   // first of this lane's 16 columns
    v4i wreg[KS][4], c0v[4];
    float osv[16];
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
        int n = cb * 64 + tn * 16 + frow;
        n = n < g.Np ? n : g.Np - 1;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) wreg[ks][tn] = *(const v4i*)(g.b + (long long)n * g.Kp + ks * 64 + fchunk * 16);
        c0v[tn] = *(const v4i*)(g.c0 + nb + 4 * tn);
        const v4i o = *(const v4i*)(g.os + nb + 4 * tn);
#pragma unroll
        for (int q = 0; q < 4; ++q) osv[4 * tn + q] = __int_as_float(o[q]);
    }
    const uint32_t xmask = (uint32_t)g.a_xor * 0x01010101u;
    const bool k16 = (g.K & 15) == 0;
    // fragment (row tile r, K step ks, row block tm) of this lane
    auto load = [&](int r, v4i (&xf)[KS][4]) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int tm = 0; tm < 4; ++tm) {
                const int m = r * 64 + tm * 16 + frow;
                const int k = ks * 64 + fchunk * 16;
                v4i v = v4i{0, 0, 0, 0};
                if (m < g.M && k < g.K) {
                    const uint8_t* src = g.a + (long long)m * g.lda + k;
                    if (k16) {
                        v = *(const v4i*)src;
                    } else {
                        // rows 8-byte aligned, K % 8 == 0: 8-byte pieces up to K
                        const uint2 lo = *(const uint2*)src;
                        const uint2 hi = k + 16 <= g.K ? *(const uint2*)(src + 8) : make_uint2(0u, 0u);
                        v = v4i{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
                    }
                }
                xf[ks][tm] = v4i{(int)((uint32_t)v.x ^ xmask), (int)((uint32_t)v.y ^ xmask),
                                 (int)((uint32_t)v.z ^ xmask), (int)((uint32_t)v.w ^ xmask)};
            }
    };
    const bool sat_u8 = g.y_type == 0 && g.lo == 0 && g.hi == 255 && g.y_zp == 0;
    const bool full16 = nb + 16 <= g.N;
    v4i xa[KS][4], xb[KS][4];
    load(rt, xa);
    for (;;) {
        v4i acc[4][4];
#pragma unroll
        for (int tm = 0; tm < 4; ++tm)
#pragma unroll
            for (int tn = 0; tn < 4; ++tn) {
                acc[tm][tn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wreg[0][tn], xa[0][tm], c0v[tn], 0, 0, 0);
#pragma unroll
                for (int ks = 1; ks < KS; ++ks)
                    acc[tm][tn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wreg[ks][tn], xa[ks][tm], acc[tm][tn], 0, 0, 0);
            }
        const int r = rt;
        rt += rstep;
        const bool more = rt < nrt;
        if (more) load(rt, xb);   // the next tile's fragments fly during the epilogue
        if (nb < g.N) {
#pragma unroll
            for (int tm = 0; tm < 4; ++tm) {
                const int m = r * 64 + tm * 16 + frow;
                if (m >= g.M) continue;
                uint8_t* yrow = (uint8_t*)g.y + (long long)m * g.ldy + nb;
                uint32_t packed[4];
                if (sat_u8) {
#pragma unroll
                    for (int tn = 0; tn < 4; ++tn) {
                        uint32_t w = 0;
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            w = __builtin_amdgcn_cvt_pk_u8_f32((float)acc[tm][tn][q] * osv[4 * tn + q], q, w);
                        packed[tn] = w;
                    }
                } else {
#pragma unroll
                    for (int tn = 0; tn < 4; ++tn) {
                        uint32_t b[4];
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            b[q] = rqb_fast(acc[tm][tn][q], osv[4 * tn + q], g.y_zp, g.lo, g.hi);
                        packed[tn] = pack_low_bytes(b[0], b[1], b[2], b[3]);
                    }
                }
                if (full16) {
                    *(v4i*)yrow = v4i{(int)packed[0], (int)packed[1], (int)packed[2], (int)packed[3]};
                } else {
                    store_bytes_prefix(yrow, packed[0], packed[1], packed[2], packed[3], g.N - nb < 16 ? g.N - nb : 16);
                }
            }
        }
        if (!more) break;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int tm = 0; tm < 4; ++tm) xa[ks][tm] = xb[ks][tm];
    }
}

namespace {

template <int BM, int BN, int S, int AMODE, int EPI, int FUSE = FUSE_NONE, int BK = 64, int KR = 0, int KSPLIT = 1>
hipError_t launch_dma(const GemmArgs& g, int batch, hipStream_t s) {
    auto kern = qgemm_dma_kernel<BM, BN, S, AMODE, EPI, FUSE, BK, KR, KSPLIT>;
    const long long tiles = (long long)((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN) * batch;
    // resident blocks of this instantiation (occupancy x CUs), computed once
    static int resident = 0;
    if (resident <= 0) {
        int per_cu = 0, dev = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, dma_threads<BM, BN, KSPLIT>(), 0) != hipSuccess ||
            per_cu < 1)
            per_cu = 1;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
            cus = 256;
        resident = per_cu * cus;
    }
    long long cap = resident;
    cap = cap < 8 ? 8 : (cap & ~7LL);
    long long G = tiles < cap ? tiles : cap;
    if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
    if constexpr (KR > 0) {
        // one column block per block: with 8 * nbn | G, every block's tiles
        // t_first + j * G / 8 share t_first's column block (batch 1)
        const long long q = 8LL * ((g.N + BN - 1) / BN);
        if (batch != 1 || g.Kp != 64 * KR) return hipErrorInvalidValue;
        G = (G / q) * q;
        if (G < q) return hipErrorInvalidValue;
    }
    GemmArgs a = g;
    a.nbatch = batch;
    {
        const uint32_t nbn = (uint32_t)((g.N + BN - 1) / BN);
        const uint32_t per_z = (uint32_t)((g.M + BM - 1) / BM) * nbn;
        fast_div_consts(per_z, &a.div_pz_mul, &a.div_pz_shift);
        fast_div_consts(nbn, &a.div_nbn_mul, &a.div_nbn_shift);
    }
    if (g.H > 0) {
        fast_div_consts((uint32_t)(g.oH * g.oW), &a.div_sp_mul, &a.div_sp_shift);
        fast_div_consts((uint32_t)g.oW, &a.div_ow_mul, &a.div_ow_shift);
    }
    if (prof_enabled()) {
        char nm[96];
        snprintf(nm, sizeof(nm), "variant:dma<%d,%d,%d,%d,%d,%d,%d,%d,%d>", BM, BN, S, AMODE, EPI, FUSE, BK, KR,
                 KSPLIT);
        prof_count(nm);
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)G, 1, 1), dim3(dma_threads<BM, BN, KSPLIT>()), 0, s, a);
    return hipGetLastError();
}

template <int BM, int BN, int S, int AMODE, int S_ADD = S, int BK = 64>
hipError_t launch_dma_epi(const GemmArgs& g, int batch, hipStream_t s) {
    if (g.dq_bias) {
        if constexpr (AMODE == A_DENSE) {
            if (g.epi == EPI_RQD)
                return g.dq_codes ? launch_dma<BM, BN, S, AMODE, EPI_RQD, FUSE_DQC, BK>(g, batch, s)
                                  : launch_dma<BM, BN, S, AMODE, EPI_RQD, FUSE_DQB, BK>(g, batch, s);
            if (g.epi == EPI_I32S) return launch_dma<BM, BN, S, AMODE, EPI_I32S, FUSE_DQB, BK>(g, batch, s);
        }
        return hipErrorNotSupported;
    }
    if (g.row_coef) {
        if constexpr (AMODE == A_CONV || AMODE == A_CONVU) {
            if (g.epi == EPI_I32 && g.H > 0)
                return launch_dma<BM, BN, S, AMODE, EPI_I32, FUSE_ROW, BK>(g, batch, s);
        }
        return hipErrorNotSupported;
    }
    if (g.add_other) {
        // the residual tile shares the block's LDS: 64-byte stages only
        if constexpr (BK == 64 && (AMODE == A_CONV || AMODE == A_CONVU || AMODE == A_DENSE)) {
            if (g.epi == EPI_RQB && batch == 1) {
                if constexpr (AMODE == A_DENSE && BM == 128 && BN == 128) {
                    // K = 64: weights in registers, so a slot holds A rows,
                    // the constants and the residual tile (25 KB): 2 stages
                    // at 3 blocks per CU (measured: ResNet-50's K = 64
                    // layers 106 -> 96 us; 3 stages at 2 blocks per CU gain
                    // half that). Only with a few tiles for every resident
                    // block. (K = 128 in registers spills at 3 blocks per CU;
                    // the one-residual-buffer kernel below is 2 % faster
                    // over ResNet-50.)
                    const long long q = 8LL * ((g.N + BN - 1) / BN);
                    const long long tiles = (long long)((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
                    if (tiles >= 4 * q && g.Kp == 64)
                        return launch_dma<BM, BN, 2, AMODE, EPI_RQB, FUSE_ADD, 64, 1>(g, batch, s);
                }
                // one residual buffer where that gains a third block per CU
                // (tiles of at least S_ADD K-steps)
                constexpr int NPX = dma_npx<EPI_RQB, FUSE_ADD>();
                if constexpr (dma_min_blocks<BM, BN, S_ADD, NPX, FUSE_ADD1, 64, 0, 1>() >
                              dma_min_blocks<BM, BN, S_ADD, NPX, FUSE_ADD, 64, 0, 1>()) {
                    if (g.Kp >= 64 * S_ADD) return launch_dma<BM, BN, S_ADD, AMODE, EPI_RQB, FUSE_ADD1>(g, batch, s);
                }
                return launch_dma<BM, BN, S_ADD, AMODE, EPI_RQB, FUSE_ADD>(g, batch, s);
            }
        }
        return hipErrorNotSupported;
    }
    switch (g.epi) {
    case EPI_RQB: return launch_dma<BM, BN, S, AMODE, EPI_RQB, FUSE_NONE, BK>(g, batch, s);
    case EPI_RQA: return launch_dma<BM, BN, S, AMODE, EPI_RQA, FUSE_NONE, BK>(g, batch, s);
    case EPI_RQD: return launch_dma<BM, BN, S, AMODE, EPI_RQD, FUSE_NONE, BK>(g, batch, s);
    case EPI_I32: return launch_dma<BM, BN, S, AMODE, EPI_I32, FUSE_NONE, BK>(g, batch, s);
    default: return hipErrorNotSupported;
    }
}

// 8-wave tiles: no fused add or dequantize (their LDS slots would not fit
// two blocks per CU)
template <int BM, int BN, int S, int AMODE>
hipError_t launch_dma_plain(const GemmArgs& g, int batch, hipStream_t s) {
    if (g.add_other || g.dq_bias) return hipErrorNotSupported;
    if (g.row_coef) {
        if constexpr (AMODE == A_CONV || AMODE == A_CONVU) {
            if (g.epi == EPI_I32 && g.H > 0) return launch_dma<BM, BN, S, AMODE, EPI_I32, FUSE_ROW>(g, batch, s);
        }
        return hipErrorNotSupported;
    }
    switch (g.epi) {
    case EPI_RQB: return launch_dma<BM, BN, S, AMODE, EPI_RQB>(g, batch, s);
    case EPI_RQA: return launch_dma<BM, BN, S, AMODE, EPI_RQA>(g, batch, s);
    case EPI_RQD: return launch_dma<BM, BN, S, AMODE, EPI_RQD>(g, batch, s);
    case EPI_I32: return launch_dma<BM, BN, S, AMODE, EPI_I32>(g, batch, s);
    default: return hipErrorNotSupported;
    }
}

// 128 x 128 tiles with K split over two waves a sub-tile (128-byte stages,
// 2 stages, 2 blocks of 8 waves per CU): dense and uniform-tap producers,
// plain RQ-B / RQ-D / int32 epilogues (the variants that fit 128 VGPRs)
template <int AMODE>
hipError_t launch_dma_ksplit(const GemmArgs& g, int batch, hipStream_t s) {
    static_assert(AMODE == A_DENSE || AMODE == A_CONVU, "K split producers");
    switch (g.epi) {
    case EPI_RQB: return launch_dma<128, 128, 2, AMODE, EPI_RQB, FUSE_NONE, 128, 0, 2>(g, batch, s);
    case EPI_RQD: return launch_dma<128, 128, 2, AMODE, EPI_RQD, FUSE_NONE, 128, 0, 2>(g, batch, s);
    case EPI_I32: return launch_dma<128, 128, 2, AMODE, EPI_I32, FUSE_NONE, 128, 0, 2>(g, batch, s);
    default: return hipErrorNotSupported;
    }
}

// first layer: RQ-C only
template <int BM, int BN, int S>
hipError_t launch_dma_first(const GemmArgs& g, int batch, hipStream_t s) {
    switch (g.epi) {
    case EPI_RQC: return launch_dma<BM, BN, S, A_CONV4, EPI_RQC>(g, batch, s);
    default: return hipErrorNotSupported;
    }
}

}  // namespace

bool qgemm_dma_eligible(const GemmArgs& g, int vec) {
    // the per-row term and an NCHW store: int32 output of a convolution only
    const bool row_term = g.row_coef != nullptr && g.epi == EPI_I32;
    if (g.y_nchw && !(row_term && g.H > 0)) return false;
    if (row_term && (g.H <= 0 || g.rowsum != nullptr || g.alpha_zp_dev || g.add_other || g.dq_bias || g.kWp > 0))
        return false;
    // accumulators start at c0: |c0| + 128*128*K must stay inside int32
    if (g.c0_absmax + 16384LL * (long long)g.Kp >= 0x7fffffffLL) return false;
    if (g.M > 0x7fffffff / 2) return false;
    if (g.kWp > 0) {
        // first layer: only on the padded multi-copy image
        if (g.copy_stride <= 0 || (g.copy_stride & 15) || (g.W & 3) || (g.kWp & 3)) return false;
        if (g.epi != EPI_RQC || g.c0 == nullptr || g.rowsum != nullptr || g.tail != TAIL_NONE) return false;
        return g.Np >= 4 && (g.Np & 3) == 0;
    }
    if (vec != 16) return false;
    // per-column constant: c0, or -alpha * colsum (GEMMs without bias)
    if (g.rowsum != nullptr) return false;
    if (g.c0 == nullptr && (g.colsum == nullptr || (g.epi != EPI_RQD && g.epi != EPI_I32 && g.epi != EPI_I32S)))
        return false;
    if (g.epi == EPI_I32S && (g.cs == nullptr || g.dq_bias == nullptr || g.H > 0)) return false;
    if (g.c0 == nullptr && 256LL * 128LL * (long long)g.Kp + 16384LL * (long long)g.Kp >= 0x7fffffffLL)
        return false;
    if (g.c0 != nullptr && g.alpha_zp_dev != nullptr) return false;
    // every per-column array the epilogue stages must exist
    if (g.epi == EPI_RQB && g.os == nullptr) return false;
    if ((g.epi == EPI_RQA || g.epi == EPI_RQC) && (g.cs == nullptr || g.bf == nullptr)) return false;
    if (g.tail != TAIL_NONE) return false;
    if (g.epi == EPI_RQB && g.bprime_from < g.N) return false;
    if (g.epi == EPI_RQC) return false;   // RQ-C is the first layer's epilogue
    if (g.Np < 4 || (g.Np & 3)) return false;
    if (g.H > 0 && (g.C % 16 || g.Cs % 16)) return false;
    if (g.H == 0 && (g.K % 16 || g.lda % 16)) return false;
    return true;
}

// the uniform-tap conv producer: every 64-byte K step inside one tap, the
// tap-validity mask of a row in 32 bits, tap offsets in int32
static bool conv_uniform_taps(const GemmArgs& g) {
    if (g.C % 64 || g.Kp != g.K || g.kH * g.kW > 32) return false;
    const long long span = ((long long)(g.kH - 1) * g.dH * g.W + (long long)(g.kW - 1) * g.dW) * g.Cs + g.C;
    return span < 0x7fffffffLL;
}

// the short-K direct kernel's shapes: dense A (K % 8 == 0, rows 8-byte
// aligned; 16-byte when K % 16 == 0) with one K step (Kp = 64), RQ-B with
// its constants precomputed, uint8 / int8 row-major output with 16-byte
// aligned rows, no fusion; batch 1. There it is faster than the pipelined
// kernel (measured per layer on ResNet-50 and MobileNetV2); with Kp = 128
// the pipelined kernel wins, and so does its fused-add variant with the
// weights in registers (a version of this kernel with the residual loaded
// one tile ahead ran ResNet-50's stage-1 conv + add layers 95 -> 121 us).
bool qgemm_direct_eligible(const GemmArgs& g, int batch) {
    if (batch != 1 || g.H > 0 || g.kWp > 0 || g.Kp != 64 || g.K <= 0 || (g.K & 7)) return false;
    if (g.epi != EPI_RQB || !g.c0 || !g.os || g.rowsum || g.alpha_zp_dev || g.row_coef || g.dq_bias) return false;
    if (g.tail != TAIL_NONE || g.bprime_from < g.N || g.y_nchw || g.y_type > 1) return false;
    if (g.Np < ((g.N + 63) & ~63)) return false;
    const uintptr_t a = (uintptr_t)g.a, y = (uintptr_t)g.y;
    if ((g.lda & 7) || (a & 7)) return false;
    if ((g.K & 15) == 0 && ((g.lda & 15) || (a & 15))) return false;
    if ((g.ldy & 15) || (y & 15)) return false;
    if (g.add_other) return false;
    return g.M > 0 && g.N > 0;
}

hipError_t launch_qgemm_direct(const GemmArgs& g, hipStream_t s) {
    auto go = [&](auto kern) {
        // resident blocks of this instantiation, computed once
        static int per_cu = 0, cus = 0;
        if (per_cu <= 0) {
            int dev = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, 0) != hipSuccess || per_cu < 1)
                per_cu = 1;
            if (hipGetDevice(&dev) != hipSuccess ||
                hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
                cus = 256;
        }
        const long long nbn = (g.N + 63) / 64, nrt = (g.M + 63) / 64;
        // waves: a multiple of the column blocks, at most the resident ones
        // and at most one per (row tile, column block)
        long long per_col = (long long)cus * per_cu * 4 / nbn;
        if (per_col > nrt) per_col = nrt;
        if (per_col < 1) per_col = 1;
        const long long waves = per_col * nbn;
        const long long blocks = (waves + 3) / 4;
        if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
        hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, s, g);
        return hipGetLastError();
    };
    if (prof_enabled()) prof_count("variant:direct");
    return go(qgemm_direct_kernel<1>);
}

hipError_t launch_qgemm_dma(const GemmArgs& g, int batch, int tile, hipStream_t s) {
    const bool conv = g.H > 0;
    if (g.kWp > 0) {
        switch (tile) {
        case TILE_128x128: return launch_dma_first<128, 128, 4>(g, batch, s);
        case TILE_256x64: return launch_dma_first<256, 64, 3>(g, batch, s);
        case TILE_64x256: return launch_dma_first<64, 256, 3>(g, batch, s);
        default: return hipErrorInvalidValue;
        }
    }
    const bool uni = conv && conv_uniform_taps(g);
    // 8-wave 256x128 tiles (2 blocks per CU, 16 waves, 3 stages; a quarter
    // fewer global->LDS bytes per MFMA op than 128x128) where N >= 256 and
    // they still give at least 384 tiles for the 512 resident blocks: fewer
    // than that leaves CUs idle, and at N = 128 the 128x128 grid balances
    // better (measured per ResNet-50 layer)
    if (tile == TILE_128x128 && g.add_other == nullptr && g.dq_bias == nullptr && g.N >= 256) {
        const long long t256 = (long long)((g.M + 255) / 256) * ((g.N + 127) / 128) * batch;
        if (t256 >= 384) tile = TILE_256x128;
    }
    if (tile == TILE_256x128) {
        if (g.add_other || g.dq_bias) tile = TILE_128x128;
        else if (!conv) return launch_dma_plain<256, 128, 3, A_DENSE>(g, batch, s);
        else return uni ? launch_dma_plain<256, 128, 3, A_CONVU>(g, batch, s)
                        : launch_dma_plain<256, 128, 3, A_CONV>(g, batch, s);
    }
    // 128-byte stages (2 stages at 2 blocks per CU) where the packed K is a
    // multiple of 128 with at least two stages per tile and, for the
    // uniform-tap producer, a step stays inside one tap. Not with a fused
    // add (its residual tile needs the LDS) nor a fused Gelu, whose long
    // fp32 epilogue hides better behind a third resident block.
    const bool wide = (g.Kp % 128) == 0 && g.Kp >= 256 && g.add_other == nullptr &&
                      !(g.dq_bias != nullptr && g.dq_gelu) && (!uni || g.C % 128 == 0);
    switch (tile) {
    case TILE_128x128:
        // 3 stages at 3 blocks per CU; the fused-add variant carries a 16 KB
        // residual tile per slot and runs 2 stages at 2 blocks per CU
        if (wide) {
            // two waves per sub-tile, each on one K half: on grids of no
            // more 128 x 128 tiles than resident 8-wave blocks (a grid of
            // 392 tiles fills 1.5 of the 4 SIMD wave slots it could use),
            // and on every uniform-tap conv grid, whose 9 or more steps per
            // tile amortize the partial-sum exchange (stage-2 3x3 layers 5 %
            // faster; dense 1x1 grids of 1568 or more tiles 3-8 % slower)
            const long long t128 = (long long)((g.M + 127) / 128) * ((g.N + 127) / 128) * batch;
            if ((t128 <= 512 || uni) && !g.add_other && !g.dq_bias && !g.row_coef && (!conv || uni) &&
                (g.epi == EPI_RQB || g.epi == EPI_RQD || g.epi == EPI_I32))
                return conv ? launch_dma_ksplit<A_CONVU>(g, batch, s) : launch_dma_ksplit<A_DENSE>(g, batch, s);
            if (!conv) return launch_dma_epi<128, 128, 2, A_DENSE, 2, 128>(g, batch, s);
            return uni ? launch_dma_epi<128, 128, 2, A_CONVU, 2, 128>(g, batch, s)
                       : launch_dma_epi<128, 128, 2, A_CONV, 2, 128>(g, batch, s);
        }
        if (!conv) return launch_dma_epi<128, 128, 3, A_DENSE, 2>(g, batch, s);
        return uni ? launch_dma_epi<128, 128, 3, A_CONVU, 2>(g, batch, s)
                   : launch_dma_epi<128, 128, 3, A_CONV, 2>(g, batch, s);
    case TILE_256x64:
        // uniform-tap convs and one-step tiles: 2 stages at 3 blocks per CU
        // (ResNet-50's stage-1 3x3 layers 17-20 % faster than 3 stages at
        // 2 blocks); dense K >= 128: 3 stages (15 % faster there)
        if (!conv)
            return g.Kp <= 64 ? launch_dma_epi<256, 64, 2, A_DENSE, 2>(g, batch, s)
                              : launch_dma_epi<256, 64, 3, A_DENSE, 2>(g, batch, s);
        return uni ? launch_dma_epi<256, 64, 2, A_CONVU, 2>(g, batch, s)
                   : launch_dma_epi<256, 64, 3, A_CONV, 2>(g, batch, s);
    case TILE_64x256:
        if (!conv) return launch_dma_epi<64, 256, 3, A_DENSE, 2>(g, batch, s);
        return uni ? launch_dma_epi<64, 256, 3, A_CONVU, 2>(g, batch, s)
                   : launch_dma_epi<64, 256, 3, A_CONV, 2>(g, batch, s);
    default:
        return hipErrorInvalidValue;
    }
}

}  // namespace nnrh
