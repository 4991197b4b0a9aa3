/*
 * nnr_vnni.c -- AVX-512 VNNI restatement of NNR's packed int8 GEMM and
 * convolution, for the CPU baseline that bench.py times beside the GPU.
 *
 * TEST INFRASTRUCTURE ONLY (see nnr_oracle.h): loaded by tests/ and by the
 * cpu_baseline leg of bench.py, never by the product path.
 *
 * What it restates (paths relative to the reference root):
 *   - the packed int8 GEMM of the VNNI conv / matmul drivers
 *     (src/backend/x64/gemm_int8_avx512.h:1000-1106, 1232-1518; the JIT
 *     micro-kernel of jit_conv_int8_ukernel.cpp): uint8 activations times
 *     int8 weights with vpdpbusd, B packed in NR = 48-column panels of
 *     4-byte K groups (3 zmm per K group), MR = 6 rows per micro-tile,
 *     MC = 48 rows per A block, the zero-point correction
 *     -x_zp * colsum[n] - w_zp * (rowsum[m] - K * x_zp) afterwards;
 *   - the implicit im2col of the conv drivers, K order (kh, kw, c)
 *     (QLinearConv_reshape.h:182-210), out-of-image taps read as x_zp;
 *   - the NHWC depthwise kernel's 16-channel int32 MAC
 *     (depthwise_int8_avx512.h:207-351, vpmulld);
 *   - the thread heuristic int8_compute_threads (src/thread_pool.h:725-737).
 * Every result is the exact int32 accumulator, so the requantize epilogues
 * of nnr_oracle.c apply unchanged and the outputs are bit-identical to the
 * scalar restatement (tests/test_oracle.py checks that on random shapes).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>
#include <immintrin.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "nnr_oracle.h"

#define VNNI_TARGET __attribute__((target("avx512f,avx512bw,avx512vl,avx512vnni")))

enum { MR = 6, NR = 48, MC = 48 };

static int g_phys = 0, g_logical = 0;

int orc_vnni_available(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vnni");
}

void orc_set_host_threads(int physical, int logical) {
    g_phys = physical;
    g_logical = logical;
}

/* src/thread_pool.h:725-737: serial below 1M ops; up to the physical cores
 * below phys x 4M ops; otherwise up to every logical thread */
int orc_int8_compute_threads(int work_items, long long total_ops) {
    int phys = g_phys > 0 ? g_phys : (int)sysconf(_SC_NPROCESSORS_ONLN);
    int logical = g_logical > 0 ? g_logical : phys;
    if (total_ops < (1LL << 20)) return 1;
    int cap = total_ops >= (long long)phys * (1LL << 22) ? logical : phys;
    if (work_items < 1) work_items = 1;
    return work_items < cap ? work_items : cap;
}

/* ---- B packing: [panel][Kp/4][48][4], column sums of (b - b_shift) ------ */
typedef struct {
    int8_t* p;       /* packed panels */
    int32_t* colsum; /* sum_k b[k][n] over the real K */
    int K, Kp, N, npanels;
} packed_b;

/* row-major B[K][N] (row stride ldb bytes), each byte ^ b_xor read as int8 */
static void pack_b(packed_b* pb, int K, int N, const void* b, long long ldb, int b_xor) {
    pb->K = K;
    pb->Kp = (K + 3) & ~3;
    pb->N = N;
    pb->npanels = (N + NR - 1) / NR;
    const size_t psz = (size_t)(pb->Kp / 4) * NR * 4;
    pb->p = (int8_t*)calloc((size_t)pb->npanels * psz, 1);
    pb->colsum = (int32_t*)calloc((size_t)pb->npanels * NR, sizeof(int32_t));
    for (int n = 0; n < N; n++) {
        const int pn = n / NR, col = n % NR;
        int32_t s = 0;
        for (int k = 0; k < K; k++) {
            int8_t v = (int8_t)(((const uint8_t*)b)[(size_t)k * ldb + n] ^ b_xor);
            pb->p[pn * psz + ((size_t)(k >> 2) * NR + col) * 4 + (k & 3)] = v;
            s += v;
        }
        pb->colsum[n] = s;
    }
}

/* conv weights [OC][C][kH][kW] in the (kh, kw, c) K order */
static void pack_b_conv(packed_b* pb, const orc_conv_params* p, const int8_t* w) {
    const int C = p->C, kH = p->kH, kW = p->kW, N = p->OC;
    const int K = kH * kW * C;
    pb->K = K;
    pb->Kp = (K + 3) & ~3;
    pb->N = N;
    pb->npanels = (N + NR - 1) / NR;
    const size_t psz = (size_t)(pb->Kp / 4) * NR * 4;
    pb->p = (int8_t*)calloc((size_t)pb->npanels * psz, 1);
    pb->colsum = (int32_t*)calloc((size_t)pb->npanels * NR, sizeof(int32_t));
    for (int n = 0; n < N; n++) {
        const int pn = n / NR, col = n % NR;
        int32_t s = 0;
        int k = 0;
        for (int a = 0; a < kH; a++)
            for (int bb = 0; bb < kW; bb++)
                for (int c = 0; c < C; c++, k++) {
                    const int8_t v = w[(((size_t)n * C + c) * kH + a) * kW + bb];
                    pb->p[pn * psz + ((size_t)(k >> 2) * NR + col) * 4 + (k & 3)] = v;
                    s += v;
                }
        pb->colsum[n] = s;
    }
}

static void free_b(packed_b* pb) {
    free(pb->p);
    free(pb->colsum);
}

/* ---- the 6 x 48 micro-kernel: c[r][0..47] = sum_k a[r][k] * b[k][n] ---
 * A rows are row-major with stride lda (a multiple of 4); each K group of a
 * row is one dword broadcast against the panel's three B vectors. */
VNNI_TARGET static void ukernel_6x48(const uint8_t* ap, long long lda, const int8_t* bp, int k4n, int rows,
                                     int32_t* c, long long ldc, int cols) {
    __m512i acc[MR][3];
    for (int r = 0; r < MR; r++)
        for (int j = 0; j < 3; j++) acc[r][j] = _mm512_setzero_si512();
    for (int k4 = 0; k4 < k4n; k4++) {
        const __m512i b0 = _mm512_loadu_si512((const void*)(bp + (size_t)k4 * NR * 4));
        const __m512i b1 = _mm512_loadu_si512((const void*)(bp + (size_t)k4 * NR * 4 + 64));
        const __m512i b2 = _mm512_loadu_si512((const void*)(bp + (size_t)k4 * NR * 4 + 128));
        const uint8_t* a4 = ap + (size_t)k4 * 4;
        for (int r = 0; r < MR; r++) {
            int32_t av;
            memcpy(&av, a4 + (size_t)r * lda, 4);
            const __m512i a = _mm512_set1_epi32(av);
            acc[r][0] = _mm512_dpbusd_epi32(acc[r][0], a, b0);
            acc[r][1] = _mm512_dpbusd_epi32(acc[r][1], a, b1);
            acc[r][2] = _mm512_dpbusd_epi32(acc[r][2], a, b2);
        }
    }
    for (int r = 0; r < rows; r++)
        for (int j = 0; j < 3; j++) {
            const int c0 = j * 16;
            if (c0 >= cols) break;
            const int m = cols - c0 >= 16 ? 16 : cols - c0;
            _mm512_mask_storeu_epi32(c + (size_t)r * ldc + c0, (__mmask16)((1u << m) - 1), acc[r][j]);
        }
}

/* One MC block of rows of C[MC][N] (row stride N) from the block's A rows,
 * row-major [MC][Kp] (rows past mc are zero): every B panel once, against
 * the block's MR-row tiles (MC = 8 x MR rows share a panel in cache). */
static void gemm_block(const uint8_t* apack, int mc, const packed_b* pb, int32_t* c) {
    const int k4n = pb->Kp / 4;
    const size_t psz = (size_t)k4n * NR * 4;
    for (int pn = 0; pn < pb->npanels; pn++) {
        const int cols = pb->N - pn * NR < NR ? pb->N - pn * NR : NR;
        for (int t = 0; t * MR < mc; t++) {
            const int rows = mc - t * MR < MR ? mc - t * MR : MR;
            ukernel_6x48(apack + (size_t)t * MR * pb->Kp, pb->Kp, pb->p + pn * psz, k4n, rows,
                         c + (size_t)t * MR * pb->N + pn * NR, pb->N, cols);
        }
    }
}

/* sum of (v - zp) over n bytes */
VNNI_TARGET static int32_t row_sum(const uint8_t* v, int n, int zp) {
    __m512i s = _mm512_setzero_si512();
    int i = 0;
    for (; i + 64 <= n; i += 64)
        s = _mm512_add_epi64(s, _mm512_sad_epu8(_mm512_loadu_si512((const void*)(v + i)), _mm512_setzero_si512()));
    long long t = _mm512_reduce_add_epi64(s);
    for (; i < n; i++) t += v[i];
    return (int32_t)(t - (long long)zp * n);
}

/* ---- packed-B cache: a model's weights are packed once, as the reference
 * packs them in reshape(); keyed by address, shape and a hash of the bytes */
typedef struct {
    const void* w;
    long long nbytes, key2;
    uint64_t hash;
    packed_b pb;
} bcache_ent;
enum { BCACHE_N = 256 };
static bcache_ent g_bcache[BCACHE_N];
static int g_bcache_n = 0;
static int g_bcache_on = 0;

void orc_vnni_cache(int on) {
    #pragma omp critical(orc_bcache)
    {
        for (int i = 0; i < g_bcache_n; i++) {
            free(g_bcache[i].pb.p);
            free(g_bcache[i].pb.colsum);
        }
        g_bcache_n = 0;
        g_bcache_on = on;
    }
}

static uint64_t bytes_hash(const void* p, long long n) {
    const uint8_t* b = (const uint8_t*)p;
    uint64_t h = 1469598103934665603ULL ^ (uint64_t)n;
    long long i = 0;
    for (; i + 8 <= n; i += 8) {
        uint64_t v;
        memcpy(&v, b + i, 8);
        h = (h ^ v) * 1099511628211ULL;
        h ^= h >> 29;
    }
    for (; i < n; i++) h = (h ^ b[i]) * 1099511628211ULL;
    return h;
}

/* a packed B from the cache, or packed now (and kept when caching is on);
 * *owned = 1 when the caller must free it */
static packed_b get_b(const void* w, long long nbytes, long long key2, int* owned,
                      void (*pack)(packed_b*, const void*, const void*), const void* arg) {
    packed_b pb;
    if (!g_bcache_on) {
        pack(&pb, w, arg);
        *owned = 1;
        return pb;
    }
    const uint64_t h = bytes_hash(w, nbytes);
    int hit = -1;
    #pragma omp critical(orc_bcache)
    {
        for (int i = 0; i < g_bcache_n; i++)
            if (g_bcache[i].w == w && g_bcache[i].nbytes == nbytes && g_bcache[i].key2 == key2 &&
                g_bcache[i].hash == h) {
                hit = i;
                break;
            }
        if (hit >= 0) pb = g_bcache[hit].pb;
    }
    if (hit >= 0) {
        *owned = 0;
        return pb;
    }
    pack(&pb, w, arg);
    *owned = 1;
    #pragma omp critical(orc_bcache)
    {
        if (g_bcache_n < BCACHE_N) {
            bcache_ent* e = &g_bcache[g_bcache_n++];
            e->w = w;
            e->nbytes = nbytes;
            e->key2 = key2;
            e->hash = h;
            e->pb = pb;
            *owned = 0;
        }
    }
    return pb;
}

static void pack_conv_cb(packed_b* pb, const void* w, const void* arg) {
    pack_b_conv(pb, (const orc_conv_params*)arg, (const int8_t*)w);
}
typedef struct { int k, n, b_xor; } mm_shape;
static void pack_mm_cb(packed_b* pb, const void* b, const void* arg) {
    const mm_shape* s = (const mm_shape*)arg;
    pack_b(pb, s->k, s->n, b, s->n, s->b_xor);
}

/* ---- convolution (group 1): exact accumulators [N][OC][oH][oW] --------- */
static int conv_vnni_ok(const orc_conv_params* p) {
    if (!orc_vnni_available() || p->group != 1) return 0;
    /* per-channel weight zero points take the reference's float path */
    for (int i = 1; i < p->w_zp_count; i++)
        if (p->w_zp[i] != p->w_zp[0]) return 0;
    return 1;
}

int orc_vnni_conv_acc(const orc_conv_params* p, const void* x, const int8_t* w, int32_t* acc) {
    return orc_vnni_conv_acc_layout(p, x, w, acc, 0);
}

int orc_vnni_conv_acc_layout(const orc_conv_params* p, const void* x, const int8_t* w, int32_t* acc,
                             int acc_nhwc) {
    if (!conv_vnni_ok(p)) return -1;
    const int N = p->N, C = p->C, H = p->H, W = p->W, OC = p->OC, kH = p->kH, kW = p->kW;
    const int oH = p->oH, oW = p->oW, sp = oH * oW;
    const int u8 = p->act_dtype == ORC_U8;
    const int shift = u8 ? 0 : 128;                 /* int8 activations as uint8 + 128 */
    const int xzu = p->x_zp + shift;                 /* zero point of the shifted values */
    const uint8_t pad = (uint8_t)xzu;
    /* w_zp through the activation type in the VNNI branches
     * (QLinearConv.cpp:386), through int8 in the float fallback (as orc_conv_acc) */
    const int8_t zb = p->w_zp_count > 0 ? p->w_zp[0] : 0;
    const int wzp = (u8 && orc_conv_dispatch(p) != ORC_BR_FLOAT) ? (int)(uint8_t)zb : (int)zb;
    int owned = 0;
    const packed_b pb = get_b(w, (long long)OC * C * kH * kW, ((long long)C << 32) | (kH << 16) | kW, &owned,
                              pack_conv_cb, p);
    const int K = pb.K, Kp = pb.Kp;
    const long long M = (long long)N * sp;
    const long long nblk = (M + MC - 1) / MC;
    const long long ops = 2LL * M * OC * K;
    const int nthr = orc_int8_compute_threads((int)(nblk < 0x7fffffff ? nblk : 0x7fffffff), ops);
    #pragma omp parallel num_threads(nthr)
    {
        uint8_t* apack = (uint8_t*)aligned_alloc(64, ((size_t)MC * Kp + 63) / 64 * 64);
        int32_t* cblk = (int32_t*)malloc(sizeof(int32_t) * (size_t)MC * OC);
        (void)K;
        int32_t* rsum = (int32_t*)malloc(sizeof(int32_t) * MC);
        #pragma omp for schedule(dynamic)
        for (long long blk = 0; blk < nblk; blk++) {
            const long long m0 = blk * MC;
            const int mc = M - m0 < MC ? (int)(M - m0) : MC;
            /* implicit im2col of the block's rows, row-major [MC][Kp]; NHWC
             * input copies each tap's C channels at once */
            for (int r = 0; r < mc; r++) {
                const long long m = m0 + r;
                const int n = (int)(m / sp), s = (int)(m % sp), oh = s / oW, ow = s % oW;
                uint8_t* row = apack + (size_t)r * Kp;
                int k = 0;
                for (int a = 0; a < kH; a++) {
                    const int ih = oh * p->sH - p->pad_t + a * p->dH;
                    for (int bb = 0; bb < kW; bb++, k += C) {
                        const int iw = ow * p->sW - p->pad_l + bb * p->dW;
                        if (ih < 0 || ih >= H || iw < 0 || iw >= W) {
                            memset(row + k, pad, (size_t)C);
                        } else if (p->x_nhwc) {
                            const uint8_t* src = (const uint8_t*)x + (((size_t)n * H + ih) * W + iw) * C;
                            if (u8) memcpy(row + k, src, (size_t)C);
                            else for (int c = 0; c < C; c++) row[k + c] = (uint8_t)(src[c] ^ 0x80);
                        } else {
                            for (int c = 0; c < C; c++)
                                row[k + c] = (uint8_t)(((const uint8_t*)x)[(((size_t)n * C + c) * H + ih) * W + iw] ^
                                                       (u8 ? 0 : 0x80));
                        }
                    }
                }
                memset(row + K, pad, (size_t)(Kp - K));
                rsum[r] = wzp ? row_sum(row, Kp, xzu) : 0;
            }
            for (int r = mc; r < ((mc + MR - 1) / MR) * MR; r++)   /* rows past the block: zero */
                memset(apack + (size_t)r * Kp, 0, (size_t)Kp);
            gemm_block(apack, mc, &pb, cblk);
            /* sum (x - x_zp)(w - w_zp) = raw - x_zp*colsum - w_zp*sum(x - x_zp)
             * (the padded taps and K padding contribute x_zp, i.e. 0) */
            for (int r = 0; r < mc; r++) {
                const long long m = m0 + r;
                const int n = (int)(m / sp), s = (int)(m % sp);
                for (int oc = 0; oc < OC; oc++) {
                    uint32_t v = (uint32_t)cblk[(size_t)r * OC + oc];
                    v -= (uint32_t)xzu * (uint32_t)pb.colsum[oc];
                    v -= (uint32_t)wzp * (uint32_t)rsum[r];
                    if (acc_nhwc) acc[(size_t)m * OC + oc] = (int32_t)v;
                    else acc[((size_t)n * OC + oc) * sp + s] = (int32_t)v;
                }
            }
        }
        free(apack);
        free(cblk);
        free(rsum);
    }
    if (owned) free_b((packed_b*)&pb);
    return 0;
}

/* ---- depthwise (NHWC, 16 channels per zmm, int32 MAC) ------------------ */
VNNI_TARGET int orc_vnni_depthwise_acc(const orc_conv_params* p, const void* x, const int8_t* w, int32_t* acc) {
    if (!orc_vnni_available() || !p->x_nhwc || p->group != p->C || p->OC != p->C) return -1;
    const int N = p->N, C = p->C, H = p->H, W = p->W, kH = p->kH, kW = p->kW;
    const int oH = p->oH, oW = p->oW, sp = oH * oW;
    const int u8 = p->act_dtype == ORC_U8;
    const int pcz = p->w_zp_count > 1;
    const int zp_as_u8 = u8 && orc_conv_dispatch(p) != ORC_BR_FLOAT;
    int32_t* wv = (int32_t*)malloc(sizeof(int32_t) * (size_t)kH * kW * ((C + 15) & ~15));
    const int Cp = (C + 15) & ~15;
    for (int t = 0; t < kH * kW; t++)
        for (int c = 0; c < Cp; c++) {
            int v = 0;
            if (c < C) {
                const int8_t zb = pcz ? p->w_zp[c] : (p->w_zp_count ? p->w_zp[0] : 0);
                const int zp = zp_as_u8 ? (int)(uint8_t)zb : (int)zb;
                v = (int)w[(size_t)c * kH * kW + t] - zp;
            }
            wv[(size_t)t * Cp + c] = v;
        }
    const long long rows = (long long)N * oH;
    const int nthr = orc_int8_compute_threads((int)rows, 2LL * N * sp * C * kH * kW);
    #pragma omp parallel for schedule(static) num_threads(nthr)
    for (long long rr = 0; rr < rows; rr++) {
        const int n = (int)(rr / oH), oh = (int)(rr % oH);
        int32_t tmp[16];
        for (int ow = 0; ow < oW; ow++) {
            for (int c0 = 0; c0 < C; c0 += 16) {
                const int cn = C - c0 < 16 ? C - c0 : 16;
                const __mmask16 mk = (__mmask16)((1u << cn) - 1);
                __m512i s = _mm512_setzero_si512();
                for (int a = 0; a < kH; a++) {
                    const int ih = oh * p->sH - p->pad_t + a * p->dH;
                    if (ih < 0 || ih >= H) continue;
                    for (int bb = 0; bb < kW; bb++) {
                        const int iw = ow * p->sW - p->pad_l + bb * p->dW;
                        if (iw < 0 || iw >= W) continue;
                        const uint8_t* src = (const uint8_t*)x + (((size_t)n * H + ih) * W + iw) * C + c0;
                        const __m128i xb = _mm_maskz_loadu_epi8(mk, src);
                        __m512i xv = u8 ? _mm512_cvtepu8_epi32(xb) : _mm512_cvtepi8_epi32(xb);
                        xv = _mm512_sub_epi32(xv, _mm512_set1_epi32(p->x_zp));
                        const __m512i wt = _mm512_loadu_si512((const void*)(wv + (size_t)(a * kW + bb) * Cp + c0));
                        s = _mm512_add_epi32(s, _mm512_mullo_epi32(xv, wt));
                    }
                }
                _mm512_storeu_si512((void*)tmp, s);
                for (int i = 0; i < cn; i++) acc[((size_t)n * C + c0 + i) * sp + oh * oW + ow] = tmp[i];
            }
        }
    }
    free(wv);
    return 0;
}

/* ---- matmul: y[b][m][n] = sum_k (a - a_zp)(b - b_zp), int32 ------------- */
int orc_vnni_matmul_integer(int batch, int m, int n, int k, const void* a, int a_dtype, long long a_bstride,
                            const void* b, int b_dtype, int a_zp, int b_zp, int32_t* y) {
    if (!orc_vnni_available()) return -1;
    const int a_shift = a_dtype == ORC_U8 ? 0 : 128;   /* A as uint8 */
    const int b_xor = b_dtype == ORC_U8 ? 0x80 : 0;    /* B as int8 (b - 128) */
    const int b_shift = b_dtype == ORC_U8 ? 128 : 0;
    const int azu = a_zp + a_shift;                     /* zero points of the shifted operands */
    const int bzs = b_zp - b_shift;
    int owned = 0;
    const mm_shape shp = {k, n, b_xor};
    const packed_b pb = get_b(b, (long long)k * n, ((long long)k << 32) | ((long long)n << 1) | (b_xor != 0),
                              &owned, pack_mm_cb, &shp);
    const int Kp = pb.Kp;
    const long long nblk = (long long)batch * ((m + MC - 1) / MC);
    const int mblk = (m + MC - 1) / MC;
    const int nthr = orc_int8_compute_threads((int)nblk, 2LL * batch * m * n * k);
    #pragma omp parallel num_threads(nthr)
    {
        uint8_t* apack = (uint8_t*)aligned_alloc(64, ((size_t)MC * Kp + 63) / 64 * 64);
        int32_t* cblk = (int32_t*)malloc(sizeof(int32_t) * (size_t)MC * n);
        int32_t* rsum = (int32_t*)malloc(sizeof(int32_t) * MC);
        #pragma omp for schedule(dynamic)
        for (long long blk = 0; blk < nblk; blk++) {
            const int bi = (int)(blk / mblk);
            const int m0 = (int)(blk % mblk) * MC;
            const int mc = m - m0 < MC ? m - m0 : MC;
            const uint8_t* ab = (const uint8_t*)a + (size_t)bi * a_bstride;
            for (int r = 0; r < ((mc + MR - 1) / MR) * MR; r++) {
                uint8_t* row = apack + (size_t)r * Kp;
                if (r >= mc) {
                    memset(row, 0, (size_t)Kp);
                    continue;
                }
                const uint8_t* src = ab + (size_t)(m0 + r) * k;
                if (a_shift) for (int kk = 0; kk < k; kk++) row[kk] = (uint8_t)(src[kk] ^ 0x80);
                else memcpy(row, src, (size_t)k);
                memset(row + k, azu, (size_t)(Kp - k));
                rsum[r] = bzs ? row_sum(row, Kp, azu) : 0;
            }
            gemm_block(apack, mc, &pb, cblk);
            /* sum (a - a_zp)(b - b_zp) = raw - azu*colsum - bzs*sum(a - a_zp) */
            for (int r = 0; r < mc; r++)
                for (int j = 0; j < n; j++) {
                    uint32_t v = (uint32_t)cblk[(size_t)r * n + j];
                    v -= (uint32_t)azu * (uint32_t)pb.colsum[j];
                    v -= (uint32_t)bzs * (uint32_t)rsum[r];
                    y[((size_t)bi * m + m0 + r) * n + j] = (int32_t)v;
                }
        }
        free(apack);
        free(cblk);
        free(rsum);
    }
    if (owned) free_b((packed_b*)&pb);
    return 0;
}
