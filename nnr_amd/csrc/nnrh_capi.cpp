// nnrh_capi.cpp -- implementation of include/nnr_hip.h.
//
// Cold path (create): validate, choose the reference's kernel branch, pack
// weights into the MFMA layout, precompute the requantize vectors with the
// same float operations as QLinearConv_reshape.h:288-336, upload.
// Hot path (run): at most a layout transform, an optional zero-point row sum
// and one GEMM / depthwise launch on the caller's stream. No allocation.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "nnr_hip.h"
#include "nnrh_elem.h"
#include "nnrh_f32.h"
#include "nnrh_internal.h"

using namespace nnrh;

namespace {

thread_local std::string g_err = "no error";

int set_err(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}
int hip_err(hipError_t e, const char* what) {
    return set_err(NNRH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}
#define HIP_TRY(expr, what)                       \
    do {                                          \
        hipError_t e__ = (expr);                  \
        if (e__ != hipSuccess) return hip_err(e__, what); \
    } while (0)

inline hipStream_t S(void* s) { return (hipStream_t)s; }
inline int round_up(int v, int m) { return (v + m - 1) / m * m; }

template <typename T>
int upload(T** dst, const T* src, size_t count) {
    *dst = nullptr;
    if (count == 0) return NNRH_OK;
    void* p = nullptr;
    HIP_TRY(hipMalloc(&p, sizeof(T) * count), "hipMalloc");
    hipError_t e = hipMemcpy(p, src, sizeof(T) * count, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(p);
        return hip_err(e, "hipMemcpy");
    }
    *dst = (T*)p;
    return NNRH_OK;
}
void dfree(void* p) {
    if (p) (void)hipFree(p);
}

// conv_shape.h:21-81 (explicit pads)
int conv_out_dim(int in, int k, int d, int s, int pb, int pe) {
    int ek = (k - 1) * d + 1;
    return (int)floorf((float)(in + pb + pe - ek) / (float)s + 1.0f);
}

// ---- launch profiler (hipEvent pairs per kernel name) ----------------------
struct ProfEntry {
    std::string name;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> ev;
    int launches = 0;
    double total_ms = 0.0;
};
struct Profiler {
    bool on = false;
    std::vector<ProfEntry> entries;
    std::vector<hipEvent_t> pool;
    hipEvent_t get() {
        if (!pool.empty()) { hipEvent_t e = pool.back(); pool.pop_back(); return e; }
        hipEvent_t e = nullptr;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        return e;
    }
    ProfEntry& entry(const char* n) {
        for (auto& e : entries) if (e.name == n) return e;
        entries.push_back(ProfEntry{});
        entries.back().name = n;
        return entries.back();
    }
    void flush() {
        for (auto& e : entries) {
            for (auto& pr : e.ev) {
                float ms = 0.f;
                (void)hipEventSynchronize(pr.second);
                if (hipEventElapsedTime(&ms, pr.first, pr.second) == hipSuccess) {
                    e.total_ms += ms;
                    e.launches++;
                }
                pool.push_back(pr.first);
                pool.push_back(pr.second);
            }
            e.ev.clear();
        }
    }
};
Profiler g_prof;

// RAII bracket around one launch
struct ProfScope {
    hipEvent_t a = nullptr, b = nullptr;
    hipStream_t s;
    const char* name;
    ProfScope(const char* n, hipStream_t st) : s(st), name(n) {
        if (!g_prof.on) return;
        a = g_prof.get();
        b = g_prof.get();
        if (a) (void)hipEventRecord(a, s);
    }
    ~ProfScope() {
        if (!a || !b) return;
        (void)hipEventRecord(b, s);
        g_prof.entry(name).ev.emplace_back(a, b);
        if (g_prof.entry(name).ev.size() > 4096) g_prof.flush();
    }
};

}  // namespace

namespace nnrh {
bool prof_enabled() { return g_prof.on; }
// a launch counted under `name` without events: which kernel instantiation
// ran (entries "variant:...")
void prof_count(const char* name) {
    if (g_prof.on) g_prof.entry(name).launches++;
}
}  // namespace nnrh

namespace {

int pick_vec(int c_or_k, int stride, uintptr_t base) {
    if (c_or_k % 16 == 0 && stride % 16 == 0 && (base & 15) == 0) return 16;
    if (c_or_k % 8 == 0 && stride % 8 == 0 && (base & 7) == 0) return 8;
    if (c_or_k % 4 == 0 && stride % 4 == 0 && (base & 3) == 0) return 4;
    return 1;
}
int pick_tile(int N) { return N <= 64 ? TILE_256x64 : TILE_128x128; }

}  // namespace

// ===========================================================================
extern "C" {

const char* nnrh_last_error(void) { return g_err.c_str(); }
const char* nnrh_version(void) { return "nnr-mi355x 0.1 (gfx950)"; }

int nnrh_device_count(int* count) {
    if (!count) return set_err(NNRH_ERR_INVALID, "count is NULL");
    HIP_TRY(hipGetDeviceCount(count), "hipGetDeviceCount");
    return NNRH_OK;
}
int nnrh_set_device(int device) {
    HIP_TRY(hipSetDevice(device), "hipSetDevice");
    return NNRH_OK;
}
int nnrh_malloc(void** p, size_t bytes) {
    if (!p) return set_err(NNRH_ERR_INVALID, "ptr is NULL");
    *p = nullptr;
    if (bytes == 0) return NNRH_OK;
    hipError_t e = hipMalloc(p, bytes);
    if (e == hipErrorOutOfMemory) return set_err(NNRH_ERR_NOMEM, "hipMalloc(%zu): out of memory", bytes);
    if (e != hipSuccess) return hip_err(e, "hipMalloc");
    return NNRH_OK;
}
int nnrh_free(void* p) {
    if (p) HIP_TRY(hipFree(p), "hipFree");
    return NNRH_OK;
}
int nnrh_memcpy(void* dst, const void* src, size_t bytes, int kind, void* stream) {
    if (bytes == 0) return NNRH_OK;
    if (!dst || !src) return set_err(NNRH_ERR_INVALID, "memcpy: NULL pointer");
    hipMemcpyKind k = kind == 0 ? hipMemcpyHostToDevice
                    : kind == 1 ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
    if (kind < 0 || kind > 2) return set_err(NNRH_ERR_INVALID, "memcpy: bad kind %d", kind);
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, k, S(stream)), "hipMemcpyAsync");
    if (kind == 1) HIP_TRY(hipStreamSynchronize(S(stream)), "hipStreamSynchronize");
    return NNRH_OK;
}
int nnrh_fill_u8(void* dst, uint8_t value, size_t bytes, void* stream) {
    if (bytes && !dst) return set_err(NNRH_ERR_INVALID, "fill: NULL pointer");
    HIP_TRY(launch_fill_u8(dst, value, (long long)bytes, S(stream)), "fill_u8");
    return NNRH_OK;
}
int nnrh_stream_create(void** s) {
    if (!s) return set_err(NNRH_ERR_INVALID, "stream is NULL");
    hipStream_t st;
    HIP_TRY(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "hipStreamCreate");
    *s = (void*)st;
    return NNRH_OK;
}
int nnrh_stream_destroy(void* s) {
    if (s) HIP_TRY(hipStreamDestroy(S(s)), "hipStreamDestroy");
    return NNRH_OK;
}
int nnrh_stream_synchronize(void* s) {
    HIP_TRY(hipStreamSynchronize(S(s)), "hipStreamSynchronize");
    return NNRH_OK;
}
int nnrh_device_synchronize(void) {
    HIP_TRY(hipDeviceSynchronize(), "hipDeviceSynchronize");
    return NNRH_OK;
}
int nnrh_event_create(void** ev) {
    if (!ev) return set_err(NNRH_ERR_INVALID, "event is NULL");
    hipEvent_t e;
    HIP_TRY(hipEventCreate(&e), "hipEventCreate");
    *ev = (void*)e;
    return NNRH_OK;
}
int nnrh_event_destroy(void* ev) {
    if (ev) HIP_TRY(hipEventDestroy((hipEvent_t)ev), "hipEventDestroy");
    return NNRH_OK;
}
int nnrh_event_record(void* ev, void* s) {
    HIP_TRY(hipEventRecord((hipEvent_t)ev, S(s)), "hipEventRecord");
    return NNRH_OK;
}
int nnrh_stream_wait_event(void* s, void* ev) {
    if (!ev) return set_err(NNRH_ERR_INVALID, "event is NULL");
    HIP_TRY(hipStreamWaitEvent(S(s), (hipEvent_t)ev, 0), "hipStreamWaitEvent");
    return NNRH_OK;
}
int nnrh_event_elapsed_ms(float* ms, void* a, void* b) {
    if (!ms) return set_err(NNRH_ERR_INVALID, "ms is NULL");
    HIP_TRY(hipEventSynchronize((hipEvent_t)b), "hipEventSynchronize");
    HIP_TRY(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b), "hipEventElapsedTime");
    return NNRH_OK;
}

}  // extern "C"

extern "C" int nnrh_profile_enable(int on) {
    g_prof.on = on != 0;
    return NNRH_OK;
}
extern "C" int nnrh_profile_enabled(void) { return g_prof.on ? 1 : 0; }

extern "C" int nnrh_graph_begin_capture(void* stream) {
    if (!stream) return set_err(NNRH_ERR_INVALID, "graph_begin_capture: the null stream cannot be captured");
    HIP_TRY(hipStreamBeginCapture(S(stream), hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    return NNRH_OK;
}
extern "C" int nnrh_graph_end_capture(void* stream, void** graph_exec) {
    if (!stream || !graph_exec) return set_err(NNRH_ERR_INVALID, "graph_end_capture: NULL argument");
    *graph_exec = nullptr;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(S(stream), &graph);
    if (e != hipSuccess || !graph) {
        if (graph) (void)hipGraphDestroy(graph);
        (void)hipGetLastError();   // a failed capture's error is not sticky here
        return hip_err(e != hipSuccess ? e : hipErrorStreamCaptureInvalidated, "hipStreamEndCapture");
    }
    hipGraphExec_t ex = nullptr;
    e = hipGraphInstantiate(&ex, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return hip_err(e, "hipGraphInstantiate");
    *graph_exec = (void*)ex;
    return NNRH_OK;
}
extern "C" int nnrh_graph_launch(void* graph_exec, void* stream) {
    if (!graph_exec) return set_err(NNRH_ERR_INVALID, "graph_launch: NULL graph");
    HIP_TRY(hipGraphLaunch((hipGraphExec_t)graph_exec, S(stream)), "hipGraphLaunch");
    return NNRH_OK;
}
extern "C" int nnrh_graph_destroy(void* graph_exec) {
    if (graph_exec) HIP_TRY(hipGraphExecDestroy((hipGraphExec_t)graph_exec), "hipGraphExecDestroy");
    return NNRH_OK;
}
extern "C" int nnrh_profile_reset(void) {
    g_prof.flush();
    g_prof.entries.clear();
    return NNRH_OK;
}
extern "C" int nnrh_profile_count(int* n) {
    if (!n) return set_err(NNRH_ERR_INVALID, "profile_count: NULL");
    g_prof.flush();
    *n = (int)g_prof.entries.size();
    return NNRH_OK;
}
extern "C" int nnrh_profile_get(int i, const char** name, int* launches, double* total_ms) {
    g_prof.flush();
    if (i < 0 || i >= (int)g_prof.entries.size() || !name || !launches || !total_ms)
        return set_err(NNRH_ERR_INVALID, "profile_get: bad index or NULL");
    *name = g_prof.entries[i].name.c_str();
    *launches = g_prof.entries[i].launches;
    *total_ms = g_prof.entries[i].total_ms;
    return NNRH_OK;
}

// ===========================================================================
// QLinearConv

namespace {

bool conv_per_channel_zp(const nnrh_qconv_desc* d) {
    // QLinearConv.cpp:136-153: an all-equal per-channel w_zp is per-tensor
    if (d->w_zp_count <= 1) return false;
    for (int i = 1; i < d->w_zp_count; ++i)
        if (d->w_zp_host[i] != d->w_zp_host[0]) return true;
    return false;
}

// First-match dispatch of QLinearConv::exec_simd_4d (QLinearConv.cpp:1337-1351)
// on an x64 AVX-512 VNNI host, with the prepack preconditions of
// QLinearConv_reshape.h:36-284.
int conv_dispatch(const nnrh_qconv_desc* d) {
    const bool u8 = d->act_dtype == NNRH_U8;
    const bool pcz = conv_per_channel_zp(d);
    const int wzp0 = d->w_zp_count > 0 ? d->w_zp_host[0] : 0;
    const int Cg = d->C / d->group;
    const bool is_dw = d->group == d->OC && Cg == 1;
    const bool vnni_ok = u8 && !pcz;
    const bool dil1 = d->dH == 1 && d->dW == 1;
    // (1) exec_dw_int8_nhwc (QLinearConv.cpp:467-526)
    if (vnni_ok && is_dw && d->y_nhwc) return NNRH_BR_DW;
    // (2) exec_first_layer_int8 (QLinearConv.cpp:665-700; reshape :233-256)
    if (vnni_ok && d->group == 1 && dil1 && Cg <= 4 && d->kH >= 3 && d->OC >= 16 && wzp0 == 0 &&
        d->C <= 4 && d->pad_t == d->pad_b && d->pad_l == d->pad_r && !d->x_nhwc)
        return NNRH_BR_FIRST;
    // (3) exec_direct_int8 (QLinearConv.cpp:579-652)
    if (vnni_ok && d->group == 1 && dil1 && wzp0 == 0 && d->oH * d->oW <= 256 && !d->y_nhwc)
        return NNRH_BR_DIRECT;
    // (4) exec_packed_nr48, NR16 predicate (QLinearConv.cpp:750-759)
    if (vnni_ok && d->group == 1) {
        if (d->kH == 3 && d->kW == 3 && d->sH == 1 && d->sW == 1 && dil1 && d->pad_t == 1 &&
            d->pad_l == 1 && d->C >= 64 && d->OC >= 64 && (d->OC % 16) == 0 && wzp0 == 0 &&
            d->y_nhwc)
            return NNRH_BR_NR16;
        return NNRH_BR_PACKED;
    }
    // (6) exec_vnni_im2col (QLinearConv.cpp:1010-1196)
    if (vnni_ok) return (d->sH == 1 && d->sW == 1) ? NNRH_BR_IM2COL_S1 : NNRH_BR_IM2COL;
    // (7) exec_float_fallback (QLinearConv.cpp:1205-1335)
    return NNRH_BR_FLOAT;
}

int validate_conv(const nnrh_qconv_desc* d) {
    if (!d) return set_err(NNRH_ERR_INVALID, "qconv: desc is NULL");
    if (d->spatial_dims != 0 && d->spatial_dims != 1 && d->spatial_dims != 2)
        return set_err(NNRH_ERR_INVALID, "qconv: spatial_dims %d", d->spatial_dims);
    if (d->spatial_dims == 1 && (d->H != 1 || d->kH != 1 || d->oH != 1 || d->sH != 1 || d->dH != 1 ||
                                 d->pad_t || d->pad_b || d->x_nhwc || d->y_nhwc))
        return set_err(NNRH_ERR_INVALID, "qconv: 1-D convolution needs H = kH = oH = 1 and NCW layouts");
    if (d->N <= 0 || d->C <= 0 || d->H <= 0 || d->W <= 0 || d->OC <= 0 || d->kH <= 0 ||
        d->kW <= 0 || d->group <= 0)
        return set_err(NNRH_ERR_INVALID, "qconv: non-positive dimension");
    if (d->C % d->group || d->OC % d->group)
        return set_err(NNRH_ERR_INVALID, "qconv: channels %d/%d not divisible by group %d", d->C,
                       d->OC, d->group);
    if (d->sH <= 0 || d->sW <= 0 || d->dH <= 0 || d->dW <= 0 || d->pad_t < 0 || d->pad_l < 0 ||
        d->pad_b < 0 || d->pad_r < 0)
        return set_err(NNRH_ERR_INVALID, "qconv: bad stride/dilation/pad");
    int oh = conv_out_dim(d->H, d->kH, d->dH, d->sH, d->pad_t, d->pad_b);
    int ow = conv_out_dim(d->W, d->kW, d->dW, d->sW, d->pad_l, d->pad_r);
    if (oh != d->oH || ow != d->oW || oh <= 0 || ow <= 0)
        return set_err(NNRH_ERR_INVALID, "qconv: output %dx%d, expected %dx%d", d->oH, d->oW, oh, ow);
    if (d->act_dtype != NNRH_U8 && d->act_dtype != NNRH_S8)
        return set_err(NNRH_ERR_UNSUPPORTED, "qconv: activation dtype %d", d->act_dtype);
    if (!d->w_host || !d->w_scale_host)
        return set_err(NNRH_ERR_INVALID, "qconv: weights / w_scale missing");
    if (d->w_scale_count != 1 && d->w_scale_count != d->OC)
        return set_err(NNRH_ERR_INVALID, "qconv: w_scale count %d (OC %d)", d->w_scale_count, d->OC);
    if (d->w_zp_count != 0 && d->w_zp_count != 1 && d->w_zp_count != d->OC)
        return set_err(NNRH_ERR_INVALID, "qconv: w_zp count %d (OC %d)", d->w_zp_count, d->OC);
    if (d->w_zp_count > 0 && !d->w_zp_host) return set_err(NNRH_ERR_INVALID, "qconv: w_zp NULL");
    if (!(d->y_scale > 0.0f) || !(d->x_scale > 0.0f))
        return set_err(NNRH_ERR_INVALID, "qconv: scales must be positive");
    long long M = (long long)d->N * d->oH * d->oW;
    if (M >= (1LL << 31) || (long long)d->N * d->H * d->W * d->C >= (1LL << 40))
        return set_err(NNRH_ERR_UNSUPPORTED, "qconv: tensor too large");
    if (d->kH * d->kW > 64 * 64) return set_err(NNRH_ERR_UNSUPPORTED, "qconv: kernel too large");
    return NNRH_OK;
}

}  // namespace

struct nnrh_qconv {
    nnrh_qconv_desc d{};
    int branch = 0;
    bool use_dw = false;         // depthwise VALU kernel
    bool dw16 = false;           // ... its dot4 variant (NHWC out, C % 16 == 0, w_zp 0)
    bool fused_add = false;      // nnrh_qconv_fuse_add was called
    bool fused_quant = false;    // nnrh_qconv_fuse_quantize was called: input is fp32
    float q_scale = 1.0f;
    int q_zp = 0;
    bool use_stem = false;       // first layer: the one-kernel stem for uint8 input ...
    bool use_stem_f32 = false;   // ... and for fp32 input with the quantize fused
    StemArgs stem{};             // its arguments but x, y and the quantize
    bool pooled = false;         // nnrh_qconv_fuse_maxpool was called: y is the pooled tensor
    StemArgs stem_pool{};        // the stem's arguments with the MaxPool fused
    int transform = 0;           // 0 none, 1 NCHW->NHWC, 2 NCHW->NHWC padded to 4 ch,
                                 // 3 first-layer padded multi-copy NHWC4 image,
                                 // 4 NHWC channels padded to a multiple of 16
    int Cx = 0;                  // channels of the tensor the kernel reads
    int groups = 1;
    bool need_rowsum = false;
    int w_zp_scalar = 0;
    int dw_L = 0, dw_tail = 0, dw_tile_h = 0;
    float inv_y = 0.f;
    int tile = 0, vec = 16;
    GemmArgs g{};
    // device buffers
    int8_t* wpack = nullptr;
    uint32_t* wdot = nullptr;    // depthwise dot4 weights [ceil(taps/4)][C]
    uint32_t* wrow3 = nullptr;   // 3x3 depthwise: per filter row {w0, w1, w2, 0} [3][C]
    bool dw3 = false;
    int32_t* colsum = nullptr;
    int32_t* c0 = nullptr;       // GEMM: per-column constant; depthwise: tap-sum correction
    int32_t* beta_col = nullptr;
    float* os = nullptr;
    float* cs = nullptr;
    float* bf = nullptr;
    int32_t* bias = nullptr;
    uint8_t* xs = nullptr;
    int32_t* rowsum = nullptr;
    int8_t* w1d = nullptr;       // 1-D: raw weights [OC][C/group][kW]
    int32_t* wzp1d = nullptr;    // 1-D: per-channel w_zp read through the activation type
    ~nnrh_qconv() {
        dfree(wpack); dfree(wdot); dfree(wrow3); dfree(colsum); dfree(c0); dfree(beta_col); dfree(os); dfree(cs); dfree(bf);
        dfree(bias); dfree(xs); dfree(rowsum); dfree(w1d); dfree(wzp1d);
    }
};

extern "C" int nnrh_qconv_dispatch(const nnrh_qconv_desc* d, int* branch) {
    int rc = validate_conv(d);
    if (rc) return rc;
    if (!branch) return set_err(NNRH_ERR_INVALID, "branch is NULL");
    // QLinearConv::exec (QLinearConv.cpp:1355-1368): non-4-D inputs go to exec_typed
    *branch = d->spatial_dims == 1 ? NNRH_BR_TYPED : conv_dispatch(d);
    return NNRH_OK;
}

namespace {
// the first layer as one kernel (nnrh_stem.hip): output rows in groups of R
// (R * oW pixels for the 4 waves' 16-pixel groups), an LDS ring of the rows
// one group reads plus the next group's, strips of groups per block
void stem_setup(nnrh_qconv_t h) {
    const nnrh_qconv_desc& d = h->d;
    const GemmArgs& g = h->g;
    StemArgs a{};
    a.w = h->wpack; a.c0 = h->c0; a.cs = h->cs; a.bf = h->bf;
    a.N = d.N; a.C = d.C; a.H = d.H; a.W = d.W; a.oH = d.oH; a.oW = d.oW;
    a.kH = d.kH; a.sH = d.sH; a.sW = d.sW; a.pad_t = d.pad_t; a.pad_l = d.pad_l;
    a.cpr = g.kWp / 4; a.Kp = g.Kp; a.KS = g.Kp / 64; a.OC = d.OC;
    a.L = round_up((d.oW - 1) * d.sW + g.kWp, 2);
    int R = std::max(1, std::min(8, 448 / std::max(1, d.oW)));
    while (R > 1 && (long long)R * d.sH * a.L > 2048) --R;
    a.R = R;
    a.WR = (R - 1) * d.sH + d.kH + R * d.sH;
    // strips of at least two groups (the rows of the next group load while
    // one computes), about 512 blocks over the batch (one round at two
    // blocks per CU: each strip pays the unpipelined fill of its first rows)
    const int groups = (d.oH + R - 1) / R;
    const int per_img = std::max(1, std::min(groups / 2, (512 + d.N - 1) / std::max(1, d.N)));
    a.strip = R * ((groups + per_img - 1) / per_img);
    a.align8 = (d.sW % 2 == 0) ? 1 : 0;
    a.sat = (g.y_type == 0 && g.L == 0 && g.hi == 255) ? 1 : 0;
    a.inv_y = g.inv_y; a.y_zp = g.y_zp; a.qmin = g.L; a.qmax = g.hi;
    a.fill = (uint32_t)(d.x_zp & 0xff);
    a.q_scale = 1.0f; a.q_inv = 1.0f; a.q_zp = 0; a.qbody = 0;
    h->stem = a;
    const bool ok = d.dH == 1 && d.dW == 1 && g.y_type == 0;
    h->use_stem = ok && stem_eligible(a, false);
    h->use_stem_f32 = ok && stem_eligible(a, true);
}
}  // namespace

extern "C" int nnrh_qconv_create(nnrh_qconv_t* out, const nnrh_qconv_desc* d) {
    if (!out) return set_err(NNRH_ERR_INVALID, "qconv: handle is NULL");
    *out = nullptr;
    int rc = validate_conv(d);
    if (rc) return rc;
    nnrh_qconv* h = new (std::nothrow) nnrh_qconv();
    if (!h) return set_err(NNRH_ERR_NOMEM, "qconv: host allocation");
    h->d = *d;
    h->d.w_host = nullptr; h->d.w_scale_host = nullptr; h->d.w_zp_host = nullptr; h->d.bias_host = nullptr;
    const int OC = d->OC, G = d->group, Cg = d->C / G, OCg = OC / G;
    const int sp = d->oH * d->oW;
    const bool u8 = d->act_dtype == NNRH_U8;
    const int lo = u8 ? 0 : -128, hi = u8 ? 255 : 127;
    const int qmin = d->post_fn ? std::max(lo, d->y_zp) : lo;     // QLinearConv.cpp:419
    const bool pcz = conv_per_channel_zp(d);
    if (d->spatial_dims == 1) {
        // exec_typed (QLinearConv.cpp:286-334): raw weights, per-channel
        // constants with the reference's float operations (:301-303)
        h->branch = NNRH_BR_TYPED;
        std::vector<float> cs1(OC), bf1(OC);
        std::vector<int32_t> wz1(OC);
        for (int oc = 0; oc < OC; ++oc) {
            const float ws = d->w_scale_count > 1 ? d->w_scale_host[oc] : d->w_scale_host[0];
            cs1[oc] = d->x_scale * ws;
            bf1[oc] = d->bias_host ? (float)d->bias_host[oc] * cs1[oc] : 0.0f;
            const int8_t zb = pcz ? d->w_zp_host[oc] : (d->w_zp_count > 0 ? d->w_zp_host[0] : 0);
            wz1[oc] = u8 ? (int32_t)(uint8_t)zb : (int32_t)zb;
        }
        const size_t wn = (size_t)OC * Cg * d->kW;
        int rc1 = upload(&h->w1d, d->w_host, wn);
        if (!rc1) rc1 = upload(&h->cs, cs1.data(), (size_t)OC);
        if (!rc1) rc1 = upload(&h->bf, bf1.data(), (size_t)OC);
        if (!rc1) rc1 = upload(&h->wzp1d, wz1.data(), (size_t)OC);
        if (rc1) { delete h; return rc1; }
        *out = h;
        return NNRH_OK;
    }
    h->branch = conv_dispatch(d);
    // The VNNI branches read w_zp through the activation type T
    // (QLinearConv.cpp:386 `(T*)inputs[5]->data`); the float fallback packs
    // weights with the weight type, int8 (QLinearConv_reshape.h:72-78).
    const bool zp_as_u8 = u8 && h->branch != NNRH_BR_FLOAT;
    auto zp_eff = [&](int8_t b) { return zp_as_u8 ? (int)(uint8_t)b : (int)b; };
    h->w_zp_scalar = d->w_zp_count > 0 ? zp_eff(d->w_zp_host[0]) : 0;
    h->groups = G;

    // ---- requantize vectors (QLinearConv_reshape.h:288-321), same float ops
    const float inv_y = 1.0f / d->y_scale;
    h->inv_y = inv_y;
    std::vector<float> cs(OC), os(OC), bf(OC);
    for (int oc = 0; oc < OC; ++oc) {
        float ws = d->w_scale_count > 1 ? d->w_scale_host[oc] : d->w_scale_host[0];
        cs[oc] = d->x_scale * ws;
        os[oc] = cs[oc] * inv_y;
        bf[oc] = d->bias_host ? (float)d->bias_host[oc] * cs[oc] : 0.0f;
    }
    std::vector<int32_t> bias(OC, 0);
    if (d->bias_host) std::copy(d->bias_host, d->bias_host + OC, bias.begin());

    // tiled im2col tile height (QLinearConv.cpp:1082-1090)
    int tile_h = d->oH;
    {
        const size_t TILE_BYTES = 256 * 1024;
        size_t CHW = (size_t)Cg * d->kH * d->kW;
        if (CHW * (size_t)sp > TILE_BYTES) {
            long th = (long)(TILE_BYTES / (CHW * (size_t)d->oW));
            tile_h = (int)std::max(1L, th);
            tile_h = std::min(tile_h, d->oH);
        }
    }

    const int br = h->branch;
    const bool is_dw = (G == OC && Cg == 1);
    h->use_dw = is_dw && u8 && !pcz &&
                (br == NNRH_BR_DW || br == NNRH_BR_IM2COL_S1 || br == NNRH_BR_IM2COL);

    auto fail = [&](int code) { delete h; return code; };

    if (h->use_dw) {
        if ((rc = upload(&h->cs, cs.data(), OC))) return fail(rc);
        if ((rc = upload(&h->bf, bf.data(), OC))) return fail(rc);
        // repack_depthwise_weights: [kH*kW][C]
        std::vector<int8_t> wdw((size_t)d->kH * d->kW * OC);
        for (int c = 0; c < OC; ++c)
            for (int t = 0; t < d->kH * d->kW; ++t) wdw[(size_t)t * OC + c] = d->w_host[(size_t)c * d->kH * d->kW + t];
        if ((rc = upload(&h->wpack, wdw.data(), wdw.size()))) return fail(rc);
        h->transform = d->x_nhwc ? 0 : 1;
        h->Cx = d->C;
        h->dw_L = (br == NNRH_BR_IM2COL) ? qmin : lo;
        h->dw_tail = (br == NNRH_BR_IM2COL) ? TAIL_TILED : TAIL_NONE;
        h->dw_tile_h = tile_h;
        // dot4 kernel: NHWC out without tails, 16-channel chunks, w_zp 0
        const int taps = d->kH * d->kW;
        h->dw16 = h->dw_tail == TAIL_NONE && d->y_nhwc && OC % 16 == 0 && OC <= 4096 &&
                  h->w_zp_scalar == 0 && taps <= 12;
        if (h->dw16) {
            const int G4 = (taps + 3) / 4;
            std::vector<uint32_t> wdot((size_t)G4 * OC, 0u);
            std::vector<int32_t> corr(OC, 0);
            // sum (x - x_zp) w = sum (x ^ 0x80) w + (128 - x_zp) sum w   (uint8)
            const uint32_t k = (uint32_t)((u8 ? 128 : 0) - d->x_zp);
            for (int c = 0; c < OC; ++c) {
                uint32_t sw = 0;
                for (int t = 0; t < taps; ++t) {
                    const int8_t v = d->w_host[(size_t)c * taps + t];
                    wdot[(size_t)(t / 4) * OC + c] |= (uint32_t)(uint8_t)v << (8 * (t % 4));
                    sw += (uint32_t)(int32_t)v;
                }
                corr[c] = (int32_t)(k * sw);
            }
            if ((rc = upload(&h->wdot, wdot.data(), wdot.size()))) return fail(rc);
            if ((rc = upload(&h->c0, corr.data(), corr.size()))) return fail(rc);
            // 3x3, stride 1 or 2, dilation 1: one dot4 per filter row
            h->dw3 = d->kH == 3 && d->kW == 3 && d->dH == 1 && d->dW == 1 && d->sH == d->sW &&
                     (d->sH == 1 || d->sH == 2);
            if (h->dw3) {
                std::vector<uint32_t> wrow((size_t)3 * OC, 0u);
                for (int c = 0; c < OC; ++c)
                    for (int t = 0; t < 9; ++t)
                        wrow[(size_t)(t / 3) * OC + c] |= (uint32_t)(uint8_t)d->w_host[(size_t)c * 9 + t]
                                                          << (8 * (t % 3));
                if ((rc = upload(&h->wrow3, wrow.data(), wrow.size()))) return fail(rc);
            }
        }
    } else {
        // ---- GEMM plan: groups on blockIdx.z, K order (kh, kw, c); every
        // per-column array is laid out [G][Np] (zero padded)
        const bool first = br == NNRH_BR_FIRST;
        // channel counts that are not a multiple of 16: the kernel reads a
        // copy padded with x_zp to the next multiple of 16 (zero weights
        // there, so the accumulators are unchanged) and keeps 16-byte loads
        // (not for a 1x1 stride-1 NHWC conv with C % 8 == 0 and C <= 64: the
        // short-K direct kernel reads its rows in 8-byte pieces as they are)
        const bool dense1x1 = d->kH == 1 && d->kW == 1 && d->sH == 1 && d->sW == 1 && d->pad_t == 0 &&
                              d->pad_l == 0 && d->pad_b == 0 && d->pad_r == 0 && d->oH == d->H && d->oW == d->W;
        const bool direct_rows = dense1x1 && d->x_nhwc && Cg % 8 == 0 && Cg <= 64 &&
                                 (br == NNRH_BR_PACKED || br == NNRH_BR_NR16);
        const bool cpad = !first && G == 1 && Cg % 16 != 0 && !direct_rows;
        const int Cgp = first ? 4 : (cpad ? round_up(Cg, 16) : Cg);
        const int kWp = first ? round_up(d->kW, 4) : d->kW;   // first layer: taps padded to 4
        const int K = d->kH * kWp * Cgp;
        const int Kp = round_up(K, 64);
        const int Np = round_up(OCg, 64);
        const int a_sub = u8 ? 128 : 0;
        const int alpha = d->x_zp - a_sub;
        const bool rqb = br == NNRH_BR_PACKED || br == NNRH_BR_NR16;
        std::vector<int8_t> wp((size_t)G * Np * Kp, 0);
        std::vector<int32_t> colsum((size_t)G * Np, 0), c0((size_t)G * Np, 0), biasp((size_t)G * Np, 0),
            betac((size_t)G * Np, 0);
        std::vector<float> osp((size_t)G * Np, 0.f), csp((size_t)G * Np, 0.f), bfp((size_t)G * Np, 0.f);
        bool any_wzp = false;
        for (int g = 0; g < G; ++g)
            for (int n = 0; n < OCg; ++n) {
                const int oc = g * OCg + n;
                const size_t pi = (size_t)g * Np + n;
                int8_t* row = wp.data() + ((size_t)g * Np + packed_row_of_col(n)) * Kp;
                int32_t s = 0;
                for (int c = 0; c < Cg; ++c)
                    for (int a = 0; a < d->kH; ++a)
                        for (int b = 0; b < d->kW; ++b) {
                            int8_t v = d->w_host[(((size_t)oc * Cg + c) * d->kH + a) * d->kW + b];
                            row[(a * kWp + b) * Cgp + c] = v;
                            s += v;
                        }
                colsum[pi] = s;
                biasp[pi] = bias[oc];
                // c0 = (RQ-B: bias) - alpha * colsum, int32 wrap-around
                uint32_t t = (uint32_t)(rqb ? bias[oc] : 0) - (uint32_t)alpha * (uint32_t)s;
                c0[pi] = (int32_t)t;
                osp[pi] = os[oc]; csp[pi] = cs[oc]; bfp[pi] = bf[oc];
                betac[pi] = pcz ? zp_eff(d->w_zp_host[oc]) : h->w_zp_scalar;
                any_wzp |= betac[pi] != 0;
            }
        for (int32_t v : c0) h->g.c0_absmax = std::max(h->g.c0_absmax, std::llabs((long long)v));
        if ((rc = upload(&h->wpack, wp.data(), wp.size()))) return fail(rc);
        if ((rc = upload(&h->colsum, colsum.data(), colsum.size()))) return fail(rc);
        if ((rc = upload(&h->c0, c0.data(), c0.size()))) return fail(rc);
        if ((rc = upload(&h->os, osp.data(), osp.size()))) return fail(rc);
        if ((rc = upload(&h->cs, csp.data(), csp.size()))) return fail(rc);
        if ((rc = upload(&h->bf, bfp.data(), bfp.size()))) return fail(rc);
        if ((rc = upload(&h->bias, biasp.data(), biasp.size()))) return fail(rc);
        h->need_rowsum = any_wzp;
        if (any_wzp && (rc = upload(&h->beta_col, betac.data(), betac.size()))) return fail(rc);

        // first layer with NHWC output: padded multi-copy image for the
        // pipelined kernel (its epilogue has no scalar tails then)
        const bool first_copies = first && d->y_nhwc && G == 1;
        if (first_copies) { h->transform = 3; h->Cx = 4; }
        else if (first) { h->transform = 2; h->Cx = 4; }
        else if (cpad) { h->transform = d->x_nhwc ? 4 : 1; h->Cx = Cgp; }
        else { h->transform = d->x_nhwc ? 0 : 1; h->Cx = d->C; }

        GemmArgs& g = h->g;
        g.a_xor = u8 ? 0x80 : 0;
        g.M = d->N * sp;
        g.N = OCg;
        g.K = K;
        g.Kp = Kp;
        g.H = d->H; g.W = d->W; g.C = Cgp; g.Cs = h->Cx;
        g.oH = d->oH; g.oW = d->oW; g.kH = d->kH; g.kW = d->kW;
        g.sH = d->sH; g.sW = d->sW; g.dH = d->dH; g.dW = d->dW;
        g.pad_t = d->pad_t; g.pad_l = d->pad_l;
        g.kWp = first ? kWp : 0;
        g.pad_byte = d->x_zp & 0xff;
        if (first_copies) {
            // pads folded into the image; rows long enough for the last
            // chunk of kWp taps; copies for every start-pixel residue mod 4
            const int Hp = std::max(d->H + d->pad_t + d->pad_b, (d->oH - 1) * d->sH + d->kH);
            const int Wc = round_up(std::max(d->W + d->pad_l + d->pad_r, (d->oW - 1) * d->sW + kWp), 4);
            g.H = Hp; g.W = Wc;
            g.pad_t = 0; g.pad_l = 0;
            g.copy_shift = (d->sW % 4 == 0) ? 2 : (d->sW % 2 == 0 ? 1 : 0);
            g.copy_stride = (long long)d->N * Hp * Wc * 4;
        }
        g.a_bstride = first ? 0 : Cg;   // group channel offset
        // a 1x1 stride-1 unpadded conv over NHWC is a plain GEMM: row m is
        // pixel m, row stride = channel stride (no tap decode, no bounds)
        if (!first && d->kH == 1 && d->kW == 1 && d->sH == 1 && d->sW == 1 && d->pad_t == 0 &&
            d->pad_l == 0 && d->pad_b == 0 && d->pad_r == 0 && d->oH == d->H && d->oW == d->W) {
            g.H = 0;
            g.lda = h->Cx;
        }
        g.b = h->wpack;
        g.b_bstride = (long long)Np * Kp;
        g.Np = Np;
        g.colsum = h->colsum;
        g.c0 = h->c0;
        g.a_sub = a_sub;
        g.alpha = alpha;
        g.rowsum_bstride = (long long)g.M;
        g.beta_col = h->beta_col;
        g.beta = 0;
        g.param_bstride = Np;
        g.os = h->os; g.bias = h->bias; g.cs = h->cs; g.bf = h->bf;
        g.inv_y = inv_y;
        g.y_zp = d->y_zp;
        g.lo = lo; g.hi = hi;
        g.bprime_from = OCg;
        g.tile_h = tile_h;
        g.y_type = u8 ? 0 : 1;
        g.y_nchw = d->y_nhwc ? 0 : 1;
        g.ldy = OC;
        g.y_bstride = d->y_nhwc ? OCg : (long long)OCg * sp;
        switch (br) {
        case NNRH_BR_FIRST:
            g.epi = EPI_RQC; g.L = qmin; g.tail = d->y_nhwc ? TAIL_NONE : TAIL_OW; break;
        case NNRH_BR_DIRECT:
        case NNRH_BR_FLOAT:
            g.epi = EPI_RQA; g.L = qmin; g.tail = TAIL_SPATIAL; break;
        case NNRH_BR_PACKED:
            g.epi = EPI_RQB;
            // RQ-B' on the third sub-panel of a partial NR48 block
            g.bprime_from = (OCg % 48 > 32) ? OCg - OCg % 48 + 32 : OCg;
            break;
        case NNRH_BR_NR16:
            g.epi = EPI_RQB; break;
        case NNRH_BR_IM2COL_S1:
            g.epi = EPI_RQA; g.L = lo; g.tail = TAIL_NONE; break;
        case NNRH_BR_IM2COL:
            g.epi = EPI_RQA; g.L = qmin; g.tail = TAIL_TILED; break;
        default:
            return fail(set_err(NNRH_ERR_UNSUPPORTED, "qconv: branch %d", br));
        }
        h->tile = pick_tile(OCg);
        h->vec = (h->Cx % 4 == 0 && Cgp % 4 == 0) ? pick_vec(Cgp, h->Cx, 0) : 1;
        if (G > 1 && (Cg % h->vec)) h->vec = 1;
        if (first_copies) stem_setup(h);
    }
    // scratch: transformed input and row sums (the stem kernel reads the
    // image itself)
    if (h->transform == 3 && !h->use_stem && !h->use_stem_f32) {
        size_t bytes = (size_t)(4 >> h->g.copy_shift) * (size_t)h->g.copy_stride;
        if ((rc = nnrh_malloc((void**)&h->xs, bytes))) return fail(rc);
    } else if (h->transform) {
        size_t bytes = (size_t)d->N * d->H * d->W * h->Cx;
        if ((rc = nnrh_malloc((void**)&h->xs, bytes))) return fail(rc);
    }
    if (h->need_rowsum) {
        if ((rc = nnrh_malloc((void**)&h->rowsum, sizeof(int32_t) * (size_t)d->N * sp * G)))
            return fail(rc);
        h->g.rowsum = h->rowsum;
    }
    *out = h;
    return NNRH_OK;
}

extern "C" int nnrh_qconv_branch(nnrh_qconv_t h, int* branch) {
    if (!h || !branch) return set_err(NNRH_ERR_INVALID, "qconv_branch: NULL");
    *branch = h->branch;
    return NNRH_OK;
}

namespace {
// everything after the input transform (src: the kernel's input image)
int qconv_compute(nnrh_qconv_t h, const uint8_t* src, void* y, hipStream_t s);
}  // namespace

namespace {
// the stem kernel's 16-byte output stores need an aligned output
bool stem_ok(nnrh_qconv_t h, const void* x, const void* y) {
    return ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0 && !h->fused_add;
}

// the multi-copy image of the two-kernel first layer, allocated when a
// stem-eligible layer is first run the other way (misaligned output)
int stem_scratch(nnrh_qconv_t h) {
    if (h->transform != 3 || h->xs) return NNRH_OK;
    const size_t bytes = (size_t)(4 >> h->g.copy_shift) * (size_t)h->g.copy_stride;
    return nnrh_malloc((void**)&h->xs, bytes);
}

int run_stem(nnrh_qconv_t h, const void* x, void* y, bool f32, hipStream_t s) {
    const nnrh_qconv_desc& d = h->d;
    StemArgs a = h->pooled ? h->stem_pool : h->stem;
    a.x = x;
    a.y = (uint8_t*)y;
    if (f32) {
        // QuantizeLinear over the whole [N, C, H, W] tensor: 16-wide body,
        // scalar tail (the last n % 16 elements; all of them below 64)
        const long long qn = (long long)d.N * d.C * d.H * d.W;
        a.q_scale = h->q_scale;
        a.q_inv = 1.0f / h->q_scale;
        a.q_zp = h->q_zp;
        a.qbody = qn >= 64 ? qn - qn % 16 : 0;
    }
    ProfScope ps(h->pooled ? "stem_conv_maxpool" : "stem_conv", s);
    HIP_TRY(launch_stem_conv(a, f32, s), "stem_conv");
    return NNRH_OK;
}

// the pooled stem has no other path: aligned buffers or an error
int run_pooled(nnrh_qconv_t h, const void* x, void* y, bool f32, hipStream_t s) {
    if (!stem_ok(h, x, y))
        return set_err(NNRH_ERR_INVALID, "qconv: with the MaxPool fused, x and y must be 16-byte aligned");
    return run_stem(h, x, y, f32, s);
}
}  // namespace

extern "C" int nnrh_qconv_run(nnrh_qconv_t h, const void* x, void* y, void* stream) {
    if (!h || !x || !y) return set_err(NNRH_ERR_INVALID, "qconv_run: NULL argument");
    if (h->fused_quant) return set_err(NNRH_ERR_INVALID, "qconv_run: quantize fused, use nnrh_qconv_run_f32");
    const nnrh_qconv_desc& d = h->d;
    hipStream_t s = S(stream);
    const uint8_t* src = (const uint8_t*)x;
    if (h->pooled) return run_pooled(h, x, y, false, s);
    if (h->use_stem && stem_ok(h, x, y)) return run_stem(h, x, y, false, s);
    if (h->transform == 3) {
        if (int rc = stem_scratch(h)) return rc;
        ProfScope ps("first_layer_copies", s);
        HIP_TRY(launch_first_layer_copies(src, h->xs, d.N, d.C, d.H, d.W, h->g.H, h->g.W, d.pad_t,
                                          d.pad_l, h->g.copy_shift, (uint8_t)(d.x_zp & 0xff), s),
                "first_layer_copies");
        src = h->xs;
    } else if (h->transform == 4) {
        ProfScope ps("pad_channels_u8", s);
        HIP_TRY(launch_pad_channels_u8(src, h->xs, (long long)d.N * d.H * d.W, d.C, h->Cx,
                                       (uint8_t)(d.x_zp & 0xff), s),
                "pad_channels");
        src = h->xs;
    } else if (h->transform) {
        ProfScope ps("nchw_to_nhwc_u8", s);
        HIP_TRY(launch_nchw_to_nhwc_u8(src, h->xs, d.N, d.C, d.H * d.W, h->Cx,
                                       (uint8_t)(d.x_zp & 0xff), s),
                "nchw_to_nhwc");
        src = h->xs;
    }
    return qconv_compute(h, src, y, s);
}

extern "C" int nnrh_qconv_fuse_quantize(nnrh_qconv_t h, float scale, int zp) {
    if (!h) return set_err(NNRH_ERR_INVALID, "qconv_fuse_quantize: NULL handle");
    if (!(scale > 0.0f) || zp < 0 || zp > 255)
        return set_err(NNRH_ERR_INVALID, "qconv_fuse_quantize: scale %g / zero point %d", (double)scale, zp);
    if (h->transform != 3 || h->d.act_dtype != NNRH_U8 || h->fused_add ||
        h->g.W + ((4 >> h->g.copy_shift) - 1) * (1 << h->g.copy_shift) > 4096)
        return set_err(NNRH_ERR_UNSUPPORTED, "qconv_fuse_quantize: only the first layer's multi-copy input");
    if (h->pooled && !stem_eligible(h->stem_pool, true))
        return set_err(NNRH_ERR_UNSUPPORTED, "qconv_fuse_quantize: the pooled first layer has no fp32-input kernel here");
    h->fused_quant = true;
    h->q_scale = scale;
    h->q_zp = zp;
    return NNRH_OK;
}

extern "C" int nnrh_qconv_run_f32(nnrh_qconv_t h, const float* x, void* y, void* stream) {
    if (!h || !x || !y) return set_err(NNRH_ERR_INVALID, "qconv_run_f32: NULL argument");
    if (!h->fused_quant) return set_err(NNRH_ERR_INVALID, "qconv_run_f32: nnrh_qconv_fuse_quantize was not called");
    const nnrh_qconv_desc& d = h->d;
    hipStream_t s = S(stream);
    if (h->pooled) return run_pooled(h, x, y, true, s);
    if (h->use_stem_f32 && stem_ok(h, x, y)) return run_stem(h, x, y, true, s);
    if (int rc = stem_scratch(h)) return rc;
    {
        ProfScope ps("quantize_first_layer_copies", s);
        HIP_TRY(launch_quantize_first_layer_copies(x, h->xs, d.N, d.C, d.H, d.W, h->g.H, h->g.W, d.pad_t,
                                                   d.pad_l, h->g.copy_shift, (uint8_t)(d.x_zp & 0xff),
                                                   h->q_scale, h->q_zp, s),
                "quantize_first_layer_copies");
    }
    return qconv_compute(h, h->xs, y, s);
}

namespace {
int qconv_compute(nnrh_qconv_t h, const uint8_t* src, void* y, hipStream_t s) {
    const nnrh_qconv_desc& d = h->d;
    if (h->branch == NNRH_BR_TYPED) {
        ProfScope ps("conv1d_typed", s);
        HIP_TRY(launch_conv1d_typed(src, h->w1d, h->wzp1d, h->cs, h->bf, (uint8_t*)y, d.N, d.C, d.W, d.OC,
                                    d.group, d.kW, d.oW, d.sW, d.dW, d.pad_l, d.x_zp, d.y_zp, d.y_scale,
                                    d.act_dtype == NNRH_U8, s),
                "conv1d_typed");
        return NNRH_OK;
    }
    if (h->use_dw && h->dw3) {
        ProfScope ps("depthwise", s);
        HIP_TRY(launch_depthwise3x3(src, h->wrow3, h->c0, (uint8_t*)y, h->cs, h->bf, d.N, d.C, d.H, d.W, d.oH,
                                    d.oW, d.sH, d.pad_t, d.pad_l, d.x_zp, d.act_dtype == NNRH_U8 ? 0x80 : 0,
                                    h->inv_y, d.y_zp, h->dw_L, d.act_dtype == NNRH_U8 ? 255 : 127, s),
                "depthwise3x3");
        return NNRH_OK;
    }
    if (h->use_dw && h->dw16) {
        ProfScope ps("depthwise", s);
        HIP_TRY(launch_depthwise16(src, h->wdot, h->c0, (uint8_t*)y, h->cs, h->bf, d.N, d.C, d.H, d.W,
                                   d.oH, d.oW, d.kH, d.kW, d.sH, d.sW, d.dH, d.dW, d.pad_t, d.pad_l,
                                   d.x_zp, d.act_dtype == NNRH_U8 ? 0x80 : 0, h->inv_y, d.y_zp,
                                   h->dw_L, d.act_dtype == NNRH_U8 ? 255 : 127, s),
                "depthwise16");
        return NNRH_OK;
    }
    if (h->use_dw) {
        ProfScope ps("depthwise", s);
        HIP_TRY(launch_depthwise(src, h->wpack, (uint8_t*)y, h->cs, h->bf, d.N, d.C, d.H, d.W, d.oH,
                                 d.oW, d.kH, d.kW, d.sH, d.sW, d.dH, d.dW, d.pad_t, d.pad_l, d.x_zp,
                                 h->w_zp_scalar, h->inv_y, d.y_zp, h->dw_L, d.act_dtype == NNRH_U8 ? 255 : 127,
                                 d.act_dtype == NNRH_S8, d.y_nhwc ? 0 : 1, h->dw_tail, h->dw_tile_h, s),
                "depthwise");
        return NNRH_OK;
    }
    if (h->need_rowsum) {
        const int Cg = h->g.C;
        ProfScope ps("rowsum", s);
        HIP_TRY(launch_rowsum_conv(src, d.N, d.H, d.W, h->Cx, Cg, Cg, h->groups, d.oH, d.oW, d.kH, d.kW,
                                   d.sH, d.sW, d.dH, d.dW, d.pad_t, d.pad_l, d.act_dtype == NNRH_S8,
                                   d.x_zp, h->rowsum, (long long)d.N * d.oH * d.oW, s),
                "rowsum_conv");
    }
    GemmArgs g = h->g;
    g.a = src;
    g.y = y;
    int vec = h->vec;
    if (vec > 1 && ((uintptr_t)src & (vec - 1))) vec = 1;
    ProfScope ps("qgemm", s);
    HIP_TRY(launch_qgemm(g, h->groups, h->tile, vec, s), "qgemm");
    return NNRH_OK;
}
}  // namespace

extern "C" int nnrh_qconv_fuse_maxpool(nnrh_qconv_t h, int kH, int kW, int sH, int sW, int pad_t, int pad_l,
                                       int pad_b, int pad_r) {
    if (!h) return set_err(NNRH_ERR_INVALID, "qconv_fuse_maxpool: NULL handle");
    if (kH != 3 || kW != 3 || sH != 2 || sW != 2 || pad_t != 1 || pad_l != 1 || pad_b != 1 || pad_r != 1)
        return set_err(NNRH_ERR_UNSUPPORTED, "qconv_fuse_maxpool: only 3x3 windows, stride 2, padding 1");
    if (h->pooled) return set_err(NNRH_ERR_INVALID, "qconv_fuse_maxpool: already fused");
    if (h->fused_add || !(h->use_stem || h->use_stem_f32))
        return set_err(NNRH_ERR_UNSUPPORTED, "qconv_fuse_maxpool: only the one-kernel first layer");
    const nnrh_qconv_desc& d = h->d;
    // groups of 4 conv rows (2 pooled rows), a ring of one group's span;
    // strips of pooled rows: about 512 blocks over the batch
    StemArgs a = h->stem;
    a.pool = 1;
    a.R = 4;
    a.WR = (a.R - 1) * d.sH + d.kH;
    a.pH = (d.oH - 1) / 2 + 1;
    a.pW = (d.oW - 1) / 2 + 1;
    const int groups = (a.pH + 1) / 2;
    const int per_img = std::max(1, std::min(std::max(1, groups / 2), (512 + d.N - 1) / std::max(1, d.N)));
    a.strip = 2 * ((groups + per_img - 1) / per_img);
    if (!stem_eligible(a, h->fused_quant))
        return set_err(NNRH_ERR_UNSUPPORTED, "qconv_fuse_maxpool: this first layer does not fit the pooled kernel");
    h->stem_pool = a;
    h->pooled = true;
    return NNRH_OK;
}

extern "C" int nnrh_qconv_fuse_add(nnrh_qconv_t h, const nnrh_qadd_fuse_desc* a) {
    if (!h || !a) return set_err(NNRH_ERR_INVALID, "qconv_fuse_add: NULL argument");
    const nnrh_qconv_desc& d = h->d;
    GemmArgs g = h->g;
    const bool rqb = h->branch == NNRH_BR_PACKED || h->branch == NNRH_BR_NR16;
    // the residual tile travels in 16-byte chunks of whole output rows;
    // uint8 output only (the kernel's fused path is the unsigned one)
    if (h->use_dw || h->transform == 3 || h->groups != 1 || !d.y_nhwc || !rqb || g.ldy != g.N ||
        (g.N % 16) != 0 || g.y_type != 0 || !qgemm_dma_eligible(g, h->vec))
        return set_err(NNRH_ERR_UNSUPPORTED, "qconv_fuse_add: this convolution's kernel has no fused add");
    // QLinearAdd.cpp:46-47,66-67 (no contraction), as nnrh_qlinear_add
    g.add_sa = a->a_scale / a->y_scale;
    g.add_sb = a->b_scale / a->y_scale;
    {
        float t1 = g.add_sa * (float)a->a_zp, t2 = g.add_sb * (float)a->b_zp;
        g.add_fixed = (float)a->y_zp - (t1 + t2);
    }
    g.add_a_zp = a->a_zp; g.add_b_zp = a->b_zp; g.add_y_zp = a->y_zp;
    // the kernel's body path needs |fma(a,sa,fma(b,sb,fixed))| < 2^22 for
    // every byte pair (then clamp-then-round is exact); otherwise no fusion
    {
        const double amax = d.act_dtype == NNRH_U8 ? 255.0 : 128.0;
        const double bound = amax * (std::fabs((double)g.add_sa) + std::fabs((double)g.add_sb)) +
                             std::fabs((double)g.add_fixed) + 2.0;
        if (!(bound < 4194304.0))
            return set_err(NNRH_ERR_UNSUPPORTED, "qconv_fuse_add: add scales out of the fused range");
    }
    g.add_conv_is_a = a->conv_is_a ? 1 : 0;
    const long long n = (long long)d.N * d.oH * d.oW * d.OC;
    g.add_body = n - n % 16;
    h->g = g;
    h->fused_add = true;
    return NNRH_OK;
}

extern "C" int nnrh_qconv_run_add(nnrh_qconv_t h, const void* x, const void* other, void* y, void* stream) {
    if (!h || !x || !other || !y) return set_err(NNRH_ERR_INVALID, "qconv_run_add: NULL argument");
    if (!h->fused_add) return set_err(NNRH_ERR_INVALID, "qconv_run_add: nnrh_qconv_fuse_add was not called");
    const nnrh_qconv_desc& d = h->d;
    hipStream_t s = S(stream);
    const uint8_t* src = (const uint8_t*)x;
    if (h->transform == 4) {
        ProfScope ps("pad_channels_u8", s);
        HIP_TRY(launch_pad_channels_u8(src, h->xs, (long long)d.N * d.H * d.W, d.C, h->Cx,
                                       (uint8_t)(d.x_zp & 0xff), s),
                "pad_channels");
        src = h->xs;
    } else if (h->transform) {
        ProfScope ps("nchw_to_nhwc_u8", s);
        HIP_TRY(launch_nchw_to_nhwc_u8(src, h->xs, d.N, d.C, d.H * d.W, h->Cx,
                                       (uint8_t)(d.x_zp & 0xff), s),
                "nchw_to_nhwc");
        src = h->xs;
    }
    if (((uintptr_t)src & 15) != 0)
        return set_err(NNRH_ERR_INVALID, "qconv_run_add: input must be 16-byte aligned");
    if (((uintptr_t)other & 15) != 0)
        return set_err(NNRH_ERR_INVALID, "qconv_run_add: other must be 16-byte aligned");
    GemmArgs g = h->g;
    g.a = src;
    g.y = y;
    g.add_other = (const uint8_t*)other;
    ProfScope ps("qgemm_add", s);
    HIP_TRY(launch_qgemm(g, 1, h->tile, h->vec, s), "qgemm_add");
    return NNRH_OK;
}

extern "C" int nnrh_qconv_destroy(nnrh_qconv_t h) {
    delete h;
    return NNRH_OK;
}

// ===========================================================================
// QLinearMatMul (constant B)

namespace {
uint16_t f32_to_f16(float v) {   // src/nnrconf.h:147-173 rounding
    uint32_t u; memcpy(&u, &v, 4);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    int e = (int)((u >> 23) & 0xffu) - 127;
    uint32_t mant = u & 0x7fffffu;
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    if (e >= -14) {
        uint32_t rb = mant & 0x1fffu;
        uint16_t y = (uint16_t)(sign | ((uint16_t)(e + 15) << 10) | (uint16_t)(mant >> 13));
        if (rb > 0x1000u || (rb == 0x1000u && (y & 1u))) y++;
        return y;
    }
    if (e >= -24) {
        mant |= 0x800000u;
        int sh = -e - 14 + 13;
        uint32_t rb = mant & ((1u << sh) - 1u);
        uint32_t half = 1u << (sh - 1);
        uint16_t y = (uint16_t)(sign | (uint16_t)(mant >> sh));
        if (rb > half || (rb == half && (y & 1u))) y++;
        return y;
    }
    return sign;
}
float f16_to_f32(uint16_t v) {   // src/nnrconf.h:175-199
    uint32_t sign = (uint32_t)(v & 0x8000u) << 16, e = (v >> 10) & 0x1fu, mant = v & 0x3ffu, u;
    if (e == 0) {
        if (mant == 0) u = sign;
        else {
            int ee = 0;
            while (!(mant & 0x400u)) { mant <<= 1; ee--; }
            mant &= 0x3ffu; ee++;
            u = sign | ((uint32_t)(ee + 127 - 15) << 23) | (mant << 13);
        }
    } else if (e == 31) u = sign | 0x7f800000u | (mant << 13);
    else u = sign | ((e + 127 - 15) << 23) | (mant << 13);
    float f; memcpy(&f, &u, 4);
    return f;
}
int ld_zp(const void* p, int dt) {
    if (!p) return 0;
    return dt == NNRH_U8 ? (int)*(const uint8_t*)p : (int)*(const int8_t*)p;
}
}  // namespace

struct nnrh_qmatmul {
    nnrh_qmatmul_desc d{};
    GemmArgs g{};
    int8_t* wpack = nullptr;
    int32_t* colsum = nullptr;
    int32_t* c0 = nullptr;
    int32_t* rowsum = nullptr;
    float* dq_bias = nullptr;   // nnrh_qmatmul_fuse_dq_bias: padded to Np
    float* colscale = nullptr;  // nnrh_matmul_integer_scaled_create: w_scale, padded to Np
    int rowsum_cap = 0;     // batches the rowsum buffer holds
    int parts_cap = 0;      // nnrh_qmatmul_set_minmax_out: pairs the caller's buffer holds
    uint8_t* codes_table = nullptr;   // nnrh_qmatmul_set_codes_out: [256][Np] quantized chain values
    int a_zp = 0, b_beta = 0;
    float b_scale = 0.f, y_scale = 0.f;
    ~nnrh_qmatmul() {
        dfree(wpack); dfree(colsum); dfree(c0); dfree(rowsum); dfree(dq_bias); dfree(colscale); dfree(codes_table);
    }
};

extern "C" int nnrh_qmatmul_create(nnrh_qmatmul_t* out, const nnrh_qmatmul_desc* d) {
    if (!out || !d) return set_err(NNRH_ERR_INVALID, "qmatmul: NULL argument");
    *out = nullptr;
    if (d->m <= 0 || d->n <= 0 || d->k <= 0) return set_err(NNRH_ERR_INVALID, "qmatmul: bad m/n/k");
    if ((d->a_dtype != NNRH_U8 && d->a_dtype != NNRH_S8) || (d->b_dtype != NNRH_U8 && d->b_dtype != NNRH_S8) ||
        (d->y_dtype != NNRH_U8 && d->y_dtype != NNRH_S8))
        return set_err(NNRH_ERR_UNSUPPORTED, "qmatmul: dtypes");
    if (d->scale_dtype != NNRH_F32 && d->scale_dtype != NNRH_F16)
        return set_err(NNRH_ERR_UNSUPPORTED, "qmatmul: scale dtype");
    if (!d->b_host || !d->a_scale_host || !d->b_scale_host || !d->y_scale_host)
        return set_err(NNRH_ERR_INVALID, "qmatmul: missing B or scales");
    nnrh_qmatmul* h = new (std::nothrow) nnrh_qmatmul();
    if (!h) return set_err(NNRH_ERR_NOMEM, "qmatmul: host allocation");
    auto fail = [&](int code) { delete h; return code; };
    h->d = *d;
    const int m = d->m, n = d->n, k = d->k;
    const int Kp = round_up(k, 64), Np = round_up(n, 64);
    const bool bu8 = d->b_dtype == NNRH_U8;
    std::vector<int8_t> wp((size_t)Np * Kp, 0);
    std::vector<int32_t> colsum(Np, 0);
    const uint8_t* braw = (const uint8_t*)d->b_host;
    for (int j = 0; j < n; ++j) {
        int8_t* row = wp.data() + (size_t)packed_row_of_col(j) * Kp;
        int32_t s = 0;
        for (int i = 0; i < k; ++i) {
            int8_t v = (int8_t)(braw[(size_t)i * n + j] ^ (bu8 ? 0x80 : 0));
            row[i] = v;
            s += v;
        }
        colsum[j] = s;
    }
    int rc;
    const bool au8 = d->a_dtype == NNRH_U8;
    h->a_zp = ld_zp(d->a_zp_host, d->a_dtype);
    std::vector<int32_t> c0(Np, 0);
    for (int j = 0; j < n; ++j)
        c0[j] = (int32_t)(0u - (uint32_t)(h->a_zp - (au8 ? 128 : 0)) * (uint32_t)colsum[j]);
    if ((rc = upload(&h->wpack, wp.data(), wp.size()))) return fail(rc);
    if ((rc = upload(&h->colsum, colsum.data(), colsum.size()))) return fail(rc);
    if ((rc = upload(&h->c0, c0.data(), c0.size()))) return fail(rc);
    for (int32_t v : c0) h->g.c0_absmax = std::max(h->g.c0_absmax, std::llabs((long long)v));
    const int b_zp = ld_zp(d->b_zp_host, d->b_dtype);   // b_zp[0] only (QLinearMatMul.cpp:119)
    h->b_beta = b_zp - (bu8 ? 128 : 0);
    // combined scale (QLinearMatMul.cpp:124-135)
    float cm;
    if (d->scale_dtype == NNRH_F16) {
        float fa = f16_to_f32(*(const uint16_t*)d->a_scale_host);
        float fb = f16_to_f32(*(const uint16_t*)d->b_scale_host);
        float fy = f16_to_f32(*(const uint16_t*)d->y_scale_host);
        uint16_t t = f32_to_f16(fa * fb);
        t = f32_to_f16(f16_to_f32(t) / fy);
        cm = f16_to_f32(t);
        h->b_scale = fb; h->y_scale = fy;
    } else {
        float as = *(const float*)d->a_scale_host, bs = *(const float*)d->b_scale_host,
              ys = *(const float*)d->y_scale_host;
        float t = as * bs;
        cm = t / ys;
        h->b_scale = bs; h->y_scale = ys;
    }
    GemmArgs& g = h->g;
    g.a_xor = au8 ? 0x80 : 0;
    g.M = m; g.N = n; g.K = k; g.Kp = Kp;
    g.lda = k;
    g.b = h->wpack; g.b_bstride = 0; g.Np = Np;
    g.colsum = h->colsum;
    g.c0 = h->c0;
    g.a_sub = au8 ? 128 : 0;
    g.alpha = h->a_zp - g.a_sub;
    g.beta = h->b_beta;
    g.param_bstride = 0;
    g.rowsum_bstride = m;
    g.epi = EPI_RQD;
    g.cm = cm;
    g.cm_b = h->b_scale; g.cm_y = h->y_scale;
    g.y_zp = ld_zp(d->y_zp_host, d->y_dtype);
    g.lo = d->y_dtype == NNRH_U8 ? 0 : -128;
    g.hi = d->y_dtype == NNRH_U8 ? 255 : 127;
    g.y_type = d->y_dtype == NNRH_U8 ? 0 : 1;
    g.ldy = n;
    g.y_bstride = (long long)m * n;
    g.bprime_from = n;
    *out = h;
    return NNRH_OK;
}

extern "C" int nnrh_qmatmul_fuse_dq_bias(nnrh_qmatmul_t h, float dq_scale, int dq_zp, const float* bias_host) {
    if (!h) return set_err(NNRH_ERR_INVALID, "qmatmul_fuse_dq_bias: NULL handle");
    const GemmArgs& g = h->g;
    // uint8 output only (the kernel's fused path reads the bytes unsigned)
    if (g.epi != EPI_RQD || h->d.scale_dtype != NNRH_F32 || dq_zp != g.y_zp || g.beta != 0 || g.K % 16 || g.lda % 16 ||
        g.y_type != 0 || g.c0_absmax + 16384LL * g.Kp >= 0x7fffffffLL)
        return set_err(NNRH_ERR_UNSUPPORTED, "qmatmul_fuse_dq_bias: not available for this QLinearMatMul");
    const int n = h->d.n, Np = g.Np;
    std::vector<float> b((size_t)Np, 0.0f);
    if (bias_host) std::copy(bias_host, bias_host + n, b.begin());
    dfree(h->dq_bias);
    h->dq_bias = nullptr;
    int rc = upload(&h->dq_bias, b.data(), b.size());
    if (rc) return rc;
    h->g.dq_bias = h->dq_bias;
    h->g.dq_scale = dq_scale;
    h->g.dq_codes = 0;   // the chain changed: codes mode is set again after it
    return NNRH_OK;
}

// MatMulInteger with a constant B whose int32 result goes through Cast ->
// Mul by fl(a_scale * w_scale[n]) -> Add(bias[n]): the per-channel form of
// dynamic quantization, one GEMM writing fp32.
extern "C" int nnrh_matmul_integer_scaled_create(nnrh_qmatmul_t* out, const nnrh_mmi_scaled_desc* d) {
    if (!out || !d) return set_err(NNRH_ERR_INVALID, "matmul_integer_scaled: NULL argument");
    *out = nullptr;
    if (d->m <= 0 || d->n <= 0 || d->k <= 0 || !d->b_host || !d->w_scale_host)
        return set_err(NNRH_ERR_INVALID, "matmul_integer_scaled: bad shape, B or scales");
    if ((d->a_dtype != NNRH_U8 && d->a_dtype != NNRH_S8) || (d->b_dtype != NNRH_U8 && d->b_dtype != NNRH_S8))
        return set_err(NNRH_ERR_UNSUPPORTED, "matmul_integer_scaled: dtypes");
    const bool bu8 = d->b_dtype == NNRH_U8;
    // the pipelined kernel has no per-row (b zero point) term
    if (d->b_zp != (bu8 ? 128 : 0))
        return set_err(NNRH_ERR_UNSUPPORTED, "matmul_integer_scaled: B zero point must be %d", bu8 ? 128 : 0);
    if (d->k % 16) return set_err(NNRH_ERR_UNSUPPORTED, "matmul_integer_scaled: K %% 16 != 0");
    nnrh_qmatmul* h = new (std::nothrow) nnrh_qmatmul();
    if (!h) return set_err(NNRH_ERR_NOMEM, "matmul_integer_scaled: host allocation");
    auto fail = [&](int code) { delete h; return code; };
    const int m = d->m, n = d->n, k = d->k;
    const int Kp = round_up(k, 64), Np = round_up(n, 64);
    std::vector<int8_t> wp((size_t)Np * Kp, 0);
    std::vector<int32_t> colsum(Np, 0);
    const uint8_t* braw = (const uint8_t*)d->b_host;
    for (int j = 0; j < n; ++j) {
        int8_t* row = wp.data() + (size_t)packed_row_of_col(j) * Kp;
        int32_t sum = 0;
        for (int i = 0; i < k; ++i) {
            const int8_t v = (int8_t)(braw[(size_t)i * n + j] ^ (bu8 ? 0x80 : 0));
            row[i] = v;
            sum += v;
        }
        colsum[j] = sum;
    }
    const bool au8 = d->a_dtype == NNRH_U8;
    std::vector<int32_t> c0(Np, 0);
    for (int j = 0; j < n; ++j)
        c0[j] = (int32_t)(0u - (uint32_t)(d->a_zp - (au8 ? 128 : 0)) * (uint32_t)colsum[j]);
    std::vector<float> ws((size_t)Np, 0.0f), b((size_t)Np, 0.0f);
    std::copy(d->w_scale_host, d->w_scale_host + n, ws.begin());
    if (d->bias_host) std::copy(d->bias_host, d->bias_host + n, b.begin());
    int rc;
    if ((rc = upload(&h->wpack, wp.data(), wp.size()))) return fail(rc);
    if ((rc = upload(&h->colsum, colsum.data(), colsum.size()))) return fail(rc);
    if ((rc = upload(&h->c0, c0.data(), c0.size()))) return fail(rc);
    if ((rc = upload(&h->colscale, ws.data(), ws.size()))) return fail(rc);
    if ((rc = upload(&h->dq_bias, b.data(), b.size()))) return fail(rc);
    for (int32_t v : c0) h->g.c0_absmax = std::max(h->g.c0_absmax, std::llabs((long long)v));
    h->d.m = m; h->d.n = n; h->d.k = k;
    h->d.a_dtype = d->a_dtype; h->d.b_dtype = d->b_dtype;
    h->d.y_dtype = NNRH_F32; h->d.scale_dtype = NNRH_F32;
    h->a_zp = d->a_zp;
    GemmArgs& g = h->g;
    g.a_xor = au8 ? 0x80 : 0;
    g.M = m; g.N = n; g.K = k; g.Kp = Kp;
    g.lda = k;
    g.b = h->wpack; g.b_bstride = 0; g.Np = Np;
    g.colsum = h->colsum;
    g.c0 = h->c0;
    g.a_sub = au8 ? 128 : 0;
    g.alpha = d->a_zp - g.a_sub;
    g.beta = 0;
    g.param_bstride = 0;
    g.epi = EPI_I32S;
    g.cm = d->a_scale;
    g.cs = h->colscale;
    g.dq_bias = h->dq_bias;
    g.dq_nobias = d->bias_host ? 0 : 1;
    g.y_type = 3;
    g.ldy = n;
    g.y_bstride = (long long)m * n;
    g.bprime_from = n;
    if (g.c0_absmax + 16384LL * g.Kp >= 0x7fffffffLL || 256LL * 128LL * Kp + 16384LL * Kp >= 0x7fffffffLL)
        return fail(set_err(NNRH_ERR_UNSUPPORTED, "matmul_integer_scaled: K too large for int32 accumulators"));
    *out = h;
    return NNRH_OK;
}

// ---------------------------------------------------------------------------
// QLinearMatMuls with fused dequantize + bias that read the same A (a
// transformer layer's Q / K / V projections) as one launch: member z is the
// GEMM's batch index, with B, colsum / c0 and the bias concatenated [z][..].
struct nnrh_qmatmul_group {
    int n = 0;
    GemmArgs g{};
    nnrh_qmatmul_desc d{};
    int8_t* wpack = nullptr;
    int32_t* colsum = nullptr;
    int32_t* c0 = nullptr;
    float* dq_bias = nullptr;
    float* colscale = nullptr;
    ~nnrh_qmatmul_group() { dfree(wpack); dfree(colsum); dfree(c0); dfree(dq_bias); dfree(colscale); }
};

extern "C" int nnrh_qmatmul_group_create(nnrh_qmatmul_group_t* out, const nnrh_qmatmul_t* hs, int n) {
    if (!out || !hs) return set_err(NNRH_ERR_INVALID, "qmatmul_group_create: NULL argument");
    *out = nullptr;
    if (n < 2 || n > 4) return set_err(NNRH_ERR_UNSUPPORTED, "qmatmul_group_create: %d members (2..4)", n);
    const nnrh_qmatmul* h0 = hs[0];
    if (!h0) return set_err(NNRH_ERR_INVALID, "qmatmul_group_create: NULL member");
    for (int i = 0; i < n; ++i) {
        const nnrh_qmatmul* h = hs[i];
        if (!h) return set_err(NNRH_ERR_INVALID, "qmatmul_group_create: NULL member");
        const GemmArgs& g = h->g;
        const bool same = h->d.m == h0->d.m && h->d.n == h0->d.n && h->d.k == h0->d.k &&
                          h->d.a_dtype == h0->d.a_dtype && h->d.b_dtype == h0->d.b_dtype &&
                          g.epi == h0->g.epi && (g.epi == EPI_I32S || h->d.y_dtype == NNRH_U8) &&
                          h->d.scale_dtype == NNRH_F32 && g.dq_nobias == h0->g.dq_nobias &&
                          (g.epi != EPI_I32S || g.cm == h0->g.cm) &&
                          g.Np == h0->g.Np && g.Kp == h0->g.Kp && g.alpha == h0->g.alpha &&
                          g.a_xor == h0->g.a_xor && g.beta == 0 && g.dq_bias && !g.dq_gelu && !g.mm_parts &&
                          !g.dq_codes;
        if (!same)
            return set_err(NNRH_ERR_UNSUPPORTED, "qmatmul_group_create: member %d differs in shape, types, "
                                                 "A quantization or fusions", i);
    }
    nnrh_qmatmul_group* G = new (std::nothrow) nnrh_qmatmul_group();
    if (!G) return set_err(NNRH_ERR_NOMEM, "qmatmul_group_create: host allocation");
    auto fail = [&](int code) { delete G; return code; };
    const int Np = h0->g.Np, Kp = h0->g.Kp;
    const size_t wsz = (size_t)Np * Kp;
    int rc;
    if ((rc = nnrh_malloc((void**)&G->wpack, wsz * n))) return fail(rc);
    if ((rc = nnrh_malloc((void**)&G->colsum, sizeof(int32_t) * Np * n))) return fail(rc);
    if ((rc = nnrh_malloc((void**)&G->c0, sizeof(int32_t) * Np * n))) return fail(rc);
    if ((rc = nnrh_malloc((void**)&G->dq_bias, sizeof(float) * Np * n))) return fail(rc);
    const bool scaled = h0->g.epi == EPI_I32S;
    if (scaled && (rc = nnrh_malloc((void**)&G->colscale, sizeof(float) * Np * n))) return fail(rc);
    GemmArgs& g = G->g;
    g = h0->g;
    g.c0_absmax = 0;
    g.dq_codes = 0;   // nnrh_qmatmul_group_set_codes_out
    for (int i = 0; i < n; ++i) {
        const nnrh_qmatmul* h = hs[i];
        if (hipMemcpy(G->wpack + wsz * i, h->wpack, wsz, hipMemcpyDeviceToDevice) != hipSuccess ||
            hipMemcpy(G->colsum + (size_t)Np * i, h->colsum, sizeof(int32_t) * Np, hipMemcpyDeviceToDevice) !=
                hipSuccess ||
            hipMemcpy(G->c0 + (size_t)Np * i, h->c0, sizeof(int32_t) * Np, hipMemcpyDeviceToDevice) != hipSuccess ||
            hipMemcpy(G->dq_bias + (size_t)Np * i, h->dq_bias, sizeof(float) * Np, hipMemcpyDeviceToDevice) !=
                hipSuccess ||
            (scaled && hipMemcpy(G->colscale + (size_t)Np * i, h->colscale, sizeof(float) * Np,
                                 hipMemcpyDeviceToDevice) != hipSuccess))
            return fail(set_err(NNRH_ERR_HIP, "qmatmul_group_create: device copy failed"));
        g.c0_absmax = std::max(g.c0_absmax, h->g.c0_absmax);
        g.grp_cm[i] = h->g.cm;
        g.grp_cm_b[i] = h->g.cm_b;
        g.grp_cm_y[i] = h->g.cm_y;
        g.grp_dq_scale[i] = h->g.dq_scale;
        g.grp_y_zp[i] = h->g.y_zp;
    }
    g.ngrp = n;
    g.b = G->wpack;
    g.b_bstride = (long long)wsz;
    g.colsum = G->colsum;
    g.c0 = G->c0;
    g.dq_bias = G->dq_bias;
    if (scaled) g.cs = G->colscale;
    g.param_bstride = Np;
    g.a_bstride = 0;
    G->n = n;
    G->d = h0->d;
    *out = G;
    return NNRH_OK;
}

extern "C" int nnrh_qmatmul_group_run(nnrh_qmatmul_group_t G, const void* a, int rows, void* const* ys,
                                      const float* a_scale_dev, const void* a_zp_dev, void* stream) {
    if (!G || !a || !ys || rows <= 0) return set_err(NNRH_ERR_INVALID, "qmatmul_group_run: bad arguments");
    for (int i = 0; i < G->n; ++i)
        if (!ys[i]) return set_err(NNRH_ERR_INVALID, "qmatmul_group_run: NULL output %d", i);
    hipStream_t s = S(stream);
    GemmArgs g = G->g;
    g.a = (const uint8_t*)a;
    g.M = rows;
    g.y = ys[0];
    g.ldy = G->d.n;
    for (int i = 0; i < G->n; ++i) g.grp_y[i] = ys[i];
    g.alpha_zp_dev = a_zp_dev;
    g.cm_a_scale_dev = a_scale_dev;
    if (a_zp_dev) g.c0 = nullptr;   // the column term needs the zero point of this call
    const int vec = pick_vec(g.K, (int)g.lda, (uintptr_t)a);
    if (vec != 16 || !qgemm_dma_eligible(g, vec))
        return set_err(NNRH_ERR_UNSUPPORTED, "qmatmul_group_run: A must be 16-byte aligned with K %% 16 == 0");
    ProfScope ps("qgemm", s);
    HIP_TRY(launch_qgemm(g, G->n, pick_tile(g.N), vec, s), "qgemm_group");
    return NNRH_OK;
}

extern "C" int nnrh_qmatmul_group_set_codes_out(nnrh_qmatmul_group_t G, int on) {
    if (!G) return set_err(NNRH_ERR_INVALID, "qmatmul_group_set_codes_out: NULL group");
    if (on && G->g.epi != EPI_RQD)
        return set_err(NNRH_ERR_UNSUPPORTED, "qmatmul_group_set_codes_out: QLinearMatMul members only");
    G->g.dq_codes = on ? 1 : 0;
    return NNRH_OK;
}

extern "C" int nnrh_qmatmul_group_destroy(nnrh_qmatmul_group_t G) {
    delete G;
    return NNRH_OK;
}

extern "C" int nnrh_qmatmul_fuse_gelu(nnrh_qmatmul_t h) {
    if (!h) return set_err(NNRH_ERR_INVALID, "qmatmul_fuse_gelu: NULL handle");
    if (!h->g.dq_bias) return set_err(NNRH_ERR_UNSUPPORTED, "qmatmul_fuse_gelu: needs nnrh_qmatmul_fuse_dq_bias first");
    h->g.dq_gelu = 1;
    h->g.dq_codes = 0;   // the chain changed: codes mode is set again after it
    return NNRH_OK;
}

// (min, max) pairs a fused-dequantize run writes: one per (tile, wave) of the
// tile the launcher picks for N
static long long qmatmul_parts(const GemmArgs& g, int batch) {
    const bool tall = pick_tile(g.N) == TILE_256x64;
    const int BM = tall ? 256 : 128, BN = tall ? 64 : 128;
    return (long long)((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN) * batch * 4;
}

extern "C" int nnrh_qmatmul_minmax_count(nnrh_qmatmul_t h, int batch, int* count) {
    if (!h || !count || batch <= 0) return set_err(NNRH_ERR_INVALID, "qmatmul_minmax_count: bad arguments");
    if (!h->g.dq_bias) return set_err(NNRH_ERR_UNSUPPORTED, "qmatmul_minmax_count: needs nnrh_qmatmul_fuse_dq_bias first");
    const long long n = qmatmul_parts(h->g, batch);
    if (n > 0x7fffffffLL) return set_err(NNRH_ERR_UNSUPPORTED, "qmatmul_minmax_count: too many tiles");
    *count = (int)n;
    return NNRH_OK;
}

extern "C" int nnrh_qmatmul_set_minmax_out(nnrh_qmatmul_t h, float* parts_dev, int capacity) {
    if (!h) return set_err(NNRH_ERR_INVALID, "qmatmul_set_minmax_out: NULL handle");
    if (parts_dev && !h->g.dq_bias)
        return set_err(NNRH_ERR_UNSUPPORTED, "qmatmul_set_minmax_out: needs nnrh_qmatmul_fuse_dq_bias first");
    if (parts_dev && (capacity <= 0 || ((uintptr_t)parts_dev & 7)))
        return set_err(NNRH_ERR_INVALID, "qmatmul_set_minmax_out: capacity %d / alignment", capacity);
    h->g.mm_parts = parts_dev;
    h->parts_cap = parts_dev ? capacity : 0;
    return NNRH_OK;
}

extern "C" int nnrh_qmatmul_set_codes_out(nnrh_qmatmul_t h, int on) {
    if (!h) return set_err(NNRH_ERR_INVALID, "qmatmul_set_codes_out: NULL handle");
    if (!on) {
        h->g.dq_codes = 0;
        return NNRH_OK;
    }
    if (h->g.epi != EPI_RQD || !h->g.dq_bias)
        return set_err(NNRH_ERR_UNSUPPORTED, "qmatmul_set_codes_out: needs nnrh_qmatmul_fuse_dq_bias first");
    // the quantizer's table, when the run writes pairs for one
    if (h->g.mm_parts && !h->codes_table) {
        int rc = nnrh_malloc((void**)&h->codes_table, dynamic_quantize_codes_table_bytes(h->g.Np));
        if (rc) return rc;
    }
    h->g.dq_codes = 1;
    return NNRH_OK;
}

extern "C" int nnrh_qmatmul_dq_params(nnrh_qmatmul_t h, int* zp, float* dq_scale, const float** bias_dev) {
    if (!h || !zp || !dq_scale || !bias_dev) return set_err(NNRH_ERR_INVALID, "qmatmul_dq_params: NULL argument");
    if (h->g.epi != EPI_RQD || !h->g.dq_bias || h->g.dq_gelu)
        return set_err(NNRH_ERR_UNSUPPORTED, "qmatmul_dq_params: needs nnrh_qmatmul_fuse_dq_bias (no Gelu)");
    *zp = h->g.y_zp;
    *dq_scale = h->g.dq_scale;
    *bias_dev = h->dq_bias;
    return NNRH_OK;
}

extern "C" int nnrh_qmatmul_dynamic_quantize_codes(nnrh_qmatmul_t h, const void* codes, int batch, uint8_t* y,
                                                   float* y_scale, uint8_t* y_zp, void* stream) {
    if (!h || !codes || !y || !y_scale || !y_zp || batch <= 0)
        return set_err(NNRH_ERR_INVALID, "qmatmul_dynamic_quantize_codes: bad arguments");
    const GemmArgs& g = h->g;
    if (!g.dq_codes || !g.mm_parts || !h->codes_table)
        return set_err(NNRH_ERR_UNSUPPORTED, "qmatmul_dynamic_quantize_codes: needs nnrh_qmatmul_set_minmax_out, "
                                             "then nnrh_qmatmul_set_codes_out");
    const long long nparts = qmatmul_parts(g, batch);
    if (nparts > h->parts_cap)
        return set_err(NNRH_ERR_INVALID, "qmatmul_dynamic_quantize_codes: %lld min/max pairs exceed the buffer's %d",
                       nparts, h->parts_cap);
    const long long rows = (long long)batch * g.M;
    if ((rows + 255) / 256 > 65535)
        return set_err(NNRH_ERR_UNSUPPORTED, "qmatmul_dynamic_quantize_codes: %lld rows", rows);
    ProfScope ps("dynamic_quantize", S(stream));
    HIP_TRY(launch_dynamic_quantize_codes((const uint8_t*)codes, rows, g.N, g.Np, g.dq_bias, g.dq_scale, g.y_zp,
                                          g.dq_gelu, g.mm_parts, (int)nparts, h->codes_table, y, y_scale, y_zp,
                                          S(stream)),
            "dynamic_quantize_codes");
    return NNRH_OK;
}

extern "C" int nnrh_qmatmul_run(nnrh_qmatmul_t h, const void* a, long long a_bstride, void* y, int batch,
                                const float* a_scale_dev, const void* a_zp_dev, void* stream) {
    if (!h || !a || !y) return set_err(NNRH_ERR_INVALID, "qmatmul_run: NULL argument");
    if (batch <= 0) return set_err(NNRH_ERR_INVALID, "qmatmul_run: batch %d", batch);
    if (a_scale_dev && h->d.scale_dtype != NNRH_F32)
        return set_err(NNRH_ERR_UNSUPPORTED, "qmatmul_run: device a_scale needs float32 scales");
    hipStream_t s = S(stream);
    GemmArgs g = h->g;
    g.a = (const uint8_t*)a;
    g.a_bstride = a_bstride;
    g.y = y;
    g.alpha_zp_dev = a_zp_dev;
    g.cm_a_scale_dev = a_scale_dev;
    if (a_zp_dev) g.c0 = nullptr;   // the column term needs the zero point of this call
    if (g.beta != 0) {
        if (h->rowsum_cap < batch) {
            dfree(h->rowsum);
            h->rowsum = nullptr;
            h->rowsum_cap = 0;
            int rc = nnrh_malloc((void**)&h->rowsum, sizeof(int32_t) * (size_t)batch * h->d.m);
            if (rc) return rc;
            h->rowsum_cap = batch;
        }
        ProfScope ps("rowsum", s);
        HIP_TRY(launch_rowsum_dense((const uint8_t*)a, g.lda, a_bstride, g.M, g.K, g.a_xor == 0,
                                    h->a_zp, a_zp_dev, h->rowsum, batch, s),
                "rowsum_dense");
        g.rowsum = h->rowsum;
    }
    int vec = pick_vec(g.K, (int)g.lda, (uintptr_t)a);
    if (a_bstride % vec) vec = 1;
    if (g.mm_parts && qmatmul_parts(g, batch) > h->parts_cap)
        return set_err(NNRH_ERR_INVALID, "qmatmul_run: %lld min/max pairs exceed the buffer's %d",
                       qmatmul_parts(g, batch), h->parts_cap);
    ProfScope ps("qgemm", s);
    HIP_TRY(launch_qgemm(g, batch, pick_tile(g.N), vec, s), "qgemm");
    return NNRH_OK;
}

extern "C" int nnrh_qmatmul_destroy(nnrh_qmatmul_t h) {
    delete h;
    return NNRH_OK;
}

// ===========================================================================
// MatMulInteger (dynamic A and B)

struct nnrh_matmul_integer {
    int m = 0, n = 0, k = 0, a_dtype = 0, b_dtype = 0, max_batch = 0, Kp = 0, Np = 0;
    int8_t* bpack = nullptr;
    int32_t* colsum = nullptr;
    int32_t* rowsum = nullptr;
    ~nnrh_matmul_integer() { dfree(bpack); dfree(colsum); dfree(rowsum); }
};

extern "C" int nnrh_matmul_integer_create(nnrh_matmul_integer_t* out, int m, int n, int k, int a_dtype,
                                          int b_dtype, int max_batch) {
    if (!out) return set_err(NNRH_ERR_INVALID, "matmul_integer: handle NULL");
    *out = nullptr;
    if (m <= 0 || n <= 0 || k <= 0 || max_batch <= 0)
        return set_err(NNRH_ERR_INVALID, "matmul_integer: bad shape");
    if ((a_dtype != NNRH_U8 && a_dtype != NNRH_S8) || (b_dtype != NNRH_U8 && b_dtype != NNRH_S8))
        return set_err(NNRH_ERR_UNSUPPORTED, "matmul_integer: dtypes");
    nnrh_matmul_integer* h = new (std::nothrow) nnrh_matmul_integer();
    if (!h) return set_err(NNRH_ERR_NOMEM, "matmul_integer: host allocation");
    h->m = m; h->n = n; h->k = k; h->a_dtype = a_dtype; h->b_dtype = b_dtype; h->max_batch = max_batch;
    h->Kp = round_up(k, 64); h->Np = round_up(n, 64);
    int rc;
    if ((rc = nnrh_malloc((void**)&h->bpack, (size_t)max_batch * h->Np * h->Kp)) ||
        (rc = nnrh_malloc((void**)&h->colsum, sizeof(int32_t) * (size_t)max_batch * h->Np)) ||
        (rc = nnrh_malloc((void**)&h->rowsum, sizeof(int32_t) * (size_t)max_batch * m))) {
        delete h;
        return rc;
    }
    *out = h;
    return NNRH_OK;
}

int matmul_integer_gemm(nnrh_matmul_integer* h, const void* a, long long a_bstride, const int8_t* bpack,
                        const int32_t* colsum, bool b_batched, int a_zp, int b_zp, int32_t* y, int batch,
                        hipStream_t s, const void* a_zp_dev = nullptr);

extern "C" int nnrh_matmul_integer_run(nnrh_matmul_integer_t h, const void* a, long long a_bstride,
                                       const void* b, long long b_bstride, int a_zp, int b_zp,
                                       int32_t* y, int batch, void* stream) {
    if (!h || !a || !b || !y) return set_err(NNRH_ERR_INVALID, "matmul_integer_run: NULL argument");
    if (batch <= 0 || batch > h->max_batch)
        return set_err(NNRH_ERR_INVALID, "matmul_integer_run: batch %d (max %d)", batch, h->max_batch);
    hipStream_t s = S(stream);
    const bool bu8 = h->b_dtype == NNRH_U8;
    const int nb_b = b_bstride == 0 ? 1 : batch;
    {
        ProfScope ps0("pack_b", s);
        HIP_TRY(launch_pack_b_dense(b, b_bstride, h->k, h->n, h->Kp, h->Np, bu8 ? 0x80 : 0, h->bpack,
                                    (long long)h->Np * h->Kp, h->colsum, h->Np, nb_b, s),
                "pack_b");
    }
    return matmul_integer_gemm(h, a, a_bstride, h->bpack, h->colsum, b_bstride != 0, a_zp, b_zp, y, batch, s);
}

extern "C" int nnrh_matmul_integer_run_dev_zp(nnrh_matmul_integer_t h, const void* a, long long a_bstride,
                                              const void* b, long long b_bstride, const void* a_zp_dev, int b_zp,
                                              int32_t* y, int batch, void* stream) {
    if (!h || !a || !b || !y || !a_zp_dev) return set_err(NNRH_ERR_INVALID, "matmul_integer_run_dev_zp: NULL argument");
    if (batch <= 0 || batch > h->max_batch)
        return set_err(NNRH_ERR_INVALID, "matmul_integer_run_dev_zp: batch %d (max %d)", batch, h->max_batch);
    hipStream_t s = S(stream);
    const bool bu8 = h->b_dtype == NNRH_U8;
    const int nb_b = b_bstride == 0 ? 1 : batch;
    {
        ProfScope ps0("pack_b", s);
        HIP_TRY(launch_pack_b_dense(b, b_bstride, h->k, h->n, h->Kp, h->Np, bu8 ? 0x80 : 0, h->bpack,
                                    (long long)h->Np * h->Kp, h->colsum, h->Np, nb_b, s),
                "pack_b");
    }
    return matmul_integer_gemm(h, a, a_bstride, h->bpack, h->colsum, b_bstride != 0, 0, b_zp, y, batch, s,
                               a_zp_dev);
}

// the GEMM of MatMulInteger over a packed B ([batch][Np][Kp] int8 and its
// column sums [batch][Np]; one shared when !b_batched)
int matmul_integer_gemm(nnrh_matmul_integer* h, const void* a, long long a_bstride, const int8_t* bpack,
                        const int32_t* colsum, bool b_batched, int a_zp, int b_zp, int32_t* y, int batch,
                        hipStream_t s, const void* a_zp_dev) {
    const bool au8 = h->a_dtype == NNRH_U8, bu8 = h->b_dtype == NNRH_U8;
    GemmArgs g{};
    g.a = (const uint8_t*)a;
    g.lda = h->k;
    g.a_bstride = a_bstride;
    g.a_xor = au8 ? 0x80 : 0;
    g.M = h->m; g.N = h->n; g.K = h->k; g.Kp = h->Kp;
    g.b = bpack;
    g.b_bstride = b_batched ? (long long)h->Np * h->Kp : 0;
    g.Np = h->Np;
    g.colsum = colsum;
    g.param_bstride = b_batched ? h->Np : 0;
    g.a_sub = au8 ? 128 : 0;
    g.alpha = a_zp - g.a_sub;
    g.alpha_zp_dev = a_zp_dev;
    g.beta = b_zp - (bu8 ? 128 : 0);
    if (g.beta != 0) {
        HIP_TRY(launch_rowsum_dense((const uint8_t*)a, g.lda, a_bstride, h->m, h->k, !au8, a_zp, a_zp_dev,
                                    h->rowsum, batch, s),
                "rowsum_dense");
        g.rowsum = h->rowsum;
        g.rowsum_bstride = h->m;
    }
    g.epi = EPI_I32;
    g.y = y;
    g.ldy = h->n;
    g.y_bstride = (long long)h->m * h->n;
    g.y_type = 2;
    g.bprime_from = h->n;
    int vec = pick_vec(h->k, h->k, (uintptr_t)a);
    if (a_bstride % vec) vec = 1;
    ProfScope ps("qgemm", s);
    HIP_TRY(launch_qgemm(g, batch, pick_tile(h->n), vec, s), "qgemm");
    return NNRH_OK;
}

extern "C" int nnrh_matmul_integer_destroy(nnrh_matmul_integer_t h) {
    delete h;
    return NNRH_OK;
}

// ===========================================================================
// element-wise ops

extern "C" int nnrh_quantize_linear(const float* x, size_t n, float scale, int zp, int y_dtype, void* y,
                                    void* stream) {
    if (n && (!x || !y)) return set_err(NNRH_ERR_INVALID, "quantize: NULL");
    if (y_dtype != NNRH_U8 && y_dtype != NNRH_S8) return set_err(NNRH_ERR_UNSUPPORTED, "quantize: dtype");
    ProfScope ps("quantize", S(stream));
    HIP_TRY(launch_quantize(x, (long long)n, scale, zp, y_dtype == NNRH_U8 ? 0 : 1, y, S(stream)), "quantize");
    return NNRH_OK;
}

extern "C" int nnrh_dequantize_linear(const void* x, int x_dtype, size_t n, float scale, int zp, float* y,
                                      void* stream) {
    if (n && (!x || !y)) return set_err(NNRH_ERR_INVALID, "dequantize: NULL");
    int dt = x_dtype == NNRH_U8 ? 0 : x_dtype == NNRH_S8 ? 1 : x_dtype == NNRH_I32 ? 2 : -1;
    if (dt < 0) return set_err(NNRH_ERR_UNSUPPORTED, "dequantize: dtype");
    ProfScope ps("dequantize", S(stream));
    HIP_TRY(launch_dequantize(x, (long long)n, dt, scale, zp, y, S(stream)), "dequantize");
    return NNRH_OK;
}

extern "C" size_t nnrh_dynamic_quantize_workspace(void) { return dynamic_quantize_workspace(); }

extern "C" int nnrh_dynamic_quantize_linear(const float* x, size_t n, uint8_t* y, float* y_scale,
                                            uint8_t* y_zp, void* ws, void* stream) {
    if (!y_scale || !y_zp || !ws || (n && (!x || !y)))
        return set_err(NNRH_ERR_INVALID, "dynamic_quantize: NULL");
    ProfScope ps("dynamic_quantize", S(stream));
    HIP_TRY(launch_dynamic_quantize(x, (long long)n, y, y_scale, y_zp, ws, S(stream)), "dynamic_quantize");
    return NNRH_OK;
}

extern "C" int nnrh_dynamic_quantize_linear_noalloc(const float* x, size_t n, uint8_t* y, float* y_scale,
                                                    uint8_t* y_zp, void* stream) {
    if (!y_scale || !y_zp || (n && (!x || !y)))
        return set_err(NNRH_ERR_INVALID, "dynamic_quantize_noalloc: NULL");
    if (n > NNRH_DYNQ_NOALLOC_MAX_N)
        return set_err(NNRH_ERR_INVALID,
                       "dynamic_quantize_noalloc: n = %zu exceeds the maximum of %llu elements", n,
                       (unsigned long long)NNRH_DYNQ_NOALLOC_MAX_N);
    HIP_TRY(launch_dynamic_quantize_noalloc(x, (long long)n, y, y_scale, y_zp, S(stream)),
            "dynamic_quantize_noalloc");
    return NNRH_OK;
}

extern "C" int nnrh_dynamic_quantize_linear_parts(const float* x, size_t n, const float* parts, int nparts,
                                                  uint8_t* y, float* y_scale, uint8_t* y_zp, void* stream) {
    if (!y_scale || !y_zp || !parts || nparts <= 0 || (n && (!x || !y)))
        return set_err(NNRH_ERR_INVALID, "dynamic_quantize_parts: bad arguments");
    ProfScope ps("dynamic_quantize", S(stream));
    HIP_TRY(launch_dynamic_quantize_parts(x, (long long)n, parts, nparts, y, y_scale, y_zp, S(stream)),
            "dynamic_quantize_parts");
    return NNRH_OK;
}

extern "C" int nnrh_qlinear_add(int kind, const void* a, const void* b, void* y, size_t n, int C, int HW,
                                int y_nhwc, int dtype, float a_scale, int a_zp, float b_scale, int b_zp,
                                float y_scale, int y_zp, void* stream) {
    if (n && (!a || !b || !y)) return set_err(NNRH_ERR_INVALID, "qlinear_add: NULL");
    if (dtype != NNRH_U8 && dtype != NNRH_S8) return set_err(NNRH_ERR_UNSUPPORTED, "qlinear_add: dtype");
    if (kind < 0 || kind > 3) return set_err(NNRH_ERR_INVALID, "qlinear_add: kind %d", kind);
    if (kind == 3 && (C <= 0 || HW <= 0 || n % ((size_t)C * HW)))
        return set_err(NNRH_ERR_INVALID, "qlinear_add: per-channel shape");
    QAddArgs p{};
    p.kind = kind; p.a = a; p.b = b; p.y = y; p.n = (long long)n;
    p.C = C; p.HW = HW; p.y_nhwc = y_nhwc; p.dt = dtype == NNRH_U8 ? 0 : 1;
    p.sa = a_scale / y_scale;
    p.sb = b_scale / y_scale;
    {   // QLinearAdd.cpp:66-67 (no contraction)
        float t1 = p.sa * (float)a_zp, t2 = p.sb * (float)b_zp;
        p.fixed = (float)y_zp - (t1 + t2);
    }
    p.a_zp = a_zp; p.b_zp = b_zp; p.y_zp = y_zp;
    p.lo = dtype == NNRH_U8 ? 0 : -128;
    p.hi = dtype == NNRH_U8 ? 255 : 127;
    ProfScope ps("qlinear_add", S(stream));
    HIP_TRY(launch_qadd(p, S(stream)), "qlinear_add");
    return NNRH_OK;
}

extern "C" int nnrh_qlinear_mul(int kind, const void* a, const void* b, void* y, size_t n, int C, int HW,
                                int y_nhwc, int dtype, float a_scale, int a_zp, float b_scale, int b_zp,
                                float y_scale, int y_zp, void* stream) {
    if (n && (!a || !b || !y)) return set_err(NNRH_ERR_INVALID, "qlinear_mul: NULL");
    if (dtype != NNRH_U8 && dtype != NNRH_S8) return set_err(NNRH_ERR_UNSUPPORTED, "qlinear_mul: dtype");
    if (kind < 0 || kind > 3) return set_err(NNRH_ERR_INVALID, "qlinear_mul: kind %d", kind);
    if (kind == 3 && (C <= 0 || HW <= 0 || n % ((size_t)C * HW)))
        return set_err(NNRH_ERR_INVALID, "qlinear_mul: per-channel shape");
    QMulArgs p{};
    p.kind = kind; p.a = a; p.b = b; p.y = y; p.n = (long long)n;
    p.C = C; p.HW = HW; p.y_nhwc = y_nhwc; p.dt = dtype == NNRH_U8 ? 0 : 1;
    p.cs = a_scale * b_scale / y_scale;   // QLinearMul.cpp:39
    p.a_zp = a_zp; p.b_zp = b_zp; p.y_zp = y_zp;
    p.lo = dtype == NNRH_U8 ? 0 : -128;
    p.hi = dtype == NNRH_U8 ? 255 : 127;
    ProfScope ps("qlinear_mul", S(stream));
    HIP_TRY(launch_qmul(p, S(stream)), "qlinear_mul");
    return NNRH_OK;
}

extern "C" int nnrh_qlinear_global_avgpool(const void* x, void* y, int N, int C, int spatial, int x_nhwc,
                                           int dtype, float x_scale, int x_zp, float y_scale, int y_zp,
                                           void* stream) {
    if (!x || !y) return set_err(NNRH_ERR_INVALID, "qlinear_global_avgpool: NULL");
    if (dtype != NNRH_U8 && dtype != NNRH_S8) return set_err(NNRH_ERR_UNSUPPORTED, "qlinear_global_avgpool: dtype");
    if (N <= 0 || C <= 0 || spatial <= 0) return set_err(NNRH_ERR_INVALID, "qlinear_global_avgpool: bad shape");
    const float rs = x_scale / (y_scale * (float)spatial);   // QLinearGlobalAveragePool.cpp:46
    ProfScope ps("qlinear_global_avgpool", S(stream));
    HIP_TRY(launch_qgap(x, y, N, C, spatial, x_nhwc, dtype == NNRH_U8 ? 0 : 1, rs, x_zp, y_zp,
                        dtype == NNRH_U8 ? 0 : -128, dtype == NNRH_U8 ? 255 : 127, S(stream)),
            "qlinear_global_avgpool");
    return NNRH_OK;
}

extern "C" int nnrh_qlinear_avgpool(const void* x, void* y, int N, int C, int iH, int iW, int oH, int oW, int kH,
                                    int kW, int sH, int sW, int pH, int pW, int nhwc, int dtype, float x_scale,
                                    int x_zp, float y_scale, int y_zp, void* stream) {
    if (!x || !y) return set_err(NNRH_ERR_INVALID, "qlinear_avgpool: NULL");
    if (dtype != NNRH_U8 && dtype != NNRH_S8) return set_err(NNRH_ERR_UNSUPPORTED, "qlinear_avgpool: dtype");
    if (N <= 0 || C <= 0 || oH <= 0 || oW <= 0 || kH <= 0 || kW <= 0 || sH <= 0 || sW <= 0)
        return set_err(NNRH_ERR_INVALID, "qlinear_avgpool: bad shape");
    ProfScope ps("qlinear_avgpool", S(stream));
    HIP_TRY(launch_qavgpool(x, y, N, C, iH, iW, oH, oW, kH, kW, sH, sW, pH, pW, nhwc, dtype == NNRH_U8 ? 0 : 1,
                            x_scale, x_zp, y_scale, y_zp, dtype == NNRH_U8 ? 0 : -128,
                            dtype == NNRH_U8 ? 255 : 127, S(stream)),
            "qlinear_avgpool");
    return NNRH_OK;
}

// ---- ConvInteger --------------------------------------------------------------
// The implicit-GEMM kernel of QLinearConv with an int32 epilogue: the NCHW
// input goes to an NHWC copy (each group's channels padded to a multiple of
// 16 with x_zp), the weights are packed per call, and
//   y = sum (x - x_zp)(w - w_zp) = acc' - alpha * colsum[n] + (b_sub - w_zp[n]) * rowsum[m]
// with acc' = sum (x - a_sub)(w - b_sub) on the MFMAs (padded taps and
// channels read x_zp, i.e. x - x_zp = 0, against zero weights), alpha = x_zp -
// a_sub and rowsum[m] = sum (x - x_zp) over pixel m's patch, which the kernel
// sums from its A fragments; stored NCHW.
struct nnrh_conv_integer {
    int N = 0, C = 0, iH = 0, iW = 0, OC = 0, G = 0, OCg = 0, Cg = 0, Cgp = 0;
    int x_dtype = 0, w_dtype = 0, Kp = 0, Np = 0;
    GemmArgs g{};
    uint8_t* xs = nullptr;        // NHWC copy [N][iH][iW][G * Cgp]
    int8_t* wpack = nullptr;      // [G][Np][Kp]
    int32_t* c0 = nullptr;        // [G][Np]
    int32_t* coef = nullptr;      // [G][Np] row-term coefficient
    ~nnrh_conv_integer() {
        dfree(xs); dfree(wpack); dfree(c0); dfree(coef);
    }
};

extern "C" int nnrh_conv_integer_create(nnrh_conv_integer_t* out, int N, int C, int iH, int iW, int OC, int kH,
                                        int kW, int sH, int sW, int pH, int pW, int dH, int dW, int oH, int oW,
                                        int group, int x_dtype, int w_dtype) {
    if (!out) return set_err(NNRH_ERR_INVALID, "conv_integer: handle NULL");
    *out = nullptr;
    if (N <= 0 || C <= 0 || iH <= 0 || iW <= 0 || OC <= 0 || kH <= 0 || kW <= 0 || sH <= 0 || sW <= 0 || dH <= 0 ||
        dW <= 0 || oH <= 0 || oW <= 0 || group <= 0 || pH < 0 || pW < 0 || C % group || OC % group)
        return set_err(NNRH_ERR_INVALID, "conv_integer: bad shape");
    if ((x_dtype != NNRH_U8 && x_dtype != NNRH_S8) || (w_dtype != NNRH_U8 && w_dtype != NNRH_S8))
        return set_err(NNRH_ERR_UNSUPPORTED, "conv_integer: dtype");
    const int G = group, Cg = C / G, OCg = OC / G;
    const int Cgp = round_up(Cg, 16);
    const long long K = (long long)kH * kW * Cgp;
    const long long M = (long long)N * oH * oW;
    // exact int32 partial sums on the MFMAs: |c0| + 128 * 128 * K per term
    if (K > 32768 || M > (1LL << 30) || (long long)G * Cgp > (1 << 20) || N > 65535 || G > 65535)
        return set_err(NNRH_ERR_UNSUPPORTED, "conv_integer: GEMM extents too large");
    auto* h = new (std::nothrow) nnrh_conv_integer();
    if (!h) return set_err(NNRH_ERR_NOMEM, "conv_integer: host allocation");
    h->N = N; h->C = C; h->iH = iH; h->iW = iW; h->OC = OC; h->G = G; h->OCg = OCg; h->Cg = Cg; h->Cgp = Cgp;
    h->x_dtype = x_dtype; h->w_dtype = w_dtype;
    h->Kp = (int)round_up(K, 64);
    h->Np = round_up(OCg, 64);
    GemmArgs& g = h->g;
    g.a_xor = x_dtype == NNRH_U8 ? 0x80 : 0;
    g.M = (int)M; g.N = OCg; g.K = (int)K; g.Kp = h->Kp;
    g.H = iH; g.W = iW; g.C = Cgp; g.Cs = G * Cgp;
    g.oH = oH; g.oW = oW; g.kH = kH; g.kW = kW; g.sH = sH; g.sW = sW; g.dH = dH; g.dW = dW;
    g.pad_t = pH; g.pad_l = pW;
    g.a_bstride = Cgp;   // group channel offset
    g.b_bstride = (long long)h->Np * h->Kp;
    g.Np = h->Np;
    g.a_sub = x_dtype == NNRH_U8 ? 128 : 0;
    g.param_bstride = h->Np;
    g.epi = EPI_I32;
    g.tail = TAIL_NONE;
    g.bprime_from = OCg;
    g.y_type = 2;
    g.y_nchw = 1;
    g.ldy = OC;
    g.y_bstride = (long long)OCg * oH * oW;
    g.c0_absmax = 16384LL * K;
    int rc = NNRH_OK;
    auto fail = [&](int code) { delete h; return code; };
    if ((rc = nnrh_malloc((void**)&h->xs, (size_t)N * iH * iW * G * Cgp))) return fail(rc);
    if ((rc = nnrh_malloc((void**)&h->wpack, (size_t)G * h->Np * h->Kp))) return fail(rc);
    if ((rc = nnrh_malloc((void**)&h->c0, sizeof(int32_t) * (size_t)G * h->Np))) return fail(rc);
    if ((rc = nnrh_malloc((void**)&h->coef, sizeof(int32_t) * (size_t)G * h->Np))) return fail(rc);
    // every call must run on the pipelined kernel (its FUSE_ROW epilogue)
    GemmArgs chk = g;
    chk.a = h->xs; chk.b = h->wpack; chk.c0 = h->c0; chk.row_coef = h->coef;
    chk.y = h->xs;
    if (!qgemm_dma_eligible(chk, 16)) return fail(set_err(NNRH_ERR_UNSUPPORTED, "conv_integer: shape"));
    *out = h;
    return NNRH_OK;
}

extern "C" int nnrh_conv_integer_run(nnrh_conv_integer_t h, const void* x, const void* w, int x_zp, int w_zp,
                                     const int32_t* w_zp_dev, int32_t* y, void* stream) {
    if (!h || !x || !w || !y) return set_err(NNRH_ERR_INVALID, "conv_integer_run: NULL argument");
    hipStream_t s = S(stream);
    const bool xu8 = h->x_dtype == NNRH_U8, wu8 = h->w_dtype == NNRH_U8;
    const int alpha = x_zp - (xu8 ? 128 : 0);
    GemmArgs g = h->g;
    {
        ConvIntPrepArgs q{};
        q.x = (const uint8_t*)x; q.xs = h->xs;
        q.N = h->N; q.HW = h->iH * h->iW; q.G = h->G; q.Cg = h->Cg; q.Cgp = h->Cgp;
        q.fill = (uint32_t)(x_zp & 0xff);
        q.w = (const uint8_t*)w; q.w_u8 = wu8 ? 1 : 0; q.OCg = h->OCg; q.kH = h->g.kH; q.kW = h->g.kW;
        q.Kp = h->Kp; q.Np = h->Np; q.alpha = alpha; q.w_zp = w_zp; q.w_zp_dev = w_zp_dev;
        q.wpack = h->wpack; q.c0 = h->c0; q.row_coef = h->coef;
        ProfScope ps("conv_integer_prep", s);
        HIP_TRY(launch_conv_integer_prep(q, s), "conv_integer_prep");
    }
    g.row_coef = h->coef;
    g.alpha = alpha;
    g.a = h->xs;
    g.b = h->wpack;
    g.c0 = h->c0;
    g.pad_byte = x_zp & 0xff;
    g.y = y;
    ProfScope ps("qgemm", s);
    HIP_TRY(launch_qgemm(g, h->G, pick_tile(h->OCg), 16, s), "qgemm");
    return NNRH_OK;
}

extern "C" int nnrh_conv_integer_destroy(nnrh_conv_integer_t h) {
    delete h;
    return NNRH_OK;
}

extern "C" int nnrh_batchnorm_u8(const void* x, int x_is_f32, uint8_t* y, const float* a, const float* b,
                                 long long N, int C, long long HW, int nhwc, void* stream) {
    if (!x || !y || !a || !b) return set_err(NNRH_ERR_INVALID, "batchnorm_u8: NULL");
    if (N < 0 || C <= 0 || HW < 0) return set_err(NNRH_ERR_INVALID, "batchnorm_u8: bad extents");
    ProfScope ps("batchnorm_u8", S(stream));
    HIP_TRY(launch_bn_affine_u8(x, x_is_f32, y, a, b, N, C, HW, nhwc, S(stream)), "batchnorm_u8");
    return NNRH_OK;
}

extern "C" int nnrh_batchnorm_f32(const float* x, float* y, const float* alpha, const float* beta, long long N,
                                  int C, long long HW, int nhwc, void* stream) {
    if (!x || !y || !alpha || !beta) return set_err(NNRH_ERR_INVALID, "batchnorm_f32: NULL");
    if (N < 0 || C <= 0 || HW < 0) return set_err(NNRH_ERR_INVALID, "batchnorm_f32: bad extents");
    ProfScope ps("batchnorm_f32", S(stream));
    HIP_TRY(launch_bn_f32(x, y, alpha, beta, N, C, HW, nhwc, S(stream)), "batchnorm_f32");
    return NNRH_OK;
}

extern "C" int nnrh_qlinear_concat_part(const void* x, void* y, long long outer, long long count, long long y_row,
                                        long long y_off, int dtype, float x_scale, int x_zp, float y_scale,
                                        int y_zp, void* stream);

extern "C" int nnrh_qlinear_concat(int ntens, const void* const* xs, const long long* counts,
                                   const float* x_scales, const int* x_zps, long long outer, int dtype,
                                   float y_scale, int y_zp, void* y, void* stream) {
    if (!xs || !counts || !x_scales || !x_zps || !y) return set_err(NNRH_ERR_INVALID, "qlinear_concat: NULL");
    if (dtype != NNRH_U8 && dtype != NNRH_S8) return set_err(NNRH_ERR_UNSUPPORTED, "qlinear_concat: dtype");
    if (ntens <= 0 || outer < 0) return set_err(NNRH_ERR_INVALID, "qlinear_concat: bad extents");
    long long row = 0;
    for (int t = 0; t < ntens; ++t) {
        if ((!xs[t] && counts[t] > 0) || counts[t] < 0) return set_err(NNRH_ERR_INVALID, "qlinear_concat: part %d", t);
        row += counts[t];
    }
    if (ntens > QCONCAT_MAX_PARTS) {   // one launch per part
        long long off = 0;
        for (int t = 0; t < ntens; ++t) {
            if (counts[t] == 0) continue;
            const int rc = nnrh_qlinear_concat_part(xs[t], y, outer, counts[t], row, off, dtype, x_scales[t],
                                                    x_zps[t], y_scale, y_zp, stream);
            if (rc != NNRH_OK) return rc;
            off += counts[t];
        }
        return NNRH_OK;
    }
    QConcatRows a{};
    a.n = 0;
    long long off = 0;
    for (int t = 0; t < ntens; ++t) {
        if (counts[t] == 0) continue;   // an empty part writes nothing
        const int k = a.n++;
        a.x[k] = xs[t];
        a.cnt[k] = counts[t];
        a.off[k] = off;
        // QLinearConcat.cpp:147: an input in the output's quantization is copied;
        // the 16-wide body covers count - count % 16 of a chunk of >= 16
        a.copy[k] = x_scales[t] == y_scale && x_zps[t] == y_zp;
        a.rs[k] = a.copy[k] ? 0.f : x_scales[t] / y_scale;
        a.zp[k] = x_zps[t];
        a.body[k] = counts[t] >= 16 ? counts[t] - counts[t] % 16 : 0;
        off += counts[t];
    }
    if (a.n == 0) return NNRH_OK;
    a.y = y;
    a.row = row;
    a.outer = outer;
    a.dt = dtype == NNRH_U8 ? 0 : 1;
    a.y_zp = y_zp;
    a.lo = dtype == NNRH_U8 ? 0 : -128;
    a.hi = dtype == NNRH_U8 ? 255 : 127;
    ProfScope ps("qlinear_concat", S(stream));
    HIP_TRY(launch_qconcat_rows(a, S(stream)), "qlinear_concat");
    return NNRH_OK;
}

extern "C" int nnrh_qlinear_concat_part(const void* x, void* y, long long outer, long long count, long long y_row,
                                        long long y_off, int dtype, float x_scale, int x_zp, float y_scale,
                                        int y_zp, void* stream) {
    if (!x || !y) return set_err(NNRH_ERR_INVALID, "qlinear_concat_part: NULL");
    if (dtype != NNRH_U8 && dtype != NNRH_S8) return set_err(NNRH_ERR_UNSUPPORTED, "qlinear_concat_part: dtype");
    if (outer < 0 || count < 0 || y_off < 0 || y_off + count > y_row)
        return set_err(NNRH_ERR_INVALID, "qlinear_concat_part: bad extents");
    // QLinearConcat.cpp:147: an input already in the output's quantization is copied
    const int copy = x_scale == y_scale && x_zp == y_zp;
    const float rs = copy ? 0.f : x_scale / y_scale;
    ProfScope ps("qlinear_concat", S(stream));
    HIP_TRY(launch_qconcat_part(x, y, outer, count, y_row, y_off, dtype == NNRH_U8 ? 0 : 1, copy, rs, x_zp, y_zp,
                                dtype == NNRH_U8 ? 0 : -128, dtype == NNRH_U8 ? 255 : 127, S(stream)),
            "qlinear_concat_part");
    return NNRH_OK;
}

extern "C" int nnrh_maxpool_u8_nhwc(const uint8_t* x, uint8_t* y, int N, int C, int iH, int iW, int oH,
                                    int oW, int kH, int kW, int sH, int sW, int pH, int pW, void* stream) {
    if (!x || !y) return set_err(NNRH_ERR_INVALID, "maxpool: NULL");
    if (N <= 0 || C <= 0 || oH <= 0 || oW <= 0 || kH <= 0 || kW <= 0 || sH <= 0 || sW <= 0)
        return set_err(NNRH_ERR_INVALID, "maxpool: bad shape");
    ProfScope ps("maxpool_u8", S(stream));
    HIP_TRY(launch_maxpool_u8_nhwc(x, y, N, C, iH, iW, oH, oW, kH, kW, sH, sW, pH, pW, S(stream)), "maxpool");
    return NNRH_OK;
}

extern "C" int nnrh_nchw_to_nhwc_u8(const uint8_t* x, uint8_t* y, int N, int C, int HW, void* stream) {
    if (!x || !y) return set_err(NNRH_ERR_INVALID, "nchw_to_nhwc: NULL");
    HIP_TRY(launch_nchw_to_nhwc_u8(x, y, N, C, HW, C, 0, S(stream)), "nchw_to_nhwc");
    return NNRH_OK;
}

// ===========================================================================
// fp32 glue

extern "C" int nnrh_global_avgpool_f32(const float* x, float* y, int N, int C, int HW, int x_nhwc,
                                       void* stream) {
    if (!x || !y || N <= 0 || C <= 0 || HW <= 0) return set_err(NNRH_ERR_INVALID, "gap: bad args");
    ProfScope ps("gap_f32", S(stream));
    HIP_TRY(launch_gap_f32(x, y, N, C, HW, x_nhwc, S(stream)), "gap_f32");
    return NNRH_OK;
}

extern "C" int nnrh_multihead_attention_workspace(int B, int seq, int hidden, int num_heads, size_t* bytes) {
    if (!bytes || B < 0 || seq < 0 || num_heads <= 0 || hidden <= 0 || hidden % num_heads)
        return set_err(NNRH_ERR_INVALID, "mha_workspace: arguments");
    // the fused head-64 kernel keeps everything in LDS and registers
    *bytes = mha_fused_shape(seq, hidden, num_heads) ? 0 : mha_workspace_bytes(B, seq, num_heads);
    return NNRH_OK;
}

extern "C" int nnrh_multihead_attention_minmax_count(int B, int seq, int hidden, int num_heads, int* pairs) {
    if (!pairs || B < 0 || seq < 0 || num_heads <= 0 || hidden <= 0 || hidden % num_heads)
        return set_err(NNRH_ERR_INVALID, "mha_minmax_count: arguments");
    *pairs = mha_minmax_pairs(B, seq, hidden, num_heads);
    return NNRH_OK;
}

extern "C" int nnrh_multihead_attention_f32(const float* q, const float* k, const float* v, float* y, int B, int seq,
                                            int hidden, int num_heads, float scale, float* minmax_parts,
                                            void* workspace, void* stream) {
    if (!q || !k || !v || !y) return set_err(NNRH_ERR_INVALID, "mha: NULL argument");
    if (B < 0 || seq < 0 || hidden <= 0 || num_heads <= 0 || hidden % num_heads)
        return set_err(NNRH_ERR_INVALID, "mha: hidden %d / heads %d", hidden, num_heads);
    if ((!workspace || minmax_parts) && !mha_fused_ok(q, k, v, y, seq, hidden, num_heads))
        return set_err(NNRH_ERR_INVALID, minmax_parts ? "mha: min / max pairs need the fused kernel (head size 64, "
                                                        "seq <= 128, 16-byte aligned q / k / v / y)"
                                                      : "mha: this shape (or unaligned q / k / v / y) needs the workspace");
    if (((uintptr_t)workspace & 255) != 0) return set_err(NNRH_ERR_INVALID, "mha: workspace must be 256-byte aligned");
    hipStream_t s = S(stream);
    ProfScope ps("multihead_attention", s);
    HIP_TRY(launch_mha_f32(q, k, v, y, B, seq, hidden, num_heads, scale, minmax_parts, workspace, s),
            "multihead_attention");
    return NNRH_OK;
}

extern "C" int nnrh_global_avgpool_dequant(const void* x, float* y, int N, int C, int HW, int x_nhwc,
                                           int x_dtype, float scale, int zp, void* stream) {
    if (!x || !y || N < 0 || C < 0 || HW <= 0) return set_err(NNRH_ERR_INVALID, "global_avgpool_dequant: arguments");
    if (x_dtype != NNRH_U8 && x_dtype != NNRH_S8)
        return set_err(NNRH_ERR_UNSUPPORTED, "global_avgpool_dequant: dtype %d", x_dtype);
    hipStream_t s = S(stream);
    ProfScope ps("gap_dequant", s);
    HIP_TRY(launch_gap_dq((const uint8_t*)x, y, N, C, HW, x_nhwc, x_dtype == NNRH_S8, scale, zp, s), "gap_dequant");
    return NNRH_OK;
}

extern "C" int nnrh_gemm_f32(const float* a, const float* b, const float* cb, float* y, int M, int N,
                             int K, int ta, int tb, float alpha, float beta, int c_mode, void* stream) {
    if (!a || !b || !y || M <= 0 || N <= 0 || K <= 0 || c_mode < 0 || c_mode > 4 || (c_mode && !cb))
        return set_err(NNRH_ERR_INVALID, "gemm_f32: bad args");
    ProfScope ps("gemm_f32", S(stream));
    HIP_TRY(launch_gemm_f32(a, b, cb, y, M, N, K, ta, tb, alpha, beta, c_mode, S(stream)), "gemm_f32");
    return NNRH_OK;
}

extern "C" int nnrh_gemm_f32_batched(const float* a, const float* b, const float* cb, float* y, int M,
                                     int N, int K, int ta, int tb, float alpha, float beta, int c_mode,
                                     int batch, long long a_bstride, long long b_bstride,
                                     long long y_bstride, void* stream) {
    if (!a || !b || !y || M <= 0 || N <= 0 || K <= 0 || batch <= 0 || c_mode < 0 || c_mode > 4 ||
        (c_mode && !cb))
        return set_err(NNRH_ERR_INVALID, "gemm_f32_batched: bad args");
    ProfScope ps("gemm_f32", S(stream));
    HIP_TRY(launch_gemm_f32_batched(a, b, cb, y, M, N, K, ta, tb, alpha, beta, c_mode, batch, a_bstride,
                                    b_bstride, y_bstride, S(stream)),
            "gemm_f32_batched");
    return NNRH_OK;
}

extern "C" int nnrh_binary_f32(int op, const float* a, const float* b, float* y, size_t n, int D,
                               int b_mode, int b_first, void* stream) {
    if (n && (!a || !b || !y)) return set_err(NNRH_ERR_INVALID, "binary_f32: NULL");
    if (op < 0 || op > 3 || b_mode < 0 || b_mode > 2 || (b_mode == 2 && (D <= 0 || n % (size_t)D)))
        return set_err(NNRH_ERR_INVALID, "binary_f32: op %d mode %d D %d", op, b_mode, D);
    ProfScope ps("binary_f32", S(stream));
    HIP_TRY(launch_binary_f32(a, b, y, (long long)n, D, b_mode, op, b_first, S(stream)), "binary_f32");
    return NNRH_OK;
}

extern "C" int nnrh_softmax_f32(const float* x, float* y, size_t rows, int D, void* stream) {
    if (rows && (!x || !y || D <= 0)) return set_err(NNRH_ERR_INVALID, "softmax_f32: bad args");
    ProfScope ps("softmax_f32", S(stream));
    HIP_TRY(launch_softmax_f32(x, y, (long long)rows, D, S(stream)), "softmax_f32");
    return NNRH_OK;
}

extern "C" int nnrh_layernorm_f32(const float* x, const float* gamma, const float* beta, float* y,
                                  size_t rows, int D, float eps, void* stream) {
    if (rows && (!x || !gamma || !y || D <= 0)) return set_err(NNRH_ERR_INVALID, "layernorm_f32: bad args");
    ProfScope ps("layernorm_f32", S(stream));
    HIP_TRY(launch_layernorm_f32(x, nullptr, gamma, beta, y, (long long)rows, D, eps, nullptr, S(stream)),
            "layernorm_f32");
    return NNRH_OK;
}

extern "C" int nnrh_add_layernorm_f32(const float* x, const float* r, const float* gamma, const float* beta,
                                      float* y, size_t rows, int D, float eps, float* parts, void* stream) {
    if (rows && (!x || !gamma || !y || D <= 0)) return set_err(NNRH_ERR_INVALID, "add_layernorm_f32: bad args");
    if (parts && ((uintptr_t)parts & 7)) return set_err(NNRH_ERR_INVALID, "add_layernorm_f32: parts alignment");
    ProfScope ps("layernorm_f32", S(stream));
    HIP_TRY(launch_layernorm_f32(x, r, gamma, beta, y, (long long)rows, D, eps, parts, S(stream)),
            "add_layernorm_f32");
    return NNRH_OK;
}

static DqCodes dq_codes_arg(const nnrh_dq_codes* c) { return DqCodes{c->codes_dev, c->zp, c->scale, c->bias_dev}; }

extern "C" int nnrh_add_layernorm_codes_f32(const nnrh_dq_codes* x, const float* r, const float* gamma,
                                            const float* beta, float* y, size_t rows, int D, float eps, float* parts,
                                            void* stream) {
    if (!x || (rows && (!x->codes_dev || !x->bias_dev || !gamma || !y || D <= 0)))
        return set_err(NNRH_ERR_INVALID, "add_layernorm_codes_f32: bad args");
    if (parts && ((uintptr_t)parts & 7)) return set_err(NNRH_ERR_INVALID, "add_layernorm_codes_f32: parts alignment");
    ProfScope ps("layernorm_f32", S(stream));
    HIP_TRY(launch_layernorm_codes_f32(dq_codes_arg(x), r, gamma, beta, y, (long long)rows, D, eps, parts,
                                       S(stream)),
            "add_layernorm_codes_f32");
    return NNRH_OK;
}

extern "C" int nnrh_multihead_attention_codes_f32(const nnrh_dq_codes* q, const nnrh_dq_codes* k,
                                                  const nnrh_dq_codes* v, float* y, int B, int seq, int hidden,
                                                  int num_heads, float scale, float* minmax_parts, void* stream) {
    if (!q || !k || !v || !y || B < 0 || seq < 0 || !q->codes_dev || !k->codes_dev || !v->codes_dev ||
        !q->bias_dev || !k->bias_dev || !v->bias_dev)
        return set_err(NNRH_ERR_INVALID, "mha_codes: bad arguments");
    const uintptr_t a4 = (uintptr_t)q->codes_dev | (uintptr_t)k->codes_dev | (uintptr_t)v->codes_dev;
    const uintptr_t a16 = (uintptr_t)y | (uintptr_t)q->bias_dev | (uintptr_t)k->bias_dev | (uintptr_t)v->bias_dev;
    if (!mha_fused_shape(seq, hidden, num_heads) || (a4 & 3) || (a16 & 15))
        return set_err(NNRH_ERR_UNSUPPORTED, "mha_codes: the fused shapes (head size 64, seq <= 128) and alignment "
                                             "only");
    if (minmax_parts && ((uintptr_t)minmax_parts & 7)) return set_err(NNRH_ERR_INVALID, "mha_codes: parts alignment");
    ProfScope ps("multihead_attention", S(stream));
    HIP_TRY(launch_mha_codes_f32(dq_codes_arg(q), dq_codes_arg(k), dq_codes_arg(v), y, B, seq, hidden, num_heads,
                                 scale, minmax_parts, S(stream)),
            "mha_codes_f32");
    return NNRH_OK;
}

extern "C" int nnrh_cast_to_f32(const void* x, int x_dtype, float* y, size_t n, void* stream) {
    if (n && (!x || !y)) return set_err(NNRH_ERR_INVALID, "cast_to_f32: NULL");
    const int dt = x_dtype == NNRH_U8 ? 0 : x_dtype == NNRH_S8 ? 1 : x_dtype == NNRH_I32 ? 2 : -1;
    if (dt < 0) return set_err(NNRH_ERR_UNSUPPORTED, "cast_to_f32: source type");
    ProfScope ps("cast_f32", S(stream));
    HIP_TRY(launch_cast_to_f32(x, dt, y, (long long)n, S(stream)), "cast_to_f32");
    return NNRH_OK;
}

extern "C" int nnrh_hardswish_f32(const float* x, float* y, size_t n, int post_op, void* stream) {
    if (n && (!x || !y)) return set_err(NNRH_ERR_INVALID, "hardswish_f32: NULL");
    ProfScope ps("hardswish_f32", S(stream));
    HIP_TRY(launch_hardswish_f32(x, y, (long long)n, post_op ? 1 : 0, S(stream)), "hardswish_f32");
    return NNRH_OK;
}

extern "C" int nnrh_gelu_f32(const float* x, float* y, size_t n, void* stream) {
    if (n && (!x || !y)) return set_err(NNRH_ERR_INVALID, "gelu_f32: NULL");
    ProfScope ps("gelu_f32", S(stream));
    HIP_TRY(launch_gelu_f32(x, y, (long long)n, S(stream)), "gelu_f32");
    return NNRH_OK;
}

extern "C" int nnrh_transpose_f32(const float* x, float* y, int ndim, const int* dims, const int* perm,
                                  void* stream) {
    if (!x || !y || !dims || !perm || ndim < 1 || ndim > 6)
        return set_err(NNRH_ERR_INVALID, "transpose_f32: bad args");
    ProfScope ps("transpose_f32", S(stream));
    HIP_TRY(launch_transpose_f32(x, y, ndim, dims, perm, S(stream)), "transpose_f32");
    return NNRH_OK;
}

extern "C" int nnrh_clip_f32(const float* x, float* y, size_t n, float lo, float hi, void* stream) {
    if (n && (!x || !y)) return set_err(NNRH_ERR_INVALID, "clip_f32: NULL");
    ProfScope ps("clip_f32", S(stream));
    HIP_TRY(launch_clip_f32(x, y, (long long)n, lo, hi, S(stream)), "clip_f32");
    return NNRH_OK;
}
