/*
 * nnr_hip.h -- C ABI of the MI355X (gfx950) backend for NNR's int8 QDQ
 * compute path.
 *
 * The reference (beru/nnr) is a C++ runtime: operators implement
 * operator_t::init/reshape/exec (src/nnr.h:331-461) and are created through
 * registry_t::solve (src/registry.cpp:10-27). The HIP backend keeps that
 * operator interface in C++ (nnr_amd/host/) and every operator crosses into
 * device code through the functions below: plain pointers and sizes, int
 * status codes, no exceptions and no C++ or torch types.
 *
 * Conventions
 *   - Pointers named *_dev are device (HBM) pointers; *_host are host pointers.
 *   - `stream` is a hipStream_t passed as void*; NULL is the default stream.
 *   - All launches are asynchronous on `stream`; create/destroy calls are
 *     cold-path and may allocate device memory.
 *   - Quantized element types: NNRH_U8 / NNRH_S8 (activations), int8 weights.
 *   - Results are bit-identical to NNR's x64 (AVX-512 VNNI) CPU kernels:
 *     exact int32 accumulators and the same requantize formula per branch.
 */
#ifndef NNR_HIP_H
#define NNR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status ------------------------------------------------------------ */
enum {
    NNRH_OK = 0,
    NNRH_ERR_INVALID = 1,      /* bad argument / shape mismatch            */
    NNRH_ERR_UNSUPPORTED = 2,  /* valid ONNX, not handled by this backend  */
    NNRH_ERR_HIP = 3,          /* a HIP runtime call failed                */
    NNRH_ERR_NOMEM = 4
};
enum { NNRH_U8 = 0, NNRH_S8 = 1, NNRH_I32 = 2, NNRH_F32 = 3, NNRH_F16 = 4 };

/* Message of the last failing call on this thread (never NULL). */
const char* nnrh_last_error(void);
/* Library version string. */
const char* nnrh_version(void);

/* ---- device plumbing (the host framework includes no HIP headers) -------
 * Replaces the host allocations of the reference's memory planner
 * (src/memory_planner.cpp:282-331) and tensor_t::data ownership (src/nnr.h:236). */
int nnrh_device_count(int* count);
int nnrh_set_device(int device);
int nnrh_malloc(void** ptr_dev, size_t bytes);
int nnrh_free(void* ptr_dev);
/* kind: 0 host->device, 1 device->host, 2 device->device */
int nnrh_memcpy(void* dst, const void* src, size_t bytes, int kind, void* stream);
int nnrh_fill_u8(void* dst_dev, uint8_t value, size_t bytes, void* stream);
int nnrh_stream_create(void** stream);
int nnrh_stream_destroy(void* stream);
int nnrh_stream_synchronize(void* stream);
int nnrh_device_synchronize(void);
int nnrh_event_create(void** event);
int nnrh_event_destroy(void* event);
int nnrh_event_record(void* event, void* stream);
/* work enqueued on `stream` after this call waits for `event`'s last record */
int nnrh_stream_wait_event(void* stream, void* event);
int nnrh_event_elapsed_ms(float* ms, void* start, void* stop);

/* ---- whole-plan HIP graphs ----------------------------------------------
 * No counterpart in the reference, whose CPU runtime executes the nodes one
 * by one (src/nnr.cpp:908-1050). Launches issued on `stream` between
 * begin_capture and end_capture are recorded (thread-local capture mode:
 * a call that would allocate or synchronize fails the capture instead of
 * running) and instantiated as one executable graph. end_capture leaves
 * the stream out of capture either way and returns NNRH_OK with
 * *graph_exec set, or an error with *graph_exec NULL. `stream` must not be
 * the null stream.                                                         */
int nnrh_graph_begin_capture(void* stream);
int nnrh_graph_end_capture(void* stream, void** graph_exec);
int nnrh_graph_launch(void* graph_exec, void* stream);
int nnrh_graph_destroy(void* graph_exec);

/* ---- profiling ------------------------------------------------------------
 * Counterpart of context_t::enable_profiling / dump_profile (src/nnr.h:518-520,
 * src/nnr.cpp:801-846): when enabled, every kernel launch of this library is
 * bracketed by hipEvents on its stream and accumulated per kernel name.
 * Reading the totals synchronizes the recorded events. Entries named
 * "variant:<kernel<template arguments>>" count the launches of each GEMM
 * kernel instantiation (tile, stages, producer, epilogue) with no time.    */
int nnrh_profile_enable(int on);
/* 1 while the launch profiler records, else 0 */
int nnrh_profile_enabled(void);
int nnrh_profile_reset(void);
int nnrh_profile_count(int* n_kernels);
int nnrh_profile_get(int index, const char** name, int* launches, double* total_ms);

/* ---- QLinearConv ---------------------------------------------------------
 * Replaces QLinearConv_operator (src/backend/cpu/QLinearConv.cpp:30-1371):
 * init() attribute parsing (:91-156), reshape() weight pre-packing and
 * requantize vectors (QLinearConv_reshape.h:18-340), exec() dispatch over the
 * kernel branches (:1337-1368). Shapes use NCHW logical dims; x_nhwc / y_nhwc
 * give the physical layout (tensor_t::format, src/nnr.h:226).            */
typedef struct nnrh_qconv_desc {
    int N, C, H, W;                 /* input                                */
    int OC, kH, kW, group;          /* weights [OC][C/group][kH][kW]        */
    int sH, sW, dH, dW;
    int pad_t, pad_l, pad_b, pad_r; /* resolved pads (auto_pad applied)     */
    int oH, oW;
    int x_nhwc, y_nhwc;
    int post_fn;                    /* a unary op was fused (operator_t::post_fn) */
    int act_dtype;                  /* NNRH_U8 or NNRH_S8 (x and y)          */
    float x_scale; int x_zp;
    const float* w_scale_host; int w_scale_count;
    const int8_t* w_zp_host; int w_zp_count;
    float y_scale; int y_zp;
    const int8_t* w_host;           /* OIHW int8                            */
    const int32_t* bias_host;       /* [OC] or NULL                         */
    int spatial_dims;               /* 0 or 2: 4-D tensors; 1: 3-D tensors
                                       [N][C][W] (H = kH = 1, pads and strides
                                       along H unused, NCW layout), the
                                       reference's exec_typed path (RQ-S,
                                       QLinearConv.cpp:286-334)             */
} nnrh_qconv_desc;

/* kernel branch of QLinearConv::exec_simd_4d (QLinearConv.cpp:1337-1351) */
enum {
    NNRH_BR_DW = 1,          /* exec_dw_int8_nhwc         RQ-A [lo,hi]       */
    NNRH_BR_FIRST = 2,       /* exec_first_layer_int8     RQ-C (+RQ-A')      */
    NNRH_BR_DIRECT = 3,      /* exec_direct_int8          RQ-A qmin (+A')    */
    NNRH_BR_PACKED = 4,      /* exec_packed_nr48 (NR48)   RQ-B (+B')         */
    NNRH_BR_NR16 = 5,        /* exec_packed_nr48 (NR16)   RQ-B               */
    NNRH_BR_IM2COL_S1 = 6,   /* exec_vnni_im2col, stride1 RQ-A [lo,hi]       */
    NNRH_BR_IM2COL = 7,      /* exec_vnni_im2col, tiled   RQ-A qmin (+A')    */
    NNRH_BR_FLOAT = 8,       /* exec_float_fallback       RQ-A qmin (+A')    */
    NNRH_BR_TYPED = 9        /* exec_typed, 3-D tensors   RQ-S               */
};

typedef struct nnrh_qconv* nnrh_qconv_t;
/* Branch the reference would take for this descriptor (no allocation). */
int nnrh_qconv_dispatch(const nnrh_qconv_desc* d, int* branch);
/* reshape(): validates, packs weights on the device, precomputes requantize
 * vectors. Host arrays in `d` are only read during the call.             */
int nnrh_qconv_create(nnrh_qconv_t* h, const nnrh_qconv_desc* d);
int nnrh_qconv_branch(nnrh_qconv_t h, int* branch);
/* exec(): x_dev / y_dev in the layouts given at create time.            */
int nnrh_qconv_run(nnrh_qconv_t h, const void* x_dev, void* y_dev, void* stream);
int nnrh_qconv_destroy(nnrh_qconv_t h);

/* QLinearConv followed by a same-shape QLinearAdd of its output, in one
 * kernel. No counterpart in the reference, which never fuses a binary Add
 * into a conv (src/graph_optimizer/fuse_post_ops.cpp:67); the result is
 * identical to nnrh_qconv_run then nnrh_qlinear_add(kind 0): the conv byte
 * and the other operand go through QLinearAdd's RQ-E body / scalar-tail
 * expressions (src/backend/cpu/QLinearAdd.cpp:66-104) with the same element
 * split. conv_is_a: 1 when the conv output is the add's input A. Available
 * for the RQ-B branches (PACKED, NR16) with group 1, NHWC output and
 * output channels % 16 == 0 and a uint8 output; otherwise returns
 * NNRH_ERR_UNSUPPORTED and leaves the handle unchanged. After a successful
 * call, run with nnrh_qconv_run_add; other_dev must be 16-byte aligned.   */
typedef struct nnrh_qadd_fuse_desc {
    int conv_is_a;
    float a_scale; int a_zp;
    float b_scale; int b_zp;
    float y_scale; int y_zp;
} nnrh_qadd_fuse_desc;
int nnrh_qconv_fuse_add(nnrh_qconv_t h, const nnrh_qadd_fuse_desc* d);
int nnrh_qconv_run_add(nnrh_qconv_t h, const void* x_dev, const void* other_dev,
                       void* y_dev, void* stream);
/* No counterpart in the reference: the QuantizeLinear that produces a
 * first-layer conv's uint8 input (QuantizeLinear.cpp:128-194, per-tensor
 * scale and uint8 zero point) runs inside the kernel that lays the input out
 * for the conv, reading the fp32 NCHW tensor directly: one pass over it
 * instead of a quantize pass and a layout pass. Every byte equals
 * QuantizeLinear's (same body / tail split by flat index). Only for the
 * first-layer branch with its multi-copy input (nnrh_qconv_branch FIRST
 * on uint8 NCHW input); otherwise NNRH_ERR_UNSUPPORTED. After a successful
 * call the handle runs with nnrh_qconv_run_f32 only.                      */
int nnrh_qconv_fuse_quantize(nnrh_qconv_t h, float scale, int zero_point);
int nnrh_qconv_run_f32(nnrh_qconv_t h, const float* x_dev, void* y_dev, void* stream);
/* No counterpart in the reference: the MaxPool that reads a first-layer
 * conv's uint8 NHWC output (3x3 window, stride 2, padding 1, no dilation,
 * floor mode: ResNet's) runs inside the conv's one kernel, which then writes
 * only the pooled tensor [N][pH][pW][OC], pH = (oH - 1) / 2 + 1 (pW alike).
 * Every byte equals nnrh_maxpool_u8_nhwc over the conv's output (the uint8
 * MaxPool of src/backend/cpu/MaxPool.cpp after fuse_qdq). Only for the
 * one-kernel first layer (FIRST branch, NHWC uint8 output, 16..64 output
 * channels, output rows of at most 112 pixels, 7x7-class kernels with four
 * MFMA K steps); otherwise NNRH_ERR_UNSUPPORTED and the handle is unchanged.
 * After a successful call nnrh_qconv_run / nnrh_qconv_run_f32 (when the
 * quantize is fused too) write the pooled tensor; x and y must be 16-byte
 * aligned. */
int nnrh_qconv_fuse_maxpool(nnrh_qconv_t h, int kH, int kW, int sH, int sW, int pad_t, int pad_l,
                            int pad_b, int pad_r);

/* ---- QLinearMatMul ------------------------------------------------------
 * Replaces QLinearMatMul_operator (src/backend/cpu/QLinearMatMul.cpp:14-233)
 * for a constant B: reshape() pre-pack (:75-91), exec() (:111-232).
 * Only b_scale[0] / b_zp[0] are used, as in the reference (:118-119).
 * A: [batch][m][k], Y: [batch][m][n] row-major; B: [k][n] constant.
 * Scales: scale_dtype NNRH_F32 or NNRH_F16 (fp16 combined scale, :125-132).*/
typedef struct nnrh_qmatmul_desc {
    int m, n, k;
    int a_dtype;                    /* NNRH_U8 / NNRH_S8                      */
    int b_dtype;                    /* NNRH_U8 / NNRH_S8                      */
    int y_dtype;                    /* NNRH_U8 / NNRH_S8                      */
    int scale_dtype;                /* NNRH_F32 / NNRH_F16                    */
    const void* a_scale_host; const void* a_zp_host;   /* may be overridden per run */
    const void* b_scale_host; const void* b_zp_host;
    const void* y_scale_host; const void* y_zp_host;
    const void* b_host;             /* [k][n]                                 */
} nnrh_qmatmul_desc;
typedef struct nnrh_qmatmul* nnrh_qmatmul_t;
int nnrh_qmatmul_create(nnrh_qmatmul_t* h, const nnrh_qmatmul_desc* d);
/* a_scale_dev (float32) / a_zp_dev (a_dtype) override the create-time A
 * quantization with device values, e.g. from DynamicQuantizeLinear; NULL
 * keeps the create-time ones. a_batch_stride = 0 broadcasts A.          */
int nnrh_qmatmul_run(nnrh_qmatmul_t h, const void* a_dev, long long a_batch_stride,
                     void* y_dev, int batch, const float* a_scale_dev,
                     const void* a_zp_dev, void* stream);
/* QLinearMatMul followed by DequantizeLinear of its output (zero point y_zp,
 * scale dq_scale) and an fp32 Add of a per-column vector bias[n] (NULL: 0),
 * in one kernel; after a successful call nnrh_qmatmul_run writes float32
 * y = fl(fl((q - y_zp) * dq_scale) + bias[col]), identical to running the
 * three operators (DequantizeLinear.cpp:133-152, binary_math.cpp). No
 * counterpart in the reference, which keeps them separate. Needs float32
 * scales, K % 16 == 0, b_zp such that no row-sum term is needed;
 * NNRH_ERR_UNSUPPORTED otherwise (the handle is unchanged).             */
int nnrh_qmatmul_fuse_dq_bias(nnrh_qmatmul_t h, float dq_scale, int dq_zp, const float* bias_host);
/* After nnrh_qmatmul_fuse_dq_bias: the float32 result then goes through
 * Gelu, erf form (src/backend/cpu/Gelu.cpp:43-47), the same expression as
 * nnrh_gelu_f32, so the bits equal running the Gelu operator after it. No
 * counterpart in the reference (a fusion of operators it runs one by one). */
int nnrh_qmatmul_fuse_gelu(nnrh_qmatmul_t h);
/* After nnrh_qmatmul_fuse_dq_bias: every run also writes (min, max) pairs of
 * its float32 outputs (0 stands in where a pair saw only larger / smaller
 * values) to parts_dev, for nnrh_dynamic_quantize_linear_parts on y; count
 * gives the pairs a run of `batch` writes, capacity is the buffer's size in
 * pairs (a run needing more fails), parts_dev NULL turns it off. No
 * counterpart in the reference: it saves DynamicQuantizeLinear's min/max
 * pass over y (DynamicQuantizeLinear.cpp:37-41).                          */
int nnrh_qmatmul_minmax_count(nnrh_qmatmul_t h, int batch, int* count);
int nnrh_qmatmul_set_minmax_out(nnrh_qmatmul_t h, float* parts_dev, int capacity);
/* After nnrh_qmatmul_fuse_dq_bias (+ _fuse_gelu) and _set_minmax_out, for a
 * chain whose float32 result is read only by a DynamicQuantizeLinear
 * (DynamicQuantizeLinear.cpp:27-58 on the output of QLinearMatMul.cpp:
 * 188-198 -> DequantizeLinear -> Add [-> Gelu]): on = 1 makes
 * nnrh_qmatmul_run write, instead of the float32 values, the uint8
 * QLinearMatMul bytes they are computed from (y then holds batch x m x n
 * bytes, same element layout) together with the values' (min, max) pairs.
 * (Without _set_minmax_out, and without Gelu, the bytes serve the readers
 * of nnrh_dq_codes below.)
 * nnrh_qmatmul_dynamic_quantize_codes then writes the DynamicQuantizeLinear
 * outputs (y, y_scale, y_zp of the run's batch) from those bytes: the chain
 * value of byte q in column j depends on (j, q) alone, so a per-column table
 * of the 256 quantized values (built after the pairs give the scale / zero
 * point) maps every byte, and the results equal running the chain and the
 * quantizer on the float32 values bit for bit. The handle owns the table
 * (256 x n rounded up to 64 bytes, allocated here when the pairs are set:
 * call _set_minmax_out first); a handle in codes mode serves one run at a
 * time (the table is rebuilt by each quantize call). A later fuse_dq_bias /
 * fuse_gelu turns codes mode off; on = 0 returns to float32 output. No
 * counterpart in the reference, which materializes the float32 tensor
 * between the operators.                                                  */
int nnrh_qmatmul_set_codes_out(nnrh_qmatmul_t h, int on);
/* The chain's dequantize parameters for a reader of its bytes (no Gelu):
 * zero point, scale and the handle's device bias vector (padded to a
 * multiple of 64 columns, 16-byte aligned, valid while the handle lives). */
int nnrh_qmatmul_dq_params(nnrh_qmatmul_t h, int* zp, float* dq_scale, const float** bias_dev);
int nnrh_qmatmul_dynamic_quantize_codes(nnrh_qmatmul_t h, const void* codes_dev, int batch, uint8_t* y_dev,
                                        float* y_scale_dev, uint8_t* y_zp_dev, void* stream);
/* 2..4 QLinearMatMuls, each with nnrh_qmatmul_fuse_dq_bias (no Gelu, no
 * min/max output), identical in shape and types and reading the same A (a
 * transformer layer's Q, K and V projections), run as one launch: the
 * members' weights, column sums and biases are copied side by side at
 * create (the member handles stay valid and unchanged). group_run takes A
 * as `rows` x k uint8 / int8 rows and writes member i's float32 result to
 * ys[i] (rows x n), each equal to nnrh_qmatmul_run of that member over the
 * same rows. No counterpart in the reference (each QLinearMatMul runs alone,
 * QLinearMatMul.cpp:155-227); it fills the GPU with 3x the tiles.          */
typedef struct nnrh_qmatmul_group* nnrh_qmatmul_group_t;
int nnrh_qmatmul_group_create(nnrh_qmatmul_group_t* h, const nnrh_qmatmul_t* members, int n);
int nnrh_qmatmul_group_run(nnrh_qmatmul_group_t h, const void* a_dev, int rows, void* const* y_devs,
                           const float* a_scale_dev, const void* a_zp_dev, void* stream);
/* The group's launch writes the members' uint8 QLinearMatMul bytes instead
 * of their fp32 chain values (as nnrh_qmatmul_set_codes_out; the members'
 * own handles give the readers their nnrh_qmatmul_dq_params).            */
int nnrh_qmatmul_group_set_codes_out(nnrh_qmatmul_group_t h, int on);
int nnrh_qmatmul_group_destroy(nnrh_qmatmul_group_t h);
int nnrh_qmatmul_destroy(nnrh_qmatmul_t h);

/* ---- MatMulInteger ------------------------------------------------------
 * Replaces MatMulInteger_operator (src/backend/cpu/MatMulInteger.cpp:11-150):
 * y[b][m][n] = sum_k (a - a_zp)(b - b_zp) in int32; both operands on the
 * device, B packed per call (the reference packs per exec, :120).
 * Strides are in elements; a stride of 0 broadcasts that operand.        */
typedef struct nnrh_matmul_integer* nnrh_matmul_integer_t;
int nnrh_matmul_integer_create(nnrh_matmul_integer_t* h, int m, int n, int k,
                               int a_dtype, int b_dtype, int max_batch);
int nnrh_matmul_integer_run(nnrh_matmul_integer_t h, const void* a_dev,
                            long long a_batch_stride, const void* b_dev,
                            long long b_batch_stride, int a_zp, int b_zp,
                            int32_t* y_dev, int batch, void* stream);
/* As nnrh_matmul_integer_run with A's zero point read from device memory
 * (one byte of A's type, e.g. the zero point DynamicQuantizeLinear wrote),
 * so the call never waits for the device.                                 */
int nnrh_matmul_integer_run_dev_zp(nnrh_matmul_integer_t h, const void* a_dev,
                                   long long a_batch_stride, const void* b_dev,
                                   long long b_batch_stride, const void* a_zp_dev, int b_zp,
                                   int32_t* y_dev, int batch, void* stream);
int nnrh_matmul_integer_destroy(nnrh_matmul_integer_t h);

/* MatMulInteger with a constant B, followed by Cast(to float), Mul by the
 * per-column scale product fl(a_scale * w_scale[n]) and an fp32 Add of
 * bias[n]: the per-channel dynamic-quantization pattern
 * DynamicQuantizeLinear -> MatMulInteger -> Cast -> Mul(Mul(a_scale,
 * w_scale)) -> Add. No counterpart in the reference, which runs MatMulInteger
 * (src/backend/cpu/MatMulInteger.cpp:11-150), Cast and the binary Mul / Add
 * (binary_math.cpp) one by one; the kernel forms
 *   y = fl(fl(float(acc) * fl(a_scale * w_scale[n])) + bias[n]),
 * acc = sum_k (a - a_zp)(b - b_zp) exact, so the bits equal theirs. Returns
 * an nnrh_qmatmul handle: run with nnrh_qmatmul_run (a_scale_dev / a_zp_dev
 * from DynamicQuantizeLinear replace the desc's a_scale / a_zp), and
 * nnrh_qmatmul_fuse_gelu, nnrh_qmatmul_minmax_count / _set_minmax_out and
 * nnrh_qmatmul_group_create (members all of this kind) apply as after
 * nnrh_qmatmul_fuse_dq_bias. Needs K % 16 == 0 and b_zp = 0 (int8 B) or 128
 * (uint8 B); NNRH_ERR_UNSUPPORTED otherwise.                                */
typedef struct nnrh_mmi_scaled_desc {
    int m, n, k;
    int a_dtype;                 /* NNRH_U8 / NNRH_S8                          */
    int b_dtype;                 /* NNRH_U8 / NNRH_S8                          */
    const void* b_host;          /* [k][n]                                    */
    int a_zp, b_zp;
    float a_scale;
    const float* w_scale_host;   /* [n]                                       */
    const float* bias_host;      /* [n], or NULL when no Add follows           */
} nnrh_mmi_scaled_desc;
int nnrh_matmul_integer_scaled_create(nnrh_qmatmul_t* h, const nnrh_mmi_scaled_desc* d);

/* ---- ConvInteger ----------------------------------------------------------
 * Replaces ConvInteger_operator's 4-D path (src/backend/cpu/ConvInteger.cpp:
 * 146-233): y[n][oc][oh][ow] = sum (x - x_zp)(w - w_zp[oc]) in int32, NCHW.
 * x / w uint8 or int8 (NNRH_U8 / NNRH_S8), w [OC][C/group][kH][kW]. The
 * reference accumulates in fp32 (im2col + float GEMM) and rounds; that equals
 * this exact integer result whenever K * max|x - x_zp| * max|w - w_zp| <=
 * 2^24 (K = C/group * kH * kW), where every partial sum is exact in float.
 * Output extents and pads are the caller's (the operator's auto_pad rules).
 * w_zp_dev: per-output-channel zero points (int32 [OC], device) or NULL for
 * the scalar w_zp. Runs as an implicit GEMM (no im2col in memory); the
 * handle owns an NHWC copy of the input, the weights packed per call and
 * the per-pixel patch sums. create returns NNRH_ERR_UNSUPPORTED when
 * C/group (padded to 16) * kH * kW > 32768 or N * oH * oW > 2^30.         */
typedef struct nnrh_conv_integer* nnrh_conv_integer_t;
int nnrh_conv_integer_create(nnrh_conv_integer_t* h, int N, int C, int iH, int iW, int OC,
                             int kH, int kW, int sH, int sW, int pH, int pW, int dH, int dW,
                             int oH, int oW, int group, int x_dtype, int w_dtype);
int nnrh_conv_integer_run(nnrh_conv_integer_t h, const void* x_dev, const void* w_dev, int x_zp,
                          int w_zp, const int32_t* w_zp_dev, int32_t* y_dev, void* stream);
int nnrh_conv_integer_destroy(nnrh_conv_integer_t h);

/* ---- QuantizeLinear / DequantizeLinear / DynamicQuantizeLinear ----------
 * QuantizeLinear.cpp:128-194 (per-tensor uint8/int8), DequantizeLinear.cpp:
 * 100-152, DynamicQuantizeLinear.cpp:27-58.                              */
int nnrh_quantize_linear(const float* x_dev, size_t n, float scale, int zp,
                         int y_dtype, void* y_dev, void* stream);
int nnrh_dequantize_linear(const void* x_dev, int x_dtype, size_t n, float scale,
                           int zp, float* y_dev, void* stream);
size_t nnrh_dynamic_quantize_workspace(void);
int nnrh_dynamic_quantize_linear(const float* x_dev, size_t n, uint8_t* y_dev,
                                 float* y_scale_dev, uint8_t* y_zp_dev,
                                 void* workspace_dev, void* stream);
/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): nnrh_dynamic_quantize_linear without the workspace
 * argument. Its min / max partials live in one 8 KiB device array of the
 * library (a copy per GPU, held until the process ends); the call allocates
 * nothing. Same scale, zero point and bytes as nnrh_dynamic_quantize_linear.
 * Calls that overlap on one GPU (other streams, other threads) share that
 * array and race; serialize them. n above NNRH_DYNQ_NOALLOC_MAX_N is
 * rejected with NNRH_ERR_INVALID. The first call on a device looks up that
 * device's array address (hipGetSymbolAddress): make it once, eagerly,
 * before capturing the call into a HIP graph.                              */
#define NNRH_DYNQ_NOALLOC_MAX_N ((size_t)1 << 40)
int nnrh_dynamic_quantize_linear_noalloc(const float* x_dev, size_t n, uint8_t* y_dev,
                                         float* y_scale_dev, uint8_t* y_zp_dev, void* stream);
/* DynamicQuantizeLinear whose min / max were found by the operator that wrote
 * x: parts_dev holds nparts (min, max) pairs covering all of x (written by
 * nnrh_add_layernorm_f32 or a fused-dequantize nnrh_qmatmul_run). Same
 * scale, zero point and bytes as nnrh_dynamic_quantize_linear (min and max
 * are exact in any order). No counterpart in the reference.               */
int nnrh_dynamic_quantize_linear_parts(const float* x_dev, size_t n, const float* parts_dev,
                                       int nparts, uint8_t* y_dev, float* y_scale_dev,
                                       uint8_t* y_zp_dev, void* stream);

/* ---- QLinearAdd ----------------------------------------------------------
 * QLinearAdd_operator::exec_typed (src/backend/cpu/QLinearAdd.cpp:33-265).
 * kind: 0 same shape, 1 B scalar, 2 A scalar, 3 per-channel (B is [C]).
 * Per-channel: y is [N][C][HW] logical, y_nhwc gives the physical layout. */
int nnrh_qlinear_add(int kind, const void* a_dev, const void* b_dev, void* y_dev,
                     size_t n, int C, int HW, int y_nhwc, int dtype,
                     float a_scale, int a_zp, float b_scale, int b_zp,
                     float y_scale, int y_zp, void* stream);

/* ---- the rest of the QLinear family (QOperator models) --------------------
 * QLinearMul_operator::exec_typed (src/backend/cpu/QLinearMul.cpp:25-231):
 * kind / layout arguments as nnrh_qlinear_add (3: a is the full tensor, b the
 * [C] one; pass the per-channel operand as b with its scale / zero point).
 * Bit-exact with the reference's 16-wide body and scalar tail.             */
int nnrh_qlinear_mul(int kind, const void* a_dev, const void* b_dev, void* y_dev,
                     size_t n, int C, int HW, int y_nhwc, int dtype,
                     float a_scale, int a_zp, float b_scale, int b_zp,
                     float y_scale, int y_zp, void* stream);
/* QLinearGlobalAveragePool (src/backend/cpu/QLinearGlobalAveragePool.cpp:
 * 38-60): x [N][C][spatial] (or [N][spatial][C] with x_nhwc) -> y [N][C]. */
int nnrh_qlinear_global_avgpool(const void* x_dev, void* y_dev, int N, int C, int spatial,
                                int x_nhwc, int dtype, float x_scale, int x_zp,
                                float y_scale, int y_zp, void* stream);
/* QLinearAveragePool (src/backend/cpu/QLinearAveragePool.cpp:67-115): 2-D,
 * in-image taps counted (count_include_pad is never set, :41-42); NCHW or
 * NHWC (nhwc) in and out; pads are the leading ones, oH / oW the caller's. */
int nnrh_qlinear_avgpool(const void* x_dev, void* y_dev, int N, int C, int iH, int iW,
                         int oH, int oW, int kH, int kW, int sH, int sW, int pH, int pW,
                         int nhwc, int dtype, float x_scale, int x_zp, float y_scale,
                         int y_zp, void* stream);
/* One input of QLinearConcat (src/backend/cpu/QLinearConcat.cpp:70-236):
 * `outer` chunks of `count` elements of x go to y at o * y_row + y_off,
 * copied when the input has the output's scale and zero point, requantized
 * otherwise (16-wide body / scalar tail within each chunk). A concat along
 * axis a calls this once per input with outer = prod(dims[:a]), count =
 * dims_t[a] * inner; along channels of NHWC tensors, outer = N*H*W.        */
int nnrh_qlinear_concat_part(const void* x_dev, void* y_dev, long long outer, long long count,
                             long long y_row, long long y_off, int dtype, float x_scale,
                             int x_zp, float y_scale, int y_zp, void* stream);
/* The whole QLinearConcat in one launch: ntens parts (host arrays of device
 * pointers, chunk lengths, scales and zero points), each contributing
 * `counts[t]` elements to every one of the `outer` output rows, in order.
 * Same arithmetic as nnrh_qlinear_concat_part per part.                     */
int nnrh_qlinear_concat(int ntens, const void* const* xs_dev, const long long* counts,
                        const float* x_scales, const int* x_zps, long long outer, int dtype,
                        float y_scale, int y_zp, void* y_dev, void* stream);

/* ---- BatchNormalization after fold_bn_qdq (src/graph_optimizer/
 * fold_bn_qdq.cpp:23-259; BatchNormalization.cpp:246-376) ---------------------
 * y[n,c,...] = uint8(A[c] * x + B[c]) with the reference's rounding per layout
 * (NCHW: 16-wide body of each plane fma + clamp + nearest-even, tail
 * x*A + B + clamp + roundf; NHWC: body of each pixel's channels fma +
 * nearest-even + unsigned saturation -- negatives become 255 for uint8 input,
 * clamped first for fp32 input -- tail A*x + B + clamp + lrintf). x is uint8
 * (DQ->BN->Q folded) or, with x_is_f32, fp32 (BN->Q folded). a, b: device
 * [C]. HW: product of the dimensions after C.                                */
int nnrh_batchnorm_u8(const void* x_dev, int x_is_f32, uint8_t* y_dev, const float* a_dev,
                      const float* b_dev, long long N, int C, long long HW, int nhwc, void* stream);
/* inference BatchNormalization in fp32 (BatchNormalization.cpp:126-160):
 * y = alpha[c] * x + beta[c], alpha = scale / sqrt(var + eps) (double),
 * beta = bias - alpha * mean, both computed by the caller                    */
int nnrh_batchnorm_f32(const float* x_dev, float* y_dev, const float* alpha_dev,
                       const float* beta_dev, long long N, int C, long long HW, int nhwc,
                       void* stream);

/* ---- uint8 MaxPool, NHWC (src/backend/x64/pool_x64.h:396-436) ----------- */
int nnrh_maxpool_u8_nhwc(const uint8_t* x_dev, uint8_t* y_dev, int N, int C,
                         int iH, int iW, int oH, int oW, int kH, int kW, int sH,
                         int sW, int pH, int pW, void* stream);

/* ---- layout: NCHW -> NHWC uint8 (transpose_nchw_nhwc_u8.h:1-126) -------- */
int nnrh_nchw_to_nhwc_u8(const uint8_t* x_dev, uint8_t* y_dev, int N, int C,
                         int HW, void* stream);

/* ---- fp32 glue of the configuration graphs ------------------------------
 * GlobalAveragePool (src/backend/cpu/global_pool.cpp): x [N][C][HW] or
 * [N][HW][C] (x_nhwc) -> y [N][C].                                        */
int nnrh_global_avgpool_f32(const float* x_dev, float* y_dev, int N, int C, int HW,
                            int x_nhwc, void* stream);
/* com.microsoft MultiHeadAttention (src/backend/cpu/MultiHeadAttention.cpp,
 * no mask): q, k, v, y are [B][seq][hidden] fp32 with hidden = num_heads *
 * head_dim; y = softmax(scale * Q_h K_h^T) V_h per (batch, head), with the
 * heads read and written in place. Head size 64 with seq <= 128 (and q, k,
 * v, y 16-byte aligned) runs as one fused fp32-MFMA kernel per (batch,
 * head) and needs no workspace (NULL is accepted); other shapes use batched
 * GEMMs and a scaled softmax over a workspace of at least
 * nnrh_multihead_attention_workspace bytes, 256-byte aligned. The size is 0
 * for the fused shapes. minmax_parts (optional, NULL for none; no
 * counterpart in the reference): the fused kernel also writes (min, max)
 * pairs of y for a DynamicQuantizeLinear that reads it
 * (nnrh_dynamic_quantize_linear_parts), nnrh_multihead_attention_minmax_count
 * of them (0 for shapes without the fused kernel, which reject the buffer). */
int nnrh_multihead_attention_workspace(int B, int seq, int hidden, int num_heads, size_t* bytes);
int nnrh_multihead_attention_minmax_count(int B, int seq, int hidden, int num_heads, int* pairs);
int nnrh_multihead_attention_f32(const float* q_dev, const float* k_dev, const float* v_dev, float* y_dev,
                                 int B, int seq, int hidden, int num_heads, float scale,
                                 float* minmax_parts_dev, void* workspace_dev, void* stream);
/* A fused QLinearMatMul -> DequantizeLinear -> Add(bias) chain stored as its
 * uint8 QLinearMatMul bytes (nnrh_qmatmul_set_codes_out, no Gelu): element
 * j of a row, byte b, stands for fl(fl((b - zp) * scale) + bias[j]), which
 * the readers below form exactly as the GEMM would have stored it. bias: the
 * producer's device vector (nnrh_qmatmul_dq_params), 16-byte aligned. No
 * counterpart in the reference, which materializes the fp32 tensor.      */
typedef struct nnrh_dq_codes {
    const uint8_t* codes_dev;
    int zp;
    float scale;
    const float* bias_dev;
} nnrh_dq_codes;
/* nnrh_multihead_attention_f32's fused kernel (head size 64, seq <= 128;
 * y 16-byte aligned, the byte tensors 4-byte aligned) with q, k, v given as
 * chain bytes: the same y bit for bit as on their fp32 values; other shapes
 * are rejected (NNRH_ERR_UNSUPPORTED).                                    */
int nnrh_multihead_attention_codes_f32(const nnrh_dq_codes* q, const nnrh_dq_codes* k, const nnrh_dq_codes* v,
                                       float* y_dev, int B, int seq, int hidden, int num_heads, float scale,
                                       float* minmax_parts_dev, void* stream);
/* No counterpart in the reference: DequantizeLinear (DequantizeLinear.cpp:
 * 133-152, per-tensor scale and zero point, uint8 or int8 x) feeding
 * GlobalAveragePool, in one pass over the 8-bit tensor. Each value is
 * fl((q - zp) * s) and the sums run in nnrh_global_avgpool_f32's order, so
 * y equals the two operators run separately.                              */
int nnrh_global_avgpool_dequant(const void* x_dev, float* y_dev, int N, int C, int HW,
                                int x_nhwc, int x_dtype, float scale, int zero_point,
                                void* stream);
/* Gemm (src/backend/cpu/Gemm.cpp): Y = alpha*op(A)*op(B) + beta*C, row-major;
 * c_mode: 0 no C, 1 scalar, 2 [N], 3 [M][N], 4 [M] (broadcast per row).   */
int nnrh_gemm_f32(const float* a_dev, const float* b_dev, const float* c_dev, float* y_dev,
                  int M, int N, int K, int trans_a, int trans_b, float alpha, float beta,
                  int c_mode, void* stream);
/* Batched Gemm / MatMul (src/backend/cpu/MatMul.cpp broadcasting over the
 * leading axes): a, b, y advance by a/b/y_bstride elements per batch (0 =
 * shared), c is broadcast as in nnrh_gemm_f32.                           */
int nnrh_gemm_f32_batched(const float* a_dev, const float* b_dev, const float* c_dev, float* y_dev,
                          int M, int N, int K, int trans_a, int trans_b, float alpha, float beta,
                          int c_mode, int batch, long long a_bstride, long long b_bstride,
                          long long y_bstride, void* stream);
/* Add / Mul / Sub / Div (src/backend/cpu/binary_math.cpp), op 0..3:
 * y = a op b, or b op a with b_first; b_mode 0 same shape, 1 scalar b,
 * 2 b of D elements broadcast over the last axis (n % D == 0).            */
int nnrh_binary_f32(int op, const float* a_dev, const float* b_dev, float* y_dev, size_t n, int D,
                    int b_mode, int b_first, void* stream);
/* Softmax over the last axis (src/backend/cpu/Softmax.cpp, opset 13). */
int nnrh_softmax_f32(const float* x_dev, float* y_dev, size_t rows, int D, void* stream);
/* LayerNormalization over the last axis (src/backend/cpu/LayerNormalization.cpp:
 * mean, variance of the row, (x - mean) / sqrt(var + eps) * gamma + beta). */
int nnrh_layernorm_f32(const float* x_dev, const float* gamma_dev, const float* beta_dev,
                       float* y_dev, size_t rows, int D, float eps, void* stream);
/* LayerNormalization of fl(x + r) (r_dev NULL: of x): a same-shape fp32 Add
 * (src/backend/cpu/binary_math.cpp) folded into the normalization, so the
 * sum is never stored. parts_dev (NULL: none) receives one (min, max) pair
 * of the outputs per group of 4 rows (rows 4i .. 4i+3 -> pair i, ceil(rows
 * / 4) pairs), for nnrh_dynamic_quantize_linear_parts. No counterpart in the
 * reference, which runs Add and LayerNormalization.                      */
int nnrh_add_layernorm_f32(const float* x_dev, const float* r_dev, const float* gamma_dev,
                           const float* beta_dev, float* y_dev, size_t rows, int D, float eps,
                           float* parts_dev, void* stream);
/* nnrh_add_layernorm_f32 with x given as chain bytes (nnrh_dq_codes; its
 * columns are the normalized axis): the same y and pairs bit for bit as on
 * x's fp32 values.                                                        */
int nnrh_add_layernorm_codes_f32(const nnrh_dq_codes* x, const float* r_dev, const float* gamma_dev,
                                 const float* beta_dev, float* y_dev, size_t rows, int D, float eps,
                                 float* parts_dev, void* stream);
/* HardSwish, fp32 (src/backend/cpu/HardSwish.cpp:18-50): y = x * clamp(x/6 +
 * 0.5, 0, 1), the 16-wide body of the first n - n % 16 elements multiplying
 * by fl(1/6), the tail dividing by 6 (vec_ops_avx512.h:96-117). post_op: 1
 * when it runs as a producer's fused post-op (fuse_post_ops.cpp:61-68), which
 * adds the zero bias of bias_hardswish (vec_ops_avx512.h:74-94) first.     */
int nnrh_hardswish_f32(const float* x_dev, float* y_dev, size_t n, int post_op, void* stream);
/* Cast to float (src/backend/cpu/Cast.cpp, Cast_array: (float)x) from
 * NNRH_U8, NNRH_S8 or NNRH_I32 (int32 rounds to nearest, ties to even).    */
int nnrh_cast_to_f32(const void* x_dev, int x_dtype, float* y_dev, size_t n, void* stream);
/* Gelu, approximate = "none" (src/backend/cpu/Gelu.cpp:43-47). */
int nnrh_gelu_f32(const float* x_dev, float* y_dev, size_t n, void* stream);
/* Transpose (src/backend/cpu/Transpose.cpp): ndim <= 6 input dims and perm. */
int nnrh_transpose_f32(const float* x_dev, float* y_dev, int ndim, const int* dims_host,
                       const int* perm_host, void* stream);
/* Clip / Relu (src/backend/cpu/Clip.cpp, Relu.cpp): y = min(max(x, lo), hi) */
int nnrh_clip_f32(const float* x_dev, float* y_dev, size_t n, float lo, float hi, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* NNR_HIP_H */
