/*
 * nnr_host.h -- C ABI of the host framework (nnr_amd/host, libnnr_host.so).
 *
 * The reference's user-facing entry is context_t (src/nnr.h:482-612):
 * load() a model, prepare(), run(), then read outputs, with
 * preferred_backend choosing the operator implementations (nnr.h:589) and
 * enable_profiling()/dump_profile() (nnr.h:518-520). This header exposes the
 * same lifecycle over a C ABI for language bindings. The configurations are
 * synthetic graphs built in memory, so graph construction replaces the ONNX
 * loader: initializers, inputs, outputs and nodes are added one by one
 * exactly as onnx_build_graph does per NodeProto (onnx_loader.cpp:595-653).
 */
#ifndef NNR_HOST_H
#define NNR_HOST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct nnr_ctx* nnr_ctx_t;

/* backend ids (registry.h backend_t): 0 CPU, 4 HIP */
enum { NNR_BACKEND_CPU = 0, NNR_BACKEND_HIP = 4 };
/* attribute kinds */
enum { NNR_ATTR_INT = 0, NNR_ATTR_FLOAT = 1, NNR_ATTR_STRING = 2, NNR_ATTR_INTS = 3,
       NNR_ATTR_FLOATS = 4 };

const char* nnr_last_error(void);
int nnr_ctx_create(nnr_ctx_t* ctx, int preferred_backend);
int nnr_ctx_destroy(nnr_ctx_t ctx);
int nnr_ctx_set_stream(nnr_ctx_t ctx, void* stream);
/* Whole-plan HIP graph (default on; no counterpart in the reference's CPU
 * runtime): from its second call on, run() replays the plan's launches as
 * one graph captured on a private stream and launched on the context's
 * stream, with the same kernels and results as node-by-node launches. Off
 * while per-node profiling or the launch profiler records; a capture that
 * fails turns it off for the context. graph_active: 1 once a graph is in
 * use. */
int nnr_ctx_set_graph(nnr_ctx_t ctx, int on);
int nnr_ctx_graph_active(nnr_ctx_t ctx, int* on);
int nnr_ctx_set_fusion(nnr_ctx_t ctx, int on);
/* fuse_conv_add (default on, needs fusion on): same-shape QLinearAdds run in
 * the epilogue of the QLinearConv producing one operand; results unchanged. */
int nnr_ctx_set_conv_add(nnr_ctx_t ctx, int on);
/* fuse_dynq_codes and fuse_codes_readers (default on, need fusion and
 * conv_add on; no counterpart in the reference): a fused QLinearMatMul ->
 * DequantizeLinear -> Add [-> Gelu] chain whose fp32 result is read only by
 * an operator that can form it from the chain's uint8 QLinearMatMul bytes
 * (a DynamicQuantizeLinear; without Gelu also a LayerNormalization with its
 * residual Add or the fused MultiHeadAttention) stores those bytes instead
 * (that tensor then reads back as uint8), and the reader's outputs are the
 * same bit for bit. Off: the fp32 tensors are materialized. Set before
 * prepare(). */
int nnr_ctx_set_codes(nnr_ctx_t ctx, int on);

/* dtype: the reference's data_type_t (src/nnr.h:20-56): 1 FLOAT32, 3 FLOAT16,
 * 5 INT8, 6 INT16, 7 INT32, 8 INT64, 9 UINT8, 10 UINT16, 13 BOOL; other
 * codes fail. (ONNX TensorProto codes are translated by the ONNX loader.) */
int nnr_ctx_add_initializer(nnr_ctx_t ctx, const char* name, int dtype, const int* dims,
                            int ndim, const void* host_data);
int nnr_ctx_add_input(nnr_ctx_t ctx, const char* name, int dtype, const int* dims, int ndim);
int nnr_ctx_add_output(nnr_ctx_t ctx, const char* name);
/* attributes: parallel arrays; for each attribute i, kinds[i] selects the
 * value: INT -> ints[offs[i]], FLOAT -> floats[offs[i]], INTS/FLOATS ->
 * counts[i] values from offs[i], STRING -> strings[i]. */
int nnr_ctx_add_node(nnr_ctx_t ctx, const char* op_type, const char* name, int n_in,
                     const char* const* inputs, int n_out, const char* const* outputs, int n_attr,
                     const char* const* attr_names, const int* kinds, const int* counts,
                     const int* offs, const int64_t* ints, const float* floats,
                     const char* const* strings);

/* graph passes, shape inference and layout assignment only: no device
 * memory, no kernel state (usable without a GPU) */
int nnr_ctx_optimize(nnr_ctx_t ctx);
int nnr_ctx_prepare(nnr_ctx_t ctx);
int nnr_ctx_run(nnr_ctx_t ctx);

/* Concurrent contexts (no counterpart in the reference, whose contexts run
 * one at a time on the calling thread). A group runs n prepared contexts as
 * one step: run() makes each context's stream wait for the work already
 * enqueued on `stream`, runs every context on its own stream (a HIP graph
 * replay once captured), and makes `stream` wait for all of them. With one
 * context per slice of a batch (each built for batch / n, inputs and outputs
 * its own), the slices' kernels share the GPU: one slice's short, latency-
 * bound launches fill the CUs another slice's leave idle. Each context keeps
 * its own results, identical to running it alone. The contexts must be
 * distinct, each with its own non-null stream; a group does not own them
 * (destroy the group first). */
typedef struct nnr_group* nnr_group_t;
int nnr_group_create(const nnr_ctx_t* ctxs, int n, nnr_group_t* group);
int nnr_group_run(nnr_group_t group, void* stream);
int nnr_group_destroy(nnr_group_t group);

/* device pointer, dtype, dims and layout (0 NCHW, 1 NHWC) of a tensor */
int nnr_ctx_tensor(nnr_ctx_t ctx, const char* name, void** data_dev, int* dtype, int* dims,
                   int* ndim, int* format);

/* executed plan after prepare(): active node i */
int nnr_ctx_node_count(nnr_ctx_t ctx, int* n);
int nnr_ctx_node_info(nnr_ctx_t ctx, int i, const char** op_type, const char** name,
                      const char** variant, int* post_fn, int* n_in, int* n_out);
int nnr_ctx_node_io(nnr_ctx_t ctx, int i, int is_output, int j, const char** tensor_name);
/* Same-shape QLinearAdd folded into active node i's kernel (fuse_conv_add,
 * no counterpart in the reference). j = -1: the add node's name; j = -2: the
 * operand the conv reads besides its input; j = 0..7: the add's inputs
 * (slot 0 or 3 is the conv result, which no longer exists as a tensor).
 * "" when nothing was folded into node i. */
int nnr_ctx_node_fused_add(nnr_ctx_t ctx, int i, int j, const char** tensor_name);
/* Graph nodes folded into active node i's kernel after it (e.g. the
 * DequantizeLinear and bias Add after a QLinearMatMul), k = 0, 1, ...; ""
 * past the last. No counterpart in the reference. */
int nnr_ctx_node_fused_chain(nnr_ctx_t ctx, int i, int k, const char** node_name);
/* Graph nodes folded into active node i's kernel before it (a
 * QuantizeLinear feeding a first-layer QLinearConv, a DequantizeLinear
 * feeding GlobalAveragePool), k = 0, 1, ...; "" past the last. Node i then
 * reads the first one's input. No counterpart in the reference. */
int nnr_ctx_node_fused_pre(nnr_ctx_t ctx, int i, int k, const char** node_name);
int nnr_ctx_fusion_stat(nnr_ctx_t ctx, const char* key, int* value);
size_t nnr_ctx_device_bytes(nnr_ctx_t ctx);
/* Bytes of the context's shared operator workspace (the reference's
 * context_t::workspace_size, src/nnr.h:557-558): the largest scratch one
 * active operator's exec needs, allocated once by prepare and included in
 * nnr_ctx_device_bytes; 0 when no operator needs scratch. */
size_t nnr_ctx_workspace_bytes(nnr_ctx_t ctx);

/* Load an ONNX model (ModelProto bytes) into an empty context: the
 * replacement of the reference's load_onnx (src/format/onnx/onnx_loader.cpp:
 * 658-732) building the graph through the calls above. model_dir: where
 * external-data "location"s are relative to (NULL / "" = the working
 * directory). sym_dim: value for symbolic input dimensions (<= 0: 1, as the
 * reference's tensor_from_value_info does, :394-409). Constant nodes become
 * initializers. Errors (malformed protobuf, unsupported tensor types, missing
 * external files) return nonzero with nnr_last_error() set. */
int nnr_ctx_load_onnx(nnr_ctx_t ctx, const void* data, size_t size, const char* model_dir, int sym_dim);
/* the same from a file; external data relative to the file's directory
 * (context_t::load_from_file, src/nnr.cpp) */
int nnr_ctx_load_onnx_file(nnr_ctx_t ctx, const char* path, int sym_dim);
/* the host copy of an initializer (as loaded or added; graph passes that
 * rewrite constants update it). No counterpart in the reference: for tests
 * and tools that compare a loaded model with an in-process build. */
int nnr_ctx_initializer(nnr_ctx_t ctx, const char* name, const void** host, size_t* nbytes);
/* graph inputs (is_output 0) / outputs (1) in declaration order
 * (context_t::graph_inputs / graph_outputs, src/nnr.h) */
int nnr_ctx_graph_io_count(nnr_ctx_t ctx, int is_output, int* n);
int nnr_ctx_graph_io(nnr_ctx_t ctx, int is_output, int i, const char** name);

/* Device memory planning (context_t::enable_memory_planning, src/nnr.h:523-529;
 * memory_planner_t::analyze / plan / apply, src/memory_planner.cpp:33-331).
 * Off by default, as in the reference; set before prepare(). Intermediates
 * whose lifetimes over the executed plan do not overlap share slots of one
 * device arena (256-byte-aligned offsets); same-size elementwise operators
 * write over an input read for the last time; the copied parts of a
 * QLinearConcat along an axis with unit dimensions before it live inside its
 * output. Graph inputs and outputs, initializers and tensors under 256 bytes
 * are never pooled. Intermediate tensors then hold valid data only until
 * their slot's next tenant is written. */
int nnr_ctx_set_memory_planning(nnr_ctx_t ctx, int on);
/* the plan without device memory, after optimize() alone (the fusions that
 * need built operators are not in it), or the applied plan after prepare() */
int nnr_ctx_plan_memory(nnr_ctx_t ctx);
int nnr_ctx_memory_stats(nnr_ctx_t ctx, int* n_intermediates, int* n_slots, int* n_inplace, int* n_concat,
                         unsigned long long* pool_bytes, unsigned long long* unpooled_bytes);
/* pooled tensor i: live over node positions [first, last]; arena byte
 * offset and size; kind 0 own slot, 1 in place over `parent`, 2 inside the
 * QLinearConcat output `parent` (parent: another entry's index, or -1) */
int nnr_ctx_memory_entry(nnr_ctx_t ctx, int i, const char** name, int* first, int* last,
                         unsigned long long* offset, unsigned long long* bytes, int* kind, int* parent);

/* per-node hipEvent timing (context_t::enable_profiling / dump_profile) */
int nnr_ctx_enable_profiling(nnr_ctx_t ctx, int on);
int nnr_ctx_profile(nnr_ctx_t ctx, int i, double* total_ms, int* runs, double* ops,
                    double* bytes);
/* average device time (ms) of active node i (plan order) run `reps` times
 * back to back between two events on the context's stream: a kernel's
 * duration without per-launch event overhead (the node's inputs must hold
 * data, i.e. after one run()) */
int nnr_ctx_time_node(nnr_ctx_t ctx, int i, int reps, double* ms);

#ifdef __cplusplus
}
#endif
#endif /* NNR_HOST_H */
