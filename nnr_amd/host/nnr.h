// nnr.h -- host-side operator framework of the MI355X backend.
//
// Mirrors the reference's core interface (src/nnr.h:154-612, src/registry.h)
// so that graph builders, the graph optimizer and the run loop drive the HIP
// operators the way NNR drives its CPU ones:
//   tensor_t      dims / type / format / quantization metadata; `data` is a
//                 device (HBM) pointer, `host` keeps a host mirror for
//                 initializers because operators read scalar scales and zero
//                 points as *(float*)t->data (QLinearConv.cpp:395-398);
//   operator_t    init() / reshape() / exec() / layout_mask / post_fn;
//   context_t     graph, preferred_backend, prepare() / run(), profiling.
// Every device operation goes through the C ABI of include/nnr_hip.h; this
// library includes no HIP header.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <set>
#include <string>
#include <utility>
#include <vector>

#include "memory_planner.h"

namespace nnr {

// Element types, in the reference's data_type_t numbering and order
// (src/nnr.h:20-56), so a tensor_t::type from NNR means the same here. ONNX
// TensorProto codes are translated by the loader (data_type_from_onnx).
enum data_type_t : uint8_t {
    NNR_DATA_TYPE_UNDEFINED = 0,
    NNR_DATA_TYPE_FLOAT32,
    NNR_DATA_TYPE_FLOAT64,
    NNR_DATA_TYPE_FLOAT16,
    NNR_DATA_TYPE_BFLOAT16,
    NNR_DATA_TYPE_INT8,
    NNR_DATA_TYPE_INT16,
    NNR_DATA_TYPE_INT32,
    NNR_DATA_TYPE_INT64,
    NNR_DATA_TYPE_UINT8,
    NNR_DATA_TYPE_UINT16,
    NNR_DATA_TYPE_UINT32,
    NNR_DATA_TYPE_UINT64,
    NNR_DATA_TYPE_BOOL,
    NNR_DATA_TYPE_STRING,
    NNR_DATA_TYPE_COMPLEX64,
    NNR_DATA_TYPE_COMPLEX128,
    NNR_DATA_TYPE_FLOAT8E4M3FN,
    NNR_DATA_TYPE_FLOAT8E4M3FNUZ,
    NNR_DATA_TYPE_FLOAT8E5M2,
    NNR_DATA_TYPE_FLOAT8E5M2FNUZ,
    NNR_DATA_TYPE_FLOAT8E8M0,
    NNR_DATA_TYPE_UINT4,
    NNR_DATA_TYPE_INT4,
    NNR_DATA_TYPE_FLOAT4E2M1,
    NNR_DATA_TYPE_UINT2,
    NNR_DATA_TYPE_INT2,
    NNR_DATA_TYPE_SEQUENCE,
    NNR_DATA_TYPE_COUNT,
};
// ONNX TensorProto.DataType -> data_type_t (UNDEFINED for codes with no
// counterpart), as the reference's loader maps them (onnx_loader.cpp:28-58)
data_type_t data_type_from_onnx(int onnx_elem_type);
// 0 when this backend stores no element of that type in device memory
size_t data_type_sizeof(data_type_t t);
// element count of dims (false: a negative dimension, or a count or byte
// size past SIZE_MAX)
bool checked_count(const std::vector<int>& dims, size_t elem_size, size_t* count);

enum class memory_layout_t : uint8_t { NCHW = 0, NHWC = 1 };
constexpr uint8_t LAYOUT_NCHW = 1;
constexpr uint8_t LAYOUT_NHWC = 2;
constexpr uint8_t LAYOUT_ALL = 0xff;

struct context_t;

struct tensor_t {
    std::string name;
    data_type_t type = NNR_DATA_TYPE_UNDEFINED;
    memory_layout_t format = memory_layout_t::NCHW;
    std::vector<int> dims;
    size_t ndata = 0;
    void* data = nullptr;          // device pointer
    bool owns_data = true;         // false for views (Flatten / Reshape)
    tensor_t* alias_of = nullptr;  // view source
    std::vector<uint8_t> host;     // host mirror (initializers, folded constants)
    bool device_only = false;      // produced on the device every run (no host mirror)

    // quantization metadata (src/nnr.h:236-266)
    float quant_scale = 0.0f;
    int32_t quant_zero_point = 0;

    int ndim() const { return (int)dims.size(); }
    size_t nbytes() const { return ndata * data_type_sizeof(type); }
    bool reshape(const std::vector<int>& d, data_type_t t);
    bool has_host() const { return !host.empty(); }
    template <typename T> const T* h() const { return (const T*)host.data(); }
    // scalar accessors over the host mirror
    float scalar_f32() const;
    int32_t scalar_int() const;
    bool is_quantized() const { return quant_scale != 0.0f; }
    void set_quant(float s, int32_t zp) { quant_scale = s; quant_zero_point = zp; }
};

// Arena for operator objects, as the reference's pool_t (src/pool.h:16-60):
// resolvers placement-new operators into context_t::attr_pool, and the
// memory goes when the context does. Objects are not freed one by one; a
// replaced operator has its destructor run (destroy_op) so that the device
// memory it owns is released at once.
struct pool_t {
    static constexpr size_t BlockSize = 64 * 1024;
    pool_t() = default;
    pool_t(const pool_t&) = delete;
    pool_t& operator=(const pool_t&) = delete;
    ~pool_t();
    void* alloc(size_t size, size_t align = alignof(std::max_align_t));
    template <typename T>
    T* alloc_arr(size_t n) { return (T*)alloc(sizeof(T) * n, alignof(T)); }

private:
    std::vector<char*> blocks_;
    size_t used_ = BlockSize;   // bytes used in blocks_.back()
};

struct attr_t {
    enum class kind_t : uint8_t { INT = 0, FLOAT, STRING, INTS, FLOATS };
    kind_t kind = kind_t::INT;
    int64_t i = 0;
    float f = 0.0f;
    std::string s;
    std::vector<int64_t> ints;
    std::vector<float> floats;
};

struct operator_t {
    virtual ~operator_t() = default;

    context_t* ctx = nullptr;
    int opset = 13;
    std::string op_type;
    std::string node_name;
    std::vector<tensor_t*> inputs;
    std::vector<tensor_t*> outputs;
    std::vector<std::pair<std::string, attr_t>> attrs;

    virtual bool init() { return true; }
    // default: output has the input's shape and type (src/nnr.h:369-381)
    virtual bool reshape();
    virtual bool exec() = 0;
    // device scratch one exec needs; it lives only for that exec, so every
    // operator of the context shares one buffer, ctx->workspace, of the
    // largest size (src/nnr.h:384, src/nnr.cpp:1067-1069)
    virtual size_t workspace_size() const { return 0; }
    // algorithmic work of one exec (per-layer TOPS / GB/s reporting)
    virtual double num_ops() const { return 0.0; }
    virtual double num_bytes() const;
    // output aliases input[view_input_index()] (src/nnr.h:404)
    virtual int view_input_index() const { return -1; }
    // kernel branch / variant name for reports
    virtual std::string variant() const { return std::string(); }

    uint8_t layout_mask = LAYOUT_NCHW;
    bool skip = false;
    bool folded = false;
    bool resolved = true;         // false: placeholder for an op this backend lacks
    // fused unary post-op (src/nnr.h:437-442). For the int8 operators the
    // only effect is QLinearConv's qmin (QLinearConv.cpp:419).
    bool fusable_unary = false;   // set in init() by Relu / Clip / HardSwish
    bool post_fn = false;
    operator_t* fused_op = nullptr;
    // the fused unary applied in place to an fp32 producer's n outputs (the
    // reference's fusable_apply with no bias); false: not a post-op provider
    virtual bool apply_post(void* /*data_dev*/, size_t /*n*/) { return false; }
    // a same-shape QLinearAdd folded into this operator's kernel
    // (fuse_conv_add); the add node is skipped and its output is ours
    operator_t* fused_add = nullptr;
    tensor_t* fused_other = nullptr;
    // accept `add` (whose input conv_side, 0 or 3, is this operator's output)
    // into the kernel; false leaves everything unchanged
    virtual bool fuse_residual_add(operator_t* /*add*/, int /*conv_side*/) { return false; }
    // a 1x1, stride-1, unpadded, ungrouped convolution (a dense GEMM over
    // the NHWC pixels): its kernel takes a fused add at HBM rate, where a
    // strided or spatial one (implicit im2col) is slower with it
    virtual bool dense_pointwise() const { return false; }
    // nodes after this one whose work its kernel now does, in graph order
    // (fuse_matmul_dq_bias); they are skipped and the last one's output is ours
    std::vector<operator_t*> fused_chain;
    virtual bool fuse_dq_bias(operator_t* /*dq*/, operator_t* /*add*/) { return false; }
    // a MaxPool reading this operator's output (fuse_conv_maxpool): k, s =
    // window and strides (h, w), pads = (top, left, bottom, right)
    virtual bool fuse_maxpool(operator_t* /*pool*/, const int* /*k*/, const int* /*s*/, const int* /*pads*/) {
        return false;
    }
    // a MaxPool's resolved window, strides and pads (false: not a plain 2-D
    // MaxPool of this backend)
    virtual bool pool_params(int* /*k*/, int* /*s*/, int* /*pads*/) const { return false; }
    // nodes before this one whose work its kernel now does (fuse_quant_prefix):
    // they are skipped and this operator reads the first one's input
    std::vector<operator_t*> fused_pre;
    virtual bool fuse_quantize_input(operator_t* /*q*/) { return false; }
    virtual bool fuse_dequantize_input(operator_t* /*dq*/) { return false; }
    // a same-shape fp32 Add before this operator (fuse_add_layernorm): this
    // operator reads the Add's two inputs; the second one is fused_other
    virtual bool fuse_residual_input(operator_t* /*add*/) { return false; }
    // a Gelu after the fused dequantize + bias (fuse_matmul_dq_bias)
    virtual bool fuse_gelu(operator_t* /*gelu*/) { return false; }
    // (min, max) pairs this operator can write beside output 0 for a
    // DynamicQuantizeLinear that reads it (0: it cannot); set_minmax_out
    // hands over a buffer of that many pairs (fuse_dynq_minmax)
    virtual int minmax_pairs() const { return 0; }
    virtual bool set_minmax_out(float* /*parts*/, int /*pairs*/) { return false; }
    float* minmax_parts = nullptr;
    int minmax_count = 0;
    // DynamicQuantizeLinear: the producer that writes its input's min / max
    operator_t* minmax_src = nullptr;
    // fuse_dynq_codes: a producer with min / max pairs whose output is read
    // only by a DynamicQuantizeLinear stores, instead of its fp32 values, the
    // uint8 bytes they are computed from (set_codes_out; false: cannot), and
    // quantize_codes writes the quantizer's three outputs from them
    virtual bool set_codes_out(bool /*on*/) { return false; }
    virtual bool quantize_codes(tensor_t* /*y*/, tensor_t* /*y_scale*/, tensor_t* /*y_zp*/) { return false; }
    // a reader of a producer's chain bytes (DynamicQuantizeLinear,
    // LayerNormalization): that producer
    operator_t* codes_src = nullptr;
    // fuse_codes_readers: this operator's byte input `which` (its own
    // numbering) will hold the uint8 bytes of producer p's fused dequantize
    // chain, whose meaning p->codes_params gives; false: it cannot read them
    // (nothing recorded). p NULL clears what was recorded.
    virtual bool set_codes_input(int /*which*/, operator_t* /*p*/) { return false; }
    // a fused QLinearMatMul -> DequantizeLinear -> Add(bias) chain (no Gelu):
    // its zero point, scale and device bias vector
    virtual bool codes_params(int* /*zp*/, float* /*scale*/, const float** /*bias*/) const { return false; }
    // operators of one kind reading the same input, run as one launch
    // (fuse_matmul_group): the leader launches for all of group_members; a
    // member's exec does nothing (its output is written by the leader, which
    // runs first)
    virtual bool fuse_group(const std::vector<operator_t*>& /*members*/) { return false; }
    // may lead or join a grouped launch, and reads the same input (and its
    // quantization) as `other`
    virtual bool groupable() const { return false; }
    virtual bool same_group_input(const operator_t* /*other*/) const { return false; }
    // MatMulInteger with a constant B followed by Cast -> Mul by the scale
    // product Mul(a_scale, w_scale) [-> Add(bias)] (fuse_matmul_integer_scale):
    // the kernel forms the fp32 result; bias NULL when no Add follows
    virtual bool fuse_int_scale(tensor_t* /*a_scale*/, tensor_t* /*w_scale*/, tensor_t* /*bias*/) { return false; }
    // BatchNormalization whose scale / bias inputs now hold fold_bn_qdq's
    // combined per-channel A / B and whose output is uint8 (false: cannot)
    virtual bool fold_affine_u8() { return false; }
    virtual bool fold_affine_u8_possible() const { return false; }
    operator_t* group_leader = nullptr;
    std::vector<operator_t*> group_members;

    // attribute accessors
    const attr_t* find_attr(const std::string& name) const;
    int64_t attribute(const std::string& name, int64_t def) const;
    float attribute_f(const std::string& name, float def) const;
    std::string attribute_s(const std::string& name, const std::string& def) const;
    std::vector<int64_t> attribute_ints(const std::string& name) const;
};

// Placeholder for ops with no resolver on any backend (the reference's
// dummy op whose exec() returns false, onnx_loader.cpp:597-602). Graph
// passes may rewrite it away (e.g. DQ->Conv->Q into QLinearConv).
struct unresolved_op_t : operator_t {
    unresolved_op_t() { resolved = false; }
    bool reshape() override { return true; }
    bool exec() override { return false; }
};

enum class backend_t : uint8_t { CPU = 0, CUDA, SYCL, VULKAN, HIP };

struct node_profile_t {
    std::string name, op_type, variant;
    double ms = 0.0;
    int runs = 0;
    double ops = 0.0, bytes = 0.0;
};

struct context_t {
    context_t();
    ~context_t();
    context_t(const context_t&) = delete;
    context_t& operator=(const context_t&) = delete;

    // ---- graph construction (what the reference's ONNX loader does) ----
    tensor_t* tensor(const std::string& name);                  // get or create
    tensor_t* find(const std::string& name) const;
    bool add_initializer(const std::string& name, data_type_t t, const std::vector<int>& dims,
                         const void* host_data);
    bool add_input(const std::string& name, data_type_t t, const std::vector<int>& dims);
    bool add_output(const std::string& name);
    bool add_node(const std::string& op_type, const std::string& name,
                  const std::vector<std::string>& ins, const std::vector<std::string>& outs,
                  std::vector<std::pair<std::string, attr_t>> attrs);

    // ---- lifecycle (src/nnr.cpp:1378-1483) ----
    bool optimize();    // graph passes + shape inference + layouts (no device work)
    bool prepare();     // optimize, reshape, plan memory, upload constants
    // the memory plan without device memory: after optimize() alone (shapes
    // known, operators not built) or the applied plan after prepare()
    bool plan_memory_dry();
    bool run();         // execute active nodes in order on `stream`
    // average device time of the i-th active node run `reps` times back to
    // back between two events (no event between the repeats), in ms
    bool time_node(int i, int reps, double* ms);

    // ---- configuration (src/nnr.h:512-589) ----
    backend_t preferred_backend = backend_t::HIP;
    int opset = 13;               // default-domain opset of the operators (the model's)
    void* stream = nullptr;       // hipStream_t of every launch
    bool enable_fusion = true;
    bool enable_conv_add = true;  // fuse_conv_add / fuse_matmul_dq_bias after the operators are built
    // fuse_dynq_codes / fuse_codes_readers (need enable_conv_add): fused
    // dequantize chains store uint8 bytes for readers that form the values
    bool enable_codes = true;
    bool enable_profiling = false;
    // run() from its second call on replays the whole plan as one HIP graph
    // captured on a private stream (off while profiling; falls back to
    // node-by-node launches for good if the capture fails)
    bool enable_graph = true;
    bool graph_active() const { return graph_exec_ != nullptr; }
    bool shape_only = false;      // reshape() computes shapes only (pre-layout pass)
    // share device memory between intermediates (src/nnr.h:523-529; off by
    // default as in the reference). Set before prepare().
    bool enable_memory_planning = false;
    memory_planner_t planner;

    // ---- state ----
    pool_t attr_pool;             // operators live here (src/nnr.h:552)
    std::map<std::string, tensor_t*> map;
    std::vector<operator_t*> nodes;
    std::vector<std::string> graph_inputs, graph_outputs;
    std::set<std::string> initializer_names;
    std::vector<node_profile_t> profile;
    std::map<std::string, int> fusion_stats;
    std::string last_error;
    bool optimized = false;
    bool prepared = false;
    size_t device_bytes = 0;
    // the operators' shared scratch (src/nnr.h:557-558): max workspace_size()
    // over the active operators, allocated in prepare(); nullptr when 0
    void* workspace = nullptr;
    size_t workspace_bytes = 0;

    bool fail(const std::string& msg);
    // device memory that lives as long as the context (nullptr on failure)
    void* device_alloc(size_t bytes);

private:
    std::vector<void*> allocations_;
    std::vector<std::pair<void*, void*>> events_;   // per-node hipEvents (profiling)
    void* graph_exec_ = nullptr;   // the captured plan
    void* cap_stream_ = nullptr;   // the stream it was captured on
    int eager_runs_ = 0;
    bool graph_failed_ = false;
    bool exec_all(bool profiled);
    bool capture_graph();
    bool plan_memory();
    bool upload_constants();
};

// graph optimizer passes (nnr_amd/host/passes.cpp)
void fold_constants(context_t* ctx);
void fuse_qdq_compute(context_t* ctx);
void fuse_qdq(context_t* ctx);
void fuse_post_ops(context_t* ctx);
void assign_layouts(context_t* ctx);
void fuse_conv_add(context_t* ctx);
void fuse_matmul_dq_bias(context_t* ctx);
void fuse_matmul_integer_scale(context_t* ctx);
void fuse_quant_prefix(context_t* ctx);
void fuse_add_layernorm(context_t* ctx);
void fuse_conv_maxpool(context_t* ctx);
void fuse_matmul_group(context_t* ctx);
void fuse_dynq_minmax(context_t* ctx);
void fuse_dynq_codes(context_t* ctx);
void fuse_codes_readers(context_t* ctx);
void fuse_attention(context_t* ctx);
void fold_bn_qdq(context_t* ctx);

// ONNX ModelProto -> this context (nnr_amd/host/onnx_loader.cpp); sym_dim
// replaces symbolic input dimensions (<= 0: 1, as the reference does)
bool load_onnx(context_t* ctx, const void* data, size_t size, const std::string& model_dir, int sym_dim);
bool load_onnx_file(context_t* ctx, const std::string& path, int sym_dim);

// operator creation through the registry (src/backend/cpu/solve_operator.cpp:29-33);
// the operator is placed in `pool`
operator_t* solve_operator(const std::string& op_type, int opset, pool_t& pool, backend_t preferred);
// runs a pool-placed operator's destructor (its memory stays in the pool)
inline void destroy_op(operator_t* op) {
    if (op) op->~operator_t();
}

}  // namespace nnr
