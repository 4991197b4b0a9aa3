// core.cpp -- tensor_t / operator_t / context_t / registry_t of the host
// framework (counterparts of src/nnr.cpp and src/registry.cpp).
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <unordered_map>
#include <unordered_set>

#include "nnr.h"
#include "nnr_hip.h"
#include "registry.h"

namespace nnr {

size_t data_type_sizeof(data_type_t t) {
    switch (t) {
    case NNR_DATA_TYPE_FLOAT32: case NNR_DATA_TYPE_INT32: return 4;
    case NNR_DATA_TYPE_UINT8: case NNR_DATA_TYPE_INT8: case NNR_DATA_TYPE_BOOL: return 1;
    case NNR_DATA_TYPE_UINT16: case NNR_DATA_TYPE_INT16: case NNR_DATA_TYPE_FLOAT16: return 2;
    case NNR_DATA_TYPE_INT64: return 8;
    default: return 0;
    }
}

data_type_t data_type_from_onnx(int onnx) {
    // TensorProto.DataType codes (onnx.proto3 TensorProto.DataType)
    static const data_type_t table[] = {
        NNR_DATA_TYPE_UNDEFINED,      NNR_DATA_TYPE_FLOAT32,        NNR_DATA_TYPE_UINT8,
        NNR_DATA_TYPE_INT8,           NNR_DATA_TYPE_UINT16,         NNR_DATA_TYPE_INT16,
        NNR_DATA_TYPE_INT32,          NNR_DATA_TYPE_INT64,          NNR_DATA_TYPE_STRING,
        NNR_DATA_TYPE_BOOL,           NNR_DATA_TYPE_FLOAT16,        NNR_DATA_TYPE_FLOAT64,
        NNR_DATA_TYPE_UINT32,         NNR_DATA_TYPE_UINT64,         NNR_DATA_TYPE_COMPLEX64,
        NNR_DATA_TYPE_COMPLEX128,     NNR_DATA_TYPE_BFLOAT16,       NNR_DATA_TYPE_FLOAT8E4M3FN,
        NNR_DATA_TYPE_FLOAT8E4M3FNUZ, NNR_DATA_TYPE_FLOAT8E5M2,     NNR_DATA_TYPE_FLOAT8E5M2FNUZ,
        NNR_DATA_TYPE_UINT4,          NNR_DATA_TYPE_INT4,           NNR_DATA_TYPE_FLOAT4E2M1,
        NNR_DATA_TYPE_FLOAT8E8M0,     NNR_DATA_TYPE_UINT2,          NNR_DATA_TYPE_INT2,
    };
    if (onnx < 0 || onnx >= (int)(sizeof(table) / sizeof(table[0]))) return NNR_DATA_TYPE_UNDEFINED;
    return table[onnx];
}

// product of dims, or false when a dimension is negative or the element
// count or its byte size would not fit in size_t
bool checked_count(const std::vector<int>& d, size_t elem_size, size_t* count) {
    size_t n = 1;
    for (int v : d) {
        if (v < 0) return false;
        if (v != 0 && n > SIZE_MAX / (size_t)v) return false;
        n *= (size_t)v;
    }
    if (elem_size && n > SIZE_MAX / elem_size) return false;
    *count = n;
    return true;
}

// ---- tensor_t --------------------------------------------------------------
bool tensor_t::reshape(const std::vector<int>& d, data_type_t t) {
    size_t n = 0;
    if (!checked_count(d, data_type_sizeof(t), &n)) return false;
    dims = d;
    type = t;
    ndata = n;
    return true;
}

float tensor_t::scalar_f32() const {
    if (host.empty()) return 0.0f;
    if (type == NNR_DATA_TYPE_FLOAT32) return *(const float*)host.data();
    return 0.0f;
}

int32_t tensor_t::scalar_int() const {
    if (host.empty()) return 0;
    switch (type) {
    case NNR_DATA_TYPE_UINT8: return *(const uint8_t*)host.data();
    case NNR_DATA_TYPE_INT8: return *(const int8_t*)host.data();
    case NNR_DATA_TYPE_INT32: return *(const int32_t*)host.data();
    case NNR_DATA_TYPE_INT64: return (int32_t)*(const int64_t*)host.data();
    default: return 0;
    }
}

// ---- operator_t ------------------------------------------------------------
bool operator_t::reshape() {
    if (inputs.empty() || outputs.empty() || !inputs[0] || !outputs[0]) return false;
    outputs[0]->format = inputs[0]->format;
    return outputs[0]->reshape(inputs[0]->dims, inputs[0]->type);
}

double operator_t::num_bytes() const {
    // a tensor given as two inputs (QLinearMul of x with x) is read once
    double b = 0;
    for (size_t i = 0; i < inputs.size(); ++i) {
        tensor_t* t = inputs[i];
        bool dup = false;
        for (size_t j = 0; j < i && !dup; ++j) dup = inputs[j] == t;
        if (t && !dup) b += (double)t->nbytes();
    }
    for (auto* t : outputs)
        if (t) b += (double)t->nbytes();
    return b;
}

const attr_t* operator_t::find_attr(const std::string& name) const {
    for (auto& kv : attrs)
        if (kv.first == name) return &kv.second;
    return nullptr;
}
int64_t operator_t::attribute(const std::string& name, int64_t def) const {
    const attr_t* a = find_attr(name);
    return a && a->kind == attr_t::kind_t::INT ? a->i : def;
}
float operator_t::attribute_f(const std::string& name, float def) const {
    const attr_t* a = find_attr(name);
    return a && a->kind == attr_t::kind_t::FLOAT ? a->f : def;
}
std::string operator_t::attribute_s(const std::string& name, const std::string& def) const {
    const attr_t* a = find_attr(name);
    return a && a->kind == attr_t::kind_t::STRING ? a->s : def;
}
std::vector<int64_t> operator_t::attribute_ints(const std::string& name) const {
    const attr_t* a = find_attr(name);
    return a && a->kind == attr_t::kind_t::INTS ? a->ints : std::vector<int64_t>{};
}

// ---- registry --------------------------------------------------------------
void registry_t::register_op(const std::string& name, backend_t b, resolver_fn fn) {
    ops_[{name, b}] = fn;
}
bool registry_t::has(const std::string& name, backend_t b) const {
    return ops_.count({name, b}) != 0;
}
operator_t* registry_t::solve(const std::string& op_type, int opset, pool_t& pool, backend_t preferred) {
    if (preferred != backend_t::CPU) {
        auto it = ops_.find({op_type, preferred});
        if (it != ops_.end()) {
            operator_t* op = it->second(opset, pool);
            if (op) return op;
        }
    }
    auto it = ops_.find({op_type, backend_t::CPU});
    if (it != ops_.end()) return it->second(opset, pool);
    return nullptr;
}
registry_t& global_registry() {
    static registry_t r;
    return r;
}
operator_t* solve_operator(const std::string& op_type, int opset, pool_t& pool, backend_t preferred) {
    return global_registry().solve(op_type, opset, pool, preferred);
}

// ---- pool_t ----------------------------------------------------------------
pool_t::~pool_t() {
    for (char* b : blocks_) ::operator delete(b);
}
void* pool_t::alloc(size_t size, size_t align) {
    if (size == 0) size = 1;
    if (size + align > BlockSize) {   // a block of its own, kept before the current one
        char* b = (char*)::operator new(size + align);
        blocks_.insert(blocks_.empty() ? blocks_.end() : blocks_.end() - 1, b);
        return (void*)(((uintptr_t)b + align - 1) & ~(uintptr_t)(align - 1));
    }
    if (!blocks_.empty()) {
        uintptr_t base = (uintptr_t)blocks_.back();
        uintptr_t p = (base + used_ + align - 1) & ~(uintptr_t)(align - 1);
        if (p + size <= base + BlockSize) {
            used_ = p + size - base;
            return (void*)p;
        }
    }
    char* b = (char*)::operator new(BlockSize);
    blocks_.push_back(b);
    uintptr_t p = ((uintptr_t)b + align - 1) & ~(uintptr_t)(align - 1);
    used_ = p + size - (uintptr_t)b;
    return (void*)p;
}

// ---- context_t -------------------------------------------------------------
context_t::context_t() = default;

context_t::~context_t() {
    if (graph_exec_) nnrh_graph_destroy(graph_exec_);
    if (cap_stream_) nnrh_stream_destroy(cap_stream_);
    for (auto& e : events_) {
        nnrh_event_destroy(e.first);
        nnrh_event_destroy(e.second);
    }
    for (void* p : allocations_) nnrh_free(p);
    for (auto* n : nodes) destroy_op(n);
    for (auto& kv : map) delete kv.second;
}

bool context_t::fail(const std::string& msg) {
    last_error = msg;
    return false;
}

tensor_t* context_t::find(const std::string& name) const {
    auto it = map.find(name);
    return it == map.end() ? nullptr : it->second;
}

tensor_t* context_t::tensor(const std::string& name) {
    if (name.empty()) return nullptr;
    auto it = map.find(name);
    if (it != map.end()) return it->second;
    tensor_t* t = new tensor_t();
    t->name = name;
    map[name] = t;
    return t;
}

bool context_t::add_initializer(const std::string& name, data_type_t t, const std::vector<int>& dims,
                                const void* host_data) {
    tensor_t* x = tensor(name);
    if (!x || !x->reshape(dims, t) || data_type_sizeof(t) == 0)
        return fail("initializer " + name + ": bad type or dims");
    x->host.assign((const uint8_t*)host_data, (const uint8_t*)host_data + x->nbytes());
    initializer_names.insert(name);
    return true;
}

bool context_t::add_input(const std::string& name, data_type_t t, const std::vector<int>& dims) {
    tensor_t* x = tensor(name);
    if (!x || !x->reshape(dims, t) || data_type_sizeof(t) == 0) return fail("input " + name + ": bad type or dims");
    graph_inputs.push_back(name);
    return true;
}

bool context_t::add_output(const std::string& name) {
    tensor(name);
    graph_outputs.push_back(name);
    return true;
}

bool context_t::add_node(const std::string& op_type, const std::string& name,
                         const std::vector<std::string>& ins, const std::vector<std::string>& outs,
                         std::vector<std::pair<std::string, attr_t>> attrs) {
    // onnx_loader.cpp:595-653: resolve through the registry, wire, init()
    operator_t* op = solve_operator(op_type, opset, attr_pool, preferred_backend);
    if (!op) op = pool_new<unresolved_op_t>(attr_pool);
    op->ctx = this;
    op->opset = opset;
    op->op_type = op_type;
    op->node_name = name;
    for (auto& s : ins) op->inputs.push_back(s.empty() ? nullptr : tensor(s));
    for (auto& s : outs) op->outputs.push_back(tensor(s));
    op->attrs = std::move(attrs);
    if (!op->init())
        fprintf(stderr, "[nnr] init failed: %s (%s)\n", name.c_str(), op_type.c_str());
    nodes.push_back(op);
    return true;
}

void* context_t::device_alloc(size_t bytes) {
    void* p = nullptr;
    if (nnrh_malloc(&p, bytes) != NNRH_OK) return nullptr;
    allocations_.push_back(p);
    device_bytes += bytes;
    return p;
}

// Device memory: with enable_memory_planning the planner places the
// intermediates in one shared arena; every other active, non-constant,
// non-view tensor gets its own device allocation (first-touch order). Views
// alias their source.
bool context_t::plan_memory_dry() {
    if (prepared) return true;
    if (!optimized && !optimize()) return false;
    planner.analyze(this);
    planner.plan();
    return true;
}

bool context_t::plan_memory() {
    // pooled intermediates first (one arena); everything else below gets an
    // allocation of its own
    if (enable_memory_planning) {
        planner.analyze(this);
        planner.plan();
        if (!planner.apply()) return false;
        device_bytes += planner.total_pool_bytes;
    }
    std::vector<tensor_t*> order;
    std::unordered_set<tensor_t*> seen;
    auto want = [&](tensor_t* t) {
        if (!t || seen.count(t)) return;
        seen.insert(t);
        order.push_back(t);
    };
    for (auto& n : graph_inputs) want(find(n));
    for (auto* op : nodes) {
        if (op->skip || op->folded) continue;
        for (auto* t : op->inputs) want(t);
        for (auto* t : op->outputs) want(t);
    }
    // a graph output no active node writes is the output of a skipped
    // post-op step: an alias of its producer's buffer, resolved below
    for (auto& n : graph_outputs) want(find(n));
    for (auto* t : order) {
        if (t->data) continue;
        if (t->alias_of) continue;
        size_t bytes = t->nbytes();
        if (bytes == 0) continue;
        void* p = nullptr;
        size_t rounded = (bytes + 255) & ~size_t(255);
        if (nnrh_malloc(&p, rounded) != NNRH_OK)
            return fail(std::string("device allocation failed for ") + t->name + ": " + nnrh_last_error());
        allocations_.push_back(p);
        device_bytes += rounded;
        t->data = p;
        t->owns_data = true;
        if (!t->host.empty() && t->host.size() == bytes) {
            if (nnrh_memcpy(p, t->host.data(), bytes, 0, stream) != NNRH_OK)
                return fail(std::string("upload failed: ") + nnrh_last_error());
        }
    }
    // resolve views after their sources have memory
    for (auto* t : order) {
        if (!t->alias_of) continue;
        tensor_t* s = t->alias_of;
        while (s->alias_of) s = s->alias_of;
        t->data = s->data;
        t->owns_data = false;
    }
    return true;
}

bool context_t::upload_constants() {
    return nnrh_stream_synchronize(stream) == NNRH_OK;
}

// Host evaluation of a folded DequantizeLinear over an initializer
// (fold_run executing constant subgraphs, src/nnr.cpp:1278-1376).
static bool fold_dequantize_host(operator_t* op) {
    tensor_t* x = op->inputs[0];
    tensor_t* s = op->inputs.size() > 1 ? op->inputs[1] : nullptr;
    tensor_t* z = op->inputs.size() > 2 ? op->inputs[2] : nullptr;
    tensor_t* y = op->outputs[0];
    if (!x || !x->has_host() || !s || !s->has_host()) return false;
    y->reshape(x->dims, NNR_DATA_TYPE_FLOAT32);
    y->host.resize(y->nbytes());
    float* py = (float*)y->host.data();
    const int axis = (int)op->attribute("axis", 1);
    const size_t ns = s->ndata;
    size_t inner = 1, ch = 1;
    if (ns > 1) {
        int a = axis < 0 ? axis + x->ndim() : axis;
        ch = (size_t)x->dims[a];
        for (int i = a + 1; i < x->ndim(); ++i) inner *= (size_t)x->dims[i];
    }
    for (size_t i = 0; i < x->ndata; ++i) {
        size_t c = ns > 1 ? (i / inner) % ch : 0;
        float sc = ((const float*)s->host.data())[c];
        int32_t zp = 0;
        if (z && z->has_host()) {
            size_t zi = z->ndata > 1 ? c : 0;
            zp = z->type == NNR_DATA_TYPE_UINT8 ? ((const uint8_t*)z->host.data())[zi]
               : z->type == NNR_DATA_TYPE_INT8 ? ((const int8_t*)z->host.data())[zi]
               : ((const int32_t*)z->host.data())[zi];
        }
        int32_t q = x->type == NNR_DATA_TYPE_UINT8 ? ((const uint8_t*)x->host.data())[i]
                  : x->type == NNR_DATA_TYPE_INT8 ? ((const int8_t*)x->host.data())[i]
                  : ((const int32_t*)x->host.data())[i];
        float d = (float)q - (float)zp;
        py[i] = d * sc;
    }
    return true;
}

bool context_t::optimize() {
    if (optimized) return true;
    // 1. graph optimizer (pass_graph_optimizer.cpp:333-398): constant folding,
    //    QDQ fusion, post-op fusion
    // PREPROCESS (pass_graph_optimizer.cpp:333-343): DQ -> BN -> Q first
    if (enable_fusion) fold_bn_qdq(this);
    fold_constants(this);
    if (enable_fusion) {
        fuse_qdq_compute(this);
        fuse_qdq(this);
        fuse_post_ops(this);
        if (enable_conv_add) fuse_attention(this);
    }
    // 2. every active node must be executable here
    std::string missing;
    for (auto* op : nodes) {
        if (op->skip || op->folded) continue;
        if (!op->resolved) missing += " " + op->op_type + "(" + op->node_name + ")";
    }
    if (!missing.empty())
        return fail("operators without a HIP implementation remain after fusion:" + missing);
    // 3. folded constants that active nodes still read get host values
    {
        std::unordered_set<tensor_t*> needed, produced;
        for (auto* op : nodes) {
            if (op->skip || op->folded) continue;
            for (auto* t : op->inputs)
                if (t) needed.insert(t);
            for (auto* t : op->outputs)
                if (t) produced.insert(t);
        }
        for (auto* t : produced) needed.erase(t);
        for (auto* op : nodes) {
            if (!op->folded || op->outputs.empty() || !needed.count(op->outputs[0])) continue;
            if (op->outputs[0]->has_host()) continue;
            if (op->op_type != "DequantizeLinear" || !fold_dequantize_host(op))
                return fail("cannot fold constant node " + op->node_name + " (" + op->op_type + ")");
        }
    }
    // 4. shape inference, then layout assignment (assign_layouts.cpp)
    shape_only = true;
    for (auto* op : nodes) {
        if (op->skip || op->folded) continue;
        if (!op->reshape()) {
            shape_only = false;
            return fail("shape inference failed: " + op->node_name + " (" + op->op_type + "): " + last_error);
        }
    }
    assign_layouts(this);
    // skipped post-op steps forward their input (and its layout)
    for (auto* op : nodes)
        if (op->skip && !op->outputs.empty() && op->outputs[0]->alias_of) {
            tensor_t* src = op->outputs[0]->alias_of;
            op->outputs[0]->reshape(src->dims, src->type);
            op->outputs[0]->format = src->format;
        }
    // a second shape pass with final layouts fixes layout-dependent state
    // (the kernel branch each QLinearConv will take)
    for (auto* op : nodes) {
        if (op->skip || op->folded) continue;
        if (!op->reshape()) {
            shape_only = false;
            return fail("shape inference failed: " + op->node_name + " (" + op->op_type + "): " + last_error);
        }
    }
    shape_only = false;
    optimized = true;
    return true;
}

bool context_t::prepare() {
    if (prepared) return true;
    if (!optimize()) return false;
    // 5. final reshape in graph order (builds each operator's device state)
    for (auto* op : nodes) {
        if (op->skip || op->folded) continue;
        if (!op->reshape())
            return fail("reshape failed: " + op->node_name + " (" + op->op_type + "): " + last_error);
        int vi = op->view_input_index();
        if (vi >= 0 && op->inputs[vi] && !op->outputs.empty()) op->outputs[0]->alias_of = op->inputs[vi];
    }
    // 5b. residual adds into their producing convolutions' kernels
    if (enable_fusion && enable_conv_add) {
        fuse_conv_add(this);
        fuse_matmul_dq_bias(this);
        fuse_matmul_integer_scale(this);
        fuse_quant_prefix(this);
        fuse_conv_maxpool(this);
        fuse_add_layernorm(this);
        fuse_dynq_minmax(this);
        fuse_matmul_group(this);
        if (enable_codes) {
            fuse_dynq_codes(this);
            fuse_codes_readers(this);
        }
    }
    // 6. device memory and constant upload; the shared operator workspace is
    // sized after the fusions, which change what some operators need
    if (!plan_memory()) return false;
    size_t ws = 0;
    for (auto* op : nodes)
        if (!op->skip && !op->folded) ws = std::max(ws, op->workspace_size());
    if (ws) {
        workspace = device_alloc((ws + 255) & ~size_t(255));
        if (!workspace) return fail(std::string("workspace allocation failed: ") + nnrh_last_error());
        workspace_bytes = ws;
    }
    if (!upload_constants()) return fail(nnrh_last_error());
    profile.clear();
    for (auto* op : nodes) {
        if (op->skip || op->folded) continue;
        node_profile_t p;
        p.name = op->node_name;
        p.op_type = op->op_type;
        p.variant = op->variant();
        p.ops = op->num_ops();
        p.bytes = op->num_bytes();
        profile.push_back(p);
    }
    prepared = true;
    return true;
}

// run loop (src/nnr.cpp:908-1050): exec active nodes in order on `stream`
bool context_t::exec_all(bool profiled) {
    size_t pi = 0;
    for (auto* op : nodes) {
        if (op->skip || op->folded) continue;
        if (profiled) nnrh_event_record(events_[pi].first, stream);
        if (!op->exec())
            return fail("exec failed: " + op->node_name + " (" + op->op_type + "): " +
                        (last_error.empty() ? std::string(nnrh_last_error()) : last_error));
        if (profiled) nnrh_event_record(events_[pi].second, stream);
        ++pi;
    }
    return true;
}

// The plan's launches recorded once into a HIP graph on a private stream
// (every tensor keeps its device address from prepare() on, so the
// recorded arguments stay valid; inputs are copied into their buffers).
// Taken after one node-by-node run, which does each operator's first-call
// set-up. A capture that fails (an operator that allocates or synchronizes
// inside exec) turns graphs off for this context.
bool context_t::capture_graph() {
    if (!cap_stream_ && nnrh_stream_create(&cap_stream_) != NNRH_OK) return false;
    void* user = stream;
    stream = cap_stream_;
    bool ok = nnrh_graph_begin_capture(stream) == NNRH_OK;
    const bool ran = ok && exec_all(false);
    void* ge = nullptr;
    if (ok) ok = nnrh_graph_end_capture(stream, &ge) == NNRH_OK && ran && ge;
    stream = user;
    if (!ok) {
        if (ge) nnrh_graph_destroy(ge);
        last_error.clear();
        return false;
    }
    graph_exec_ = ge;
    return true;
}

bool context_t::run() {
    if (!prepared && !prepare()) return false;
    const bool graph = enable_graph && !enable_profiling && !graph_failed_ && !nnrh_profile_enabled();
    if (graph && !graph_exec_ && eager_runs_ > 0 && !capture_graph()) graph_failed_ = true;
    if (graph && graph_exec_) {
        if (nnrh_graph_launch(graph_exec_, stream) != NNRH_OK)
            return fail(std::string("graph launch failed: ") + nnrh_last_error());
        return true;
    }
    if (enable_profiling && events_.size() < profile.size()) {
        while (events_.size() < profile.size()) {
            void *a = nullptr, *b = nullptr;
            if (nnrh_event_create(&a) || nnrh_event_create(&b)) return fail(nnrh_last_error());
            events_.emplace_back(a, b);
        }
    }
    if (!exec_all(enable_profiling)) return false;
    ++eager_runs_;
    const size_t pi = profile.size();
    if (enable_profiling) {
        for (size_t i = 0; i < pi; ++i) {
            float ms = 0.f;
            if (nnrh_event_elapsed_ms(&ms, events_[i].first, events_[i].second) == NNRH_OK) {
                profile[i].ms += ms;
                profile[i].runs++;
            }
        }
    }
    return true;
}

bool context_t::time_node(int i, int reps, double* ms) {
    if (!prepared && !prepare()) return false;
    operator_t* op = nullptr;
    int pi = 0;
    for (auto* o : nodes) {
        if (o->skip || o->folded) continue;
        if (pi++ == i) {
            op = o;
            break;
        }
    }
    if (!op || reps < 1 || !ms) return fail("time_node: bad node index or repeat count");
    void *a = nullptr, *b = nullptr;
    if (nnrh_event_create(&a) || nnrh_event_create(&b)) {
        if (a) nnrh_event_destroy(a);
        return fail(nnrh_last_error());
    }
    bool okay = nnrh_event_record(a, stream) == NNRH_OK;
    for (int r = 0; okay && r < reps; ++r) okay = op->exec();
    okay = okay && nnrh_event_record(b, stream) == NNRH_OK && nnrh_stream_synchronize(stream) == NNRH_OK;
    float t = 0.0f;
    okay = okay && nnrh_event_elapsed_ms(&t, a, b) == NNRH_OK;
    nnrh_event_destroy(a);
    nnrh_event_destroy(b);
    if (!okay) return fail("time_node: " + op->node_name + ": " + nnrh_last_error());
    *ms = (double)t / reps;
    return true;
}

}  // namespace nnr
