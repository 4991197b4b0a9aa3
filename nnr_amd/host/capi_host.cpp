// capi_host.cpp -- implementation of include/nnr_host.h over context_t.
#include <cstring>
#include <exception>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "nnr.h"
#include "nnr_hip.h"
#include "nnr_host.h"

namespace nnr {
int hip_backend_op_count();
}

using namespace nnr;

struct nnr_ctx {
    context_t ctx;
    std::vector<operator_t*> plan;   // active nodes after prepare()
    std::string scratch;
};

namespace {
thread_local std::string g_err = "no error";
int err(const std::string& m) {
    g_err = m;
    return 1;
}
int ctx_err(nnr_ctx_t c) { return err(c->ctx.last_error); }
// Every entry point runs under this: no C++ exception (std::bad_alloc from a
// huge tensor, std::length_error, ...) crosses the C ABI; it becomes an
// error code and a message, as the reference's bool-returning calls would.
template <class F>
int guarded(const char* what, F&& f) {
    try {
        return f();
    } catch (const std::bad_alloc&) {
        return err(std::string(what) + ": out of host memory");
    } catch (const std::exception& e) {
        return err(std::string(what) + ": " + e.what());
    } catch (...) {
        return err(std::string(what) + ": unknown exception");
    }
}
}  // namespace

extern "C" {

const char* nnr_last_error(void) { return g_err.c_str(); }

int nnr_ctx_create(nnr_ctx_t* out, int backend) {
    return guarded("ctx_create", [&]() -> int {
        if (!out) return err("ctx is NULL");
        if (hip_backend_op_count() <= 0) return err("no HIP operators registered");
        nnr_ctx* c = new nnr_ctx();
        c->ctx.preferred_backend = (backend_t)backend;
        *out = c;
        return 0;
    });
}

int nnr_ctx_destroy(nnr_ctx_t c) {
    return guarded("ctx_destroy", [&]() -> int {
        delete c;
        return 0;
    });
}

int nnr_ctx_set_stream(nnr_ctx_t c, void* s) {
    return guarded("ctx_set_stream", [&]() -> int {
        if (!c) return err("ctx is NULL");
        c->ctx.stream = s;
        return 0;
    });
}

int nnr_ctx_set_graph(nnr_ctx_t c, int on) {
    return guarded("ctx_set_graph", [&]() -> int {
        if (!c) return err("ctx is NULL");
        c->ctx.enable_graph = on != 0;
        return 0;
    });
}

int nnr_ctx_graph_active(nnr_ctx_t c, int* on) {
    return guarded("ctx_graph_active", [&]() -> int {
        if (!c || !on) return err("graph_active: NULL argument");
        *on = c->ctx.enable_graph && c->ctx.graph_active() ? 1 : 0;
        return 0;
    });
}

int nnr_ctx_set_fusion(nnr_ctx_t c, int on) {
    return guarded("ctx_set_fusion", [&]() -> int {
        if (!c) return err("ctx is NULL");
        c->ctx.enable_fusion = on != 0;
        return 0;
    });
}

int nnr_ctx_set_conv_add(nnr_ctx_t c, int on) {
    return guarded("ctx_set_conv_add", [&]() -> int {
        if (!c) return err("ctx is NULL");
        c->ctx.enable_conv_add = on != 0;
        return 0;
    });
}

int nnr_ctx_set_codes(nnr_ctx_t c, int on) {
    return guarded("ctx_set_codes", [&]() -> int {
        if (!c) return err("ctx is NULL");
        c->ctx.enable_codes = on != 0;
        return 0;
    });
}

int nnr_ctx_load_onnx(nnr_ctx_t c, const void* data, size_t size, const char* model_dir, int sym_dim) {
    return guarded("ctx_load_onnx", [&]() -> int {
        if (!c || !data) return err("load_onnx: NULL argument");
        if (!nnr::load_onnx(&c->ctx, data, size, model_dir ? model_dir : "", sym_dim)) return err(c->ctx.last_error);
        return 0;
    });
}

int nnr_ctx_load_onnx_file(nnr_ctx_t c, const char* path, int sym_dim) {
    return guarded("ctx_load_onnx_file", [&]() -> int {
        if (!c || !path) return err("load_onnx_file: NULL argument");
        if (!nnr::load_onnx_file(&c->ctx, path, sym_dim)) return err(c->ctx.last_error);
        return 0;
    });
}

int nnr_ctx_initializer(nnr_ctx_t c, const char* name, const void** host, size_t* nbytes) {
    return guarded("ctx_initializer", [&]() -> int {
        if (!c || !name || !host || !nbytes) return err("initializer: NULL argument");
        if (!c->ctx.initializer_names.count(name)) return err(std::string("initializer: no initializer ") + name);
        const nnr::tensor_t* t = c->ctx.find(name);
        *host = t && t->has_host() ? t->host.data() : nullptr;
        *nbytes = t ? t->host.size() : 0;
        return 0;
    });
}

int nnr_ctx_graph_io_count(nnr_ctx_t c, int is_output, int* n) {
    return guarded("ctx_graph_io_count", [&]() -> int {
        if (!c || !n) return err("graph_io_count: NULL argument");
        *n = (int)(is_output ? c->ctx.graph_outputs.size() : c->ctx.graph_inputs.size());
        return 0;
    });
}

int nnr_ctx_graph_io(nnr_ctx_t c, int is_output, int i, const char** name) {
    return guarded("ctx_graph_io", [&]() -> int {
        if (!c || !name) return err("graph_io: NULL argument");
        const auto& v = is_output ? c->ctx.graph_outputs : c->ctx.graph_inputs;
        if (i < 0 || i >= (int)v.size()) return err("graph_io: index out of range");
        *name = v[i].c_str();
        return 0;
    });
}

int nnr_ctx_set_memory_planning(nnr_ctx_t c, int on) {
    return guarded("ctx_set_memory_planning", [&]() -> int {
        if (!c) return err("ctx is NULL");
        if (c->ctx.prepared) return err("set_memory_planning: the context is already prepared");
        c->ctx.enable_memory_planning = on != 0;
        return 0;
    });
}

int nnr_ctx_plan_memory(nnr_ctx_t c) {
    return guarded("ctx_plan_memory", [&]() -> int {
        if (!c) return err("ctx is NULL");
        if (!c->ctx.plan_memory_dry()) return err(c->ctx.last_error);
        return 0;
    });
}

int nnr_ctx_memory_stats(nnr_ctx_t c, int* n_intermediates, int* n_slots, int* n_inplace, int* n_concat,
                         unsigned long long* pool_bytes, unsigned long long* unpooled_bytes) {
    return guarded("ctx_memory_stats", [&]() -> int {
        if (!c || !n_intermediates || !n_slots || !n_inplace || !n_concat || !pool_bytes || !unpooled_bytes)
            return err("memory_stats: NULL argument");
        const auto& p = c->ctx.planner;
        *n_intermediates = p.num_intermediates;
        *n_slots = p.num_slots;
        *n_inplace = p.num_inplace;
        *n_concat = p.num_concat;
        *pool_bytes = p.total_pool_bytes;
        *unpooled_bytes = p.total_unpooled_bytes;
        return 0;
    });
}

int nnr_ctx_memory_entry(nnr_ctx_t c, int i, const char** name, int* first, int* last,
                         unsigned long long* offset, unsigned long long* bytes, int* kind, int* parent) {
    return guarded("ctx_memory_entry", [&]() -> int {
        if (!c || !name || !first || !last || !offset || !bytes || !kind || !parent)
            return err("memory_entry: NULL argument");
        const auto& L = c->ctx.planner.lifetimes;
        if (i < 0 || i >= (int)L.size()) return err("memory_entry: index out of range");
        const auto& lt = L[i];
        *name = lt.tensor->name.c_str();
        *first = lt.first;
        *last = lt.last;
        *offset = lt.offset;
        *bytes = lt.bytes;
        *kind = (int)lt.kind;
        *parent = lt.parent;
        return 0;
    });
}

int nnr_ctx_add_initializer(nnr_ctx_t c, const char* name, int dtype, const int* dims, int ndim,
                            const void* data) {
    return guarded("ctx_add_initializer", [&]() -> int {
        if (!c || !name || (ndim && !dims) || !data) return err("add_initializer: NULL argument");
        if (dtype <= 0 || dtype >= NNR_DATA_TYPE_COUNT) return err("add_initializer: bad data_type_t");
        std::vector<int> d(dims, dims + ndim);
        if (!c->ctx.add_initializer(name, (data_type_t)dtype, d, data)) return ctx_err(c);
        return 0;
    });
}

int nnr_ctx_add_input(nnr_ctx_t c, const char* name, int dtype, const int* dims, int ndim) {
    return guarded("ctx_add_input", [&]() -> int {
        if (!c || !name || (ndim && !dims)) return err("add_input: NULL argument");
        if (dtype <= 0 || dtype >= NNR_DATA_TYPE_COUNT) return err("add_input: bad data_type_t");
        if (!c->ctx.add_input(name, (data_type_t)dtype, std::vector<int>(dims, dims + ndim))) return ctx_err(c);
        return 0;
    });
}

int nnr_ctx_add_output(nnr_ctx_t c, const char* name) {
    return guarded("ctx_add_output", [&]() -> int {
        if (!c || !name) return err("add_output: NULL argument");
        c->ctx.add_output(name);
        return 0;
    });
}

int nnr_ctx_add_node(nnr_ctx_t c, const char* op_type, const char* name, int n_in,
                     const char* const* inputs, int n_out, const char* const* outputs, int n_attr,
                     const char* const* attr_names, const int* kinds, const int* counts, const int* offs,
                     const int64_t* ints, const float* floats, const char* const* strings) {
    return guarded("ctx_add_node", [&]() -> int {
        if (!c || !op_type || !name) return err("add_node: NULL argument");
        std::vector<std::string> ins, outs;
        for (int i = 0; i < n_in; ++i) ins.push_back(inputs[i] ? inputs[i] : "");
        for (int i = 0; i < n_out; ++i) outs.push_back(outputs[i] ? outputs[i] : "");
        std::vector<std::pair<std::string, attr_t>> attrs;
        for (int i = 0; i < n_attr; ++i) {
            attr_t a;
            a.kind = (attr_t::kind_t)kinds[i];
            switch (kinds[i]) {
            case NNR_ATTR_INT: a.i = ints[offs[i]]; break;
            case NNR_ATTR_FLOAT: a.f = floats[offs[i]]; break;
            case NNR_ATTR_STRING: a.s = strings[i] ? strings[i] : ""; break;
            case NNR_ATTR_INTS: a.ints.assign(ints + offs[i], ints + offs[i] + counts[i]); break;
            case NNR_ATTR_FLOATS: a.floats.assign(floats + offs[i], floats + offs[i] + counts[i]); break;
            default: return err("add_node: bad attribute kind");
            }
            attrs.emplace_back(attr_names[i], std::move(a));
        }
        if (!c->ctx.add_node(op_type, name, ins, outs, std::move(attrs))) return ctx_err(c);
        return 0;
    });
}

int nnr_ctx_prepare(nnr_ctx_t c) {
    return guarded("ctx_prepare", [&]() -> int {
        if (!c) return err("ctx is NULL");
        if (!c->ctx.prepare()) return ctx_err(c);
        c->plan.clear();
        for (auto* op : c->ctx.nodes)
            if (!op->skip && !op->folded) c->plan.push_back(op);
        return 0;
    });
}

int nnr_ctx_optimize(nnr_ctx_t c) {
    return guarded("ctx_optimize", [&]() -> int {
        if (!c) return err("ctx is NULL");
        if (!c->ctx.optimize()) return ctx_err(c);
        c->plan.clear();
        for (auto* op : c->ctx.nodes)
            if (!op->skip && !op->folded) c->plan.push_back(op);
        return 0;
    });
}

int nnr_ctx_run(nnr_ctx_t c) {
    return guarded("ctx_run", [&]() -> int {
        if (!c) return err("ctx is NULL");
        if (!c->ctx.run()) return ctx_err(c);
        return 0;
    });
}

// ---- concurrent contexts ---------------------------------------------------
struct nnr_group {
    std::vector<nnr_ctx_t> parts;
    void* fork = nullptr;               // recorded on the caller's stream at run()
    std::vector<void*> done;            // recorded on each part's stream after its run
    ~nnr_group() {
        if (fork) nnrh_event_destroy(fork);
        for (void* e : done)
            if (e) nnrh_event_destroy(e);
    }
};

int nnr_group_create(const nnr_ctx_t* ctxs, int n, nnr_group_t* out) {
    return guarded("group_create", [&]() -> int {
        if (!out) return err("group is NULL");
        *out = nullptr;
        if (!ctxs || n < 1) return err("group_create: no contexts");
        for (int i = 0; i < n; ++i) {
            if (!ctxs[i]) return err("group_create: context " + std::to_string(i) + " is NULL");
            if (!ctxs[i]->ctx.stream)
                return err("group_create: context " + std::to_string(i) + " needs a stream of its own");
            for (int j = 0; j < i; ++j)
                if (ctxs[j] == ctxs[i] || ctxs[j]->ctx.stream == ctxs[i]->ctx.stream)
                    return err("group_create: contexts " + std::to_string(j) + " and " + std::to_string(i) +
                               " share a context or a stream");
        }
        std::unique_ptr<nnr_group> g(new nnr_group());
        g->parts.assign(ctxs, ctxs + n);
        if (nnrh_event_create(&g->fork) != 0) return err(nnrh_last_error());
        g->done.assign((size_t)n, nullptr);
        for (auto& e : g->done)
            if (nnrh_event_create(&e) != 0) return err(nnrh_last_error());
        *out = g.release();
        return 0;
    });
}

int nnr_group_run(nnr_group_t g, void* stream) {
    return guarded("group_run", [&]() -> int {
        if (!g) return err("group is NULL");
        // fork: every part's stream starts after the caller's work so far
        if (nnrh_event_record(g->fork, stream) != 0) return err(nnrh_last_error());
        for (size_t i = 0; i < g->parts.size(); ++i) {
            nnr_ctx_t c = g->parts[i];
            if (nnrh_stream_wait_event(c->ctx.stream, g->fork) != 0) return err(nnrh_last_error());
            if (!c->ctx.run()) return ctx_err(c);
            if (nnrh_event_record(g->done[i], c->ctx.stream) != 0) return err(nnrh_last_error());
        }
        // join: the caller's later work waits for every part
        for (void* e : g->done)
            if (nnrh_stream_wait_event(stream, e) != 0) return err(nnrh_last_error());
        return 0;
    });
}

int nnr_group_destroy(nnr_group_t g) {
    return guarded("group_destroy", [&]() -> int {
        delete g;
        return 0;
    });
}

int nnr_ctx_tensor(nnr_ctx_t c, const char* name, void** data, int* dtype, int* dims, int* ndim,
                   int* format) {
    return guarded("ctx_tensor", [&]() -> int {
        if (!c || !name) return err("tensor: NULL argument");
        tensor_t* t = c->ctx.find(name);
        if (!t) return err(std::string("no tensor named ") + name);
        if (data) *data = t->data;
        if (dtype) *dtype = (int)t->type;
        if (ndim) *ndim = t->ndim();
        if (dims)
            for (int i = 0; i < t->ndim() && i < 8; ++i) dims[i] = t->dims[i];
        if (format) *format = t->format == memory_layout_t::NHWC ? 1 : 0;
        return 0;
    });
}

int nnr_ctx_node_count(nnr_ctx_t c, int* n) {
    return guarded("ctx_node_count", [&]() -> int {
        if (!c || !n) return err("node_count: NULL");
        *n = (int)c->plan.size();
        return 0;
    });
}

int nnr_ctx_node_info(nnr_ctx_t c, int i, const char** op_type, const char** name, const char** variant,
                      int* post_fn, int* n_in, int* n_out) {
    return guarded("ctx_node_info", [&]() -> int {
        if (!c || i < 0 || i >= (int)c->plan.size()) return err("node_info: bad index");
        operator_t* op = c->plan[i];
        if (op_type) *op_type = op->op_type.c_str();
        if (name) *name = op->node_name.c_str();
        if (variant) {
            c->scratch = op->variant();
            *variant = c->scratch.c_str();
        }
        if (post_fn) *post_fn = op->post_fn ? 1 : 0;
        if (n_in) *n_in = (int)op->inputs.size();
        if (n_out) *n_out = (int)op->outputs.size();
        return 0;
    });
}

int nnr_ctx_node_io(nnr_ctx_t c, int i, int is_out, int j, const char** tname) {
    return guarded("ctx_node_io", [&]() -> int {
        if (!c || i < 0 || i >= (int)c->plan.size() || !tname) return err("node_io: bad index");
        auto& v = is_out ? c->plan[i]->outputs : c->plan[i]->inputs;
        if (j < 0 || j >= (int)v.size()) return err("node_io: bad slot");
        *tname = v[j] ? v[j]->name.c_str() : "";
        return 0;
    });
}

int nnr_ctx_node_fused_add(nnr_ctx_t c, int i, int j, const char** name) {
    return guarded("ctx_node_fused_add", [&]() -> int {
        if (!c || i < 0 || i >= (int)c->plan.size() || !name) return err("node_fused_add: bad index");
        operator_t* op = c->plan[i];
        *name = "";
        if (!op->fused_add) return 0;
        if (j == -1) {
            *name = op->fused_add->node_name.c_str();
        } else if (j == -2) {
            *name = op->fused_other ? op->fused_other->name.c_str() : "";
        } else if (j >= 0 && j < (int)op->fused_add->inputs.size()) {
            tensor_t* t = op->fused_add->inputs[j];
            *name = t ? t->name.c_str() : "";
        } else {
            return err("node_fused_add: bad slot");
        }
        return 0;
    });
}

int nnr_ctx_node_fused_chain(nnr_ctx_t c, int i, int k, const char** name) {
    return guarded("ctx_node_fused_chain", [&]() -> int {
        if (!c || i < 0 || i >= (int)c->plan.size() || !name) return err("node_fused_chain: bad index");
        operator_t* op = c->plan[i];
        *name = (k >= 0 && k < (int)op->fused_chain.size()) ? op->fused_chain[k]->node_name.c_str() : "";
        return 0;
    });
}

int nnr_ctx_node_fused_pre(nnr_ctx_t c, int i, int k, const char** name) {
    return guarded("ctx_node_fused_pre", [&]() -> int {
        if (!c || i < 0 || i >= (int)c->plan.size() || !name) return err("node_fused_pre: bad index");
        operator_t* op = c->plan[i];
        *name = (k >= 0 && k < (int)op->fused_pre.size()) ? op->fused_pre[k]->node_name.c_str() : "";
        return 0;
    });
}

int nnr_ctx_fusion_stat(nnr_ctx_t c, const char* key, int* value) {
    return guarded("ctx_fusion_stat", [&]() -> int {
        if (!c || !key || !value) return err("fusion_stat: NULL");
        auto it = c->ctx.fusion_stats.find(key);
        *value = it == c->ctx.fusion_stats.end() ? 0 : it->second;
        return 0;
    });
}

size_t nnr_ctx_device_bytes(nnr_ctx_t c) { return c ? c->ctx.device_bytes : 0; }
size_t nnr_ctx_workspace_bytes(nnr_ctx_t c) { return c ? c->ctx.workspace_bytes : 0; }

int nnr_ctx_enable_profiling(nnr_ctx_t c, int on) {
    return guarded("ctx_enable_profiling", [&]() -> int {
        if (!c) return err("ctx is NULL");
        c->ctx.enable_profiling = on != 0;
        for (auto& p : c->ctx.profile) {
            p.ms = 0;
            p.runs = 0;
        }
        return 0;
    });
}

int nnr_ctx_profile(nnr_ctx_t c, int i, double* ms, int* runs, double* ops, double* bytes) {
    return guarded("ctx_profile", [&]() -> int {
        if (!c || i < 0 || i >= (int)c->ctx.profile.size()) return err("profile: bad index");
        auto& p = c->ctx.profile[i];
        if (ms) *ms = p.ms;
        if (runs) *runs = p.runs;
        if (ops) *ops = p.ops;
        if (bytes) *bytes = p.bytes;
        return 0;
    });
}

int nnr_ctx_time_node(nnr_ctx_t c, int i, int reps, double* ms) {
    return guarded("ctx_time_node", [&]() -> int {
        if (!c || !ms) return err("time_node: NULL argument");
        if (!c->ctx.time_node(i, reps, ms)) return ctx_err(c);
        return 0;
    });
}

}  // extern "C"
