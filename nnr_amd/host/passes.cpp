// passes.cpp -- the graph-optimizer passes that decide numerics and kernel
// dispatch on the int8 path, restated for the HIP backend:
//   fold_constants    src/graph_optimizer/fold_constants.cpp:13-59
//   fuse_qdq_compute  src/graph_optimizer/fuse_qdq_compute.cpp:25-350
//   fuse_qdq          src/graph_optimizer/fuse_qdq.cpp:10-170
//   fuse_post_ops     src/graph_optimizer/fuse_post_ops.cpp:10-73
//   assign_layouts    src/graph_optimizer/assign_layouts.cpp:84-360 (int8
//                     chains: force-accepted NHWC, then propagation)
//   fuse_conv_add     no counterpart (the reference never fuses a binary Add,
//                     fuse_post_ops.cpp:67): a same-shape QLinearAdd whose
//                     input is a QLinearConv's only use runs in that conv's
//                     epilogue, with bit-identical results
//   fuse_attention     the head split / merge and scaled softmax attention of
//                     a transformer layer become one MultiHeadAttention
//                     (the com.microsoft contrib op, MultiHeadAttention.cpp);
//                     the reference's fuse_sdpa.cpp matches a narrower pattern
//   fuse_quant_prefix  no counterpart: QuantizeLinear -> first-layer
//                     QLinearConv and DequantizeLinear -> GlobalAveragePool
//                     run as one kernel each, bit-identical to the two operators
//   fuse_matmul_dq_bias  no counterpart: QLinearMatMul -> DequantizeLinear ->
//                     Add(constant last-axis vector) (-> Gelu) runs as one
//                     kernel with an fp32 output, bit-identical to the
//                     operators it replaces
//   fuse_add_layernorm  no counterpart: a same-shape fp32 Add feeding only a
//                     LayerNormalization is formed inside the normalization
//   fuse_dynq_minmax  no counterpart: the producer of a DynamicQuantizeLinear
//                     input writes its min / max pairs as it stores it
//   fuse_matmul_group no counterpart: fused-dequantize QLinearMatMuls reading
//                     the same input run as one launch
//   fuse_dynq_codes   no counterpart: a fused dequantize chain read only by
//                     a DynamicQuantizeLinear stores its uint8 QLinearMatMul
//                     bytes; the quantizer maps them through a per-column
//                     table of the chain's quantized values (bit-identical)
//   fuse_codes_readers no counterpart: a fused dequantize chain (no Gelu)
//                     read only by a LayerNormalization (with its residual
//                     Add) or by the fused attention stores its bytes, from
//                     which the reader forms the values (bit-identical)
//   fuse_conv_maxpool no counterpart: the uint8 MaxPool reading a first-layer
//                     QLinearConv's output runs in the conv's kernel, which
//                     writes only the pooled tensor (bit-identical)
// The fused operators are created through the registry with the context's
// preferred backend, exactly where the reference calls solve_operator.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <unordered_map>
#include <unordered_set>

#include "nnr.h"

namespace nnr {

namespace {

bool active(const operator_t* op) { return !op->skip && !op->folded; }

int count_consumers(context_t* ctx, tensor_t* t, int skip_idx) {
    int c = 0;
    auto& nodes = ctx->nodes;
    for (int j = 0; j < (int)nodes.size(); ++j) {
        if (j == skip_idx || !active(nodes[j])) continue;
        for (auto* x : nodes[j]->inputs)
            if (x == t) c++;
    }
    return c;
}

tensor_t* input_or_null(operator_t* op, size_t i) {
    return op->inputs.size() > i ? op->inputs[i] : nullptr;
}

// fuse_qdq_compute.cpp:7-23 -- uint8 weights become int8 (w - 128, zp - 128)
void convert_weight_uint8_to_int8(tensor_t* w, tensor_t* w_zp) {
    if (!w || w->type != NNR_DATA_TYPE_UINT8 || !w->has_host()) return;
    for (auto& b : w->host) b = (uint8_t)(int8_t)((int)b - 128);
    w->type = NNR_DATA_TYPE_INT8;
    if (w_zp && w_zp->type == NNR_DATA_TYPE_UINT8 && w_zp->has_host()) {
        for (auto& b : w_zp->host) b = (uint8_t)(int8_t)((int)b - 128);
        w_zp->type = NNR_DATA_TYPE_INT8;
    }
}

}  // namespace

// ---------------------------------------------------------------------------
void fold_constants(context_t* ctx) {
    std::unordered_set<const tensor_t*> constants;
    for (auto& name : ctx->initializer_names) {
        tensor_t* t = ctx->find(name);
        if (t) constants.insert(t);
    }
    for (auto* n : ctx->nodes) {
        if (n->skip) continue;
        bool all_const = !n->inputs.empty();
        for (auto* t : n->inputs)
            if (t && !constants.count(t)) { all_const = false; break; }
        if (!all_const) continue;
        n->folded = true;
        for (auto* t : n->outputs)
            if (t) constants.insert(t);
    }
}

// ---------------------------------------------------------------------------
void fuse_qdq_compute(context_t* ctx) {
    auto& nodes = ctx->nodes;
    const int n = (int)nodes.size();
    std::unordered_map<tensor_t*, int> producer, all_producer;
    auto rebuild = [&]() {
        producer.clear();
        all_producer.clear();
        for (int i = 0; i < n; ++i) {
            for (auto* t : nodes[i]->outputs) all_producer[t] = i;
            if (!active(nodes[i])) continue;
            for (auto* t : nodes[i]->outputs) producer[t] = i;
        }
    };
    rebuild();
    auto dq_of = [&](tensor_t* t, bool any) -> operator_t* {
        auto& m = any ? all_producer : producer;
        auto it = m.find(t);
        if (it == m.end()) return nullptr;
        operator_t* nd = nodes[it->second];
        return nd->op_type == "DequantizeLinear" ? nd : nullptr;
    };
    auto q_consumer = [&](tensor_t* t, int src) -> int {
        for (int j = 0; j < n; ++j) {
            if (j == src || !active(nodes[j])) continue;
            if (nodes[j]->op_type != "QuantizeLinear") continue;
            if (!nodes[j]->inputs.empty() && nodes[j]->inputs[0] == t) return j;
        }
        return -1;
    };

    int fused = 0;
    // Phase 1: DQ -> Conv/MatMul -> Q   =>  QLinearConv / QLinearMatMul
    for (int i = 0; i < n; ++i) {
        operator_t* op = nodes[i];
        if (!active(op)) continue;
        const bool is_conv = op->op_type == "Conv", is_mm = op->op_type == "MatMul";
        if (!is_conv && !is_mm) continue;
        if (op->inputs.size() < 2 || !op->inputs[0] || !op->inputs[1]) continue;
        operator_t* dq_x = dq_of(op->inputs[0], false);
        if (!dq_x || dq_x->inputs.size() < 2) continue;
        operator_t* dq_w = dq_of(op->inputs[1], true);
        if (!dq_w || dq_w->inputs.size() < 2) continue;
        operator_t* dq_b = nullptr;
        if (is_conv && op->inputs.size() >= 3 && op->inputs[2]) dq_b = dq_of(op->inputs[2], true);
        if (op->outputs.empty() || !op->outputs[0]) continue;
        tensor_t* out = op->outputs[0];
        if (count_consumers(ctx, out, i) != 1) continue;
        int qi = q_consumer(out, i);
        if (qi < 0) continue;
        operator_t* q_y = nodes[qi];
        if (q_y->inputs.size() < 2) continue;

        const char* new_type = is_conv ? "QLinearConv" : "QLinearMatMul";
        operator_t* f = solve_operator(new_type, op->opset, ctx->attr_pool, ctx->preferred_backend);
        if (!f) continue;
        f->ctx = ctx;
        f->opset = op->opset;
        f->op_type = new_type;
        f->node_name = op->node_name;
        f->inputs = {dq_x->inputs[0], dq_x->inputs[1], input_or_null(dq_x, 2),
                     dq_w->inputs[0], dq_w->inputs[1], input_or_null(dq_w, 2),
                     q_y->inputs[1], input_or_null(q_y, 2)};
        if (dq_b) f->inputs.push_back(dq_b->inputs[0]);
        if (is_conv) f->attrs = op->attrs;
        f->outputs = {q_y->outputs[0]};
        convert_weight_uint8_to_int8(f->inputs[3], f->inputs[5]);
        f->init();
        nodes[i] = f;
        destroy_op(op);
        if (count_consumers(ctx, dq_x->outputs[0], all_producer[dq_x->outputs[0]]) == 0) dq_x->folded = true;
        dq_w->folded = true;
        if (dq_b) dq_b->folded = true;
        q_y->folded = true;
        fused++;
    }

    // Phase 2: DQ + DQ -> Add [-> Relu] -> Q  =>  QLinearAdd
    rebuild();
    auto implicit_dq = [&](tensor_t* fp32) -> operator_t* {
        int qi = -1;
        for (int j = 0; j < n; ++j) {
            if (nodes[j]->skip || nodes[j]->op_type != "QuantizeLinear") continue;
            if (!nodes[j]->inputs.empty() && nodes[j]->inputs[0] == fp32) { qi = j; break; }
        }
        if (qi < 0) return nullptr;
        tensor_t* qo = nodes[qi]->outputs[0];
        for (int j = 0; j < n; ++j) {
            if (nodes[j]->skip || nodes[j]->op_type != "DequantizeLinear") continue;
            if (!nodes[j]->inputs.empty() && nodes[j]->inputs[0] == qo) return nodes[j];
        }
        return nullptr;
    };
    int add_fused = 0;
    for (int i = 0; i < n; ++i) {
        operator_t* op = nodes[i];
        if (!active(op) || op->op_type != "Add") continue;
        if (op->inputs.size() < 2 || !op->inputs[0] || !op->inputs[1]) continue;
        operator_t* dq_a = dq_of(op->inputs[0], false);
        if (!dq_a) dq_a = implicit_dq(op->inputs[0]);
        operator_t* dq_b = dq_of(op->inputs[1], false);
        if (!dq_b) dq_b = implicit_dq(op->inputs[1]);
        if (!dq_a || dq_a->inputs.size() < 2 || !dq_b || dq_b->inputs.size() < 2) continue;
        if (op->outputs.empty() || !op->outputs[0]) continue;
        tensor_t* add_out = op->outputs[0];
        if (count_consumers(ctx, add_out, i) != 1) continue;
        int relu = -1;
        tensor_t* pre_q = add_out;
        for (int j = 0; j < n; ++j) {
            if (j == i || !active(nodes[j])) continue;
            bool uses = false;
            for (auto* t : nodes[j]->inputs) uses |= (t == add_out);
            if (!uses) continue;
            if (nodes[j]->op_type == "Relu") {
                relu = j;
                pre_q = nodes[j]->outputs[0];
            }
            break;
        }
        if (relu >= 0 && count_consumers(ctx, pre_q, relu) != 1) continue;
        int qi = q_consumer(pre_q, relu >= 0 ? relu : i);
        if (qi < 0) continue;
        operator_t* q_y = nodes[qi];
        if (q_y->inputs.size() < 2) continue;
        operator_t* f = solve_operator("QLinearAdd", op->opset, ctx->attr_pool, ctx->preferred_backend);
        if (!f) continue;
        f->ctx = ctx;
        f->opset = op->opset;
        f->op_type = "QLinearAdd";
        f->node_name = op->node_name;
        f->inputs = {dq_a->inputs[0], dq_a->inputs[1], input_or_null(dq_a, 2),
                     dq_b->inputs[0], dq_b->inputs[1], input_or_null(dq_b, 2),
                     q_y->inputs[1], input_or_null(q_y, 2)};
        f->outputs = {q_y->outputs[0]};
        f->init();
        tensor_t* in0 = op->inputs[0];
        tensor_t* in1 = op->inputs[1];
        nodes[i] = f;
        destroy_op(op);
        if (count_consumers(ctx, dq_a->outputs[0], all_producer[in0]) == 0) dq_a->folded = true;
        if (count_consumers(ctx, dq_b->outputs[0], all_producer[in1]) == 0) dq_b->folded = true;
        if (relu >= 0) nodes[relu]->folded = true;
        q_y->folded = true;
        add_fused++;
    }
    ctx->fusion_stats["qdq_compute"] += fused;
    ctx->fusion_stats["qdq_add"] += add_fused;
    if (fused || add_fused)
        fprintf(stderr, "[nnr] Fused %d QDQ compute + %d QDQ add patterns\n", fused, add_fused);
}

// ---------------------------------------------------------------------------
void fuse_qdq(context_t* ctx) {
    auto& nodes = ctx->nodes;
    const int n = (int)nodes.size();
    static const std::unordered_set<std::string> quant_capable = {
        "MaxPool", "AveragePool", "Concat", "Reshape", "Transpose", "Flatten", "Squeeze",
        "Unsqueeze", "Relu", "Clip", "Pad", "Slice", "Gather", "Split", "Resize"};
    auto scale_zp = [](operator_t* op, float& s, int32_t& zp) -> bool {
        if (op->inputs.size() < 2 || !op->inputs[1]) return false;
        tensor_t* st = op->inputs[1];
        if (st->ndata != 1 || !st->has_host() || st->type != NNR_DATA_TYPE_FLOAT32) return false;
        s = st->scalar_f32();
        zp = 0;
        if (op->inputs.size() >= 3 && op->inputs[2] && op->inputs[2]->ndata > 0)
            zp = op->inputs[2]->scalar_int();
        return true;
    };
    int fused = 0;
    for (int i = 0; i < n; ++i) {
        operator_t* nd = nodes[i];
        if (!active(nd) || nd->op_type != "DequantizeLinear" || nd->outputs.empty()) continue;
        tensor_t* dq_out = nd->outputs[0];
        tensor_t* dq_in = nd->inputs[0];
        if (count_consumers(ctx, dq_out, i) != 1) continue;
        int ci = -1;
        for (int j = 0; j < n && ci < 0; ++j) {
            if (j == i || !active(nodes[j])) continue;
            for (auto* t : nodes[j]->inputs)
                if (t == dq_out) { ci = j; break; }
        }
        if (ci < 0) continue;
        operator_t* c = nodes[ci];
        if (c->op_type == "DequantizeLinear" || c->op_type == "QuantizeLinear") continue;
        if (!quant_capable.count(c->op_type) || !c->resolved) continue;
        if (c->outputs.empty()) continue;
        tensor_t* c_out = c->outputs[0];
        int qi = -1;
        for (int j = 0; j < n && qi < 0; ++j) {
            if (j == ci || !active(nodes[j]) || nodes[j]->op_type != "QuantizeLinear") continue;
            for (auto* t : nodes[j]->inputs)
                if (t == c_out) { qi = j; break; }
        }
        if (qi < 0) continue;
        operator_t* q = nodes[qi];
        if (count_consumers(ctx, c_out, ci) != 1) continue;
        float ds, qs;
        int32_t dz, qz;
        if (!scale_zp(nd, ds, dz) || !scale_zp(q, qs, qz)) continue;
        dq_in->set_quant(ds, dz);
        tensor_t* q_out = q->outputs[0];
        q_out->set_quant(qs, qz);
        for (auto& t : c->inputs)
            if (t == dq_out) t = dq_in;
        for (auto& t : c->outputs)
            if (t == c_out) t = q_out;
        nd->folded = true;
        q->folded = true;
        fused++;
    }
    ctx->fusion_stats["qdq_transparent"] += fused;
    if (fused) fprintf(stderr, "[nnr] Fused %d QDQ patterns\n", fused);
}

// ---------------------------------------------------------------------------
void fuse_post_ops(context_t* ctx) {
    auto& nodes = ctx->nodes;
    const int n = (int)nodes.size();
    int fused = 0;
    for (int i = 0; i + 1 < n; ++i) {
        operator_t* p = nodes[i];
        if (p->skip || p->post_fn) continue;
        const std::string& t = p->op_type;
        if (t != "Conv" && t != "Gemm" && t != "MatMul" && t != "QLinearConv") continue;
        if (p->outputs.empty()) continue;
        tensor_t* eff = p->outputs[0];
        int j = i + 1;
        for (; j < n && (nodes[j]->skip || nodes[j]->folded); ++j) {
            operator_t* sk = nodes[j];
            if (!sk->inputs.empty() && !sk->outputs.empty() && sk->inputs[0] == eff) eff = sk->outputs[0];
        }
        if (j >= n) continue;
        operator_t* c = nodes[j];
        if (!c->fusable_unary || c->inputs.empty()) continue;
        tensor_t* raw = p->outputs[0];
        tensor_t* matched = nullptr;
        for (auto* x : c->inputs)
            if (x == eff || x == raw) { matched = x; break; }
        if (!matched) continue;
        if (count_consumers(ctx, matched, -1) != 1) continue;
        if (c->inputs.size() == 2) continue;   // binary ops are never fused
        // HardSwish's bits depend on an element's position (its 16-wide body
        // multiplies by fl(1/6), the last n % 16 elements divide by 6). Gemm
        // applies a fused unary over its whole output (Gemm.cpp:146-151), as
        // the standalone operator does; MatMul applies it per GEMM output
        // tile of its CPU blocking (gemm_post_t, MatMul.cpp:218-280), whose
        // positions this backend does not have. So MatMul takes only the
        // position-free Relu / Clip, and a HardSwish after it runs on its own.
        if (t == "MatMul" && c->op_type == "HardSwish") continue;
        p->post_fn = true;
        p->fused_op = c;
        c->skip = true;
        // an fp32 producer applies the fused op to its output in place
        // (apply_post); on QLinearConv the fusion only raises qmin
        if (t != "QLinearConv") p->fused_chain.push_back(c);
        // a skipped step forwards its input buffer (src/nnr.cpp:914-918)
        if (!c->outputs.empty()) c->outputs[0]->alias_of = matched;
        fused++;
    }
    ctx->fusion_stats["post_ops"] += fused;
}

// ---------------------------------------------------------------------------
void assign_layouts(context_t* ctx) {
    auto& nodes = ctx->nodes;
    const int n = (int)nodes.size();
    std::unordered_map<tensor_t*, int> consumers;
    std::unordered_map<tensor_t*, int> first_consumer;
    for (int i = 0; i < n; ++i) {
        if (!active(nodes[i])) continue;
        for (auto* t : nodes[i]->inputs) {
            if (!t) continue;
            if (!consumers[t]++) first_consumer[t] = i;
        }
    }
    std::unordered_set<tensor_t*> graph_outs;
    for (auto& s : ctx->graph_outputs) graph_outs.insert(ctx->find(s));
    std::unordered_set<tensor_t*> nhwc;
    std::unordered_map<tensor_t*, int> producer;
    for (int i = 0; i < n; ++i)
        if (active(nodes[i]))
            for (auto* t : nodes[i]->outputs) producer[t] = i;
    auto is_act4d = [&](tensor_t* t) {
        return t && t->ndim() == 4 && !ctx->initializer_names.count(t->name);
    };
    std::vector<bool> visited(n, false);
    // chain formation from each NHWC-capable QLinearConv (:84-297). Chains of
    // QLinearConv are force-accepted (all-int8), so no cost model is needed.
    for (int s = 0; s < n; ++s) {
        operator_t* op = nodes[s];
        if (!active(op) || op->op_type != "QLinearConv" || !(op->layout_mask & LAYOUT_NHWC) || visited[s])
            continue;
        std::vector<int> chain;
        int cur = s;
        while (cur >= 0 && cur < n) {
            operator_t* nd = nodes[cur];
            if (!active(nd)) { cur++; continue; }
            if (!(nd->layout_mask & LAYOUT_NHWC)) break;
            int n4 = 0, in_chain = 0;
            for (auto* t : nd->inputs) {
                if (!is_act4d(t)) continue;
                n4++;
                bool ok = false;
                auto it = producer.find(t);
                if (it != producer.end())
                    for (int e : chain) ok |= (e == it->second);
                if (!ok && nhwc.count(t)) ok = true;
                in_chain += ok;
            }
            if (n4 > 1 && in_chain < n4) break;
            if (nd->op_type == "Conv") break;   // float chains need the cost model
            chain.push_back(cur);
            visited[cur] = true;
            if (nd->outputs.empty()) break;
            tensor_t* out = nd->outputs[0];
            if (graph_outs.count(out) || consumers[out] != 1) break;
            auto fc = first_consumer.find(out);
            if (fc == first_consumer.end() || visited[fc->second]) break;
            cur = fc->second;
        }
        for (int e : chain)
            for (auto* t : nodes[e]->outputs)
                if (t && t->ndim() == 4 &&
                    (t->type == NNR_DATA_TYPE_FLOAT32 || t->type == NNR_DATA_TYPE_UINT8 ||
                     t->type == NNR_DATA_TYPE_INT8)) {
                    t->format = memory_layout_t::NHWC;
                    nhwc.insert(t);
                }
    }
    // propagation through NHWC-capable inter-chain nodes (:283-360)
    auto consumers_safe = [&](tensor_t* t) {
        for (int j = 0; j < n; ++j) {
            operator_t* c = nodes[j];
            if (!active(c)) continue;
            for (auto* x : c->inputs) {
                if (x != t) continue;
                bool out_nhwc = !c->outputs.empty() && nhwc.count(c->outputs[0]);
                bool sup = c->layout_mask == LAYOUT_ALL || (c->layout_mask & LAYOUT_NHWC);
                if (!out_nhwc && !sup) return false;
                break;
            }
        }
        return true;
    };
    bool changed = true;
    while (changed) {
        changed = false;
        for (int i = 0; i < n; ++i) {
            operator_t* nd = nodes[i];
            if (!active(nd)) continue;
            bool all = nd->layout_mask == LAYOUT_ALL;
            if (!all && !(nd->layout_mask & LAYOUT_NHWC)) continue;
            bool has = false;
            for (auto* t : nd->inputs) has |= (t && nhwc.count(t));
            if (!has) continue;
            if (!all) {
                bool ok = true;
                for (auto* t : nd->inputs)
                    if (is_act4d(t) && !nhwc.count(t)) ok = false;
                if (!ok) continue;
            }
            for (auto* t : nd->outputs) {
                if (!t || t->ndim() != 4 || nhwc.count(t)) continue;
                if (!consumers_safe(t)) continue;
                t->format = memory_layout_t::NHWC;
                nhwc.insert(t);
                changed = true;
            }
        }
    }
    ctx->fusion_stats["nhwc_tensors"] = (int)nhwc.size();
}

// ---------------------------------------------------------------------------
// Runs after every operator is built (the conv decides whether its kernel
// can take the add). The residual operand must be produced before the conv
// runs; when both add inputs are conv outputs, the later conv takes the add.
void fuse_conv_add(context_t* ctx) {
    auto& nodes = ctx->nodes;
    const int n = (int)nodes.size();
    std::unordered_map<tensor_t*, int> producer;
    auto rebuild_producer = [&]() {
        producer.clear();
        for (int j = 0; j < n; ++j) {
            if (!active(nodes[j])) continue;
            for (auto* t : nodes[j]->outputs)
                if (t) producer[t] = j;
        }
    };
    rebuild_producer();
    std::unordered_set<tensor_t*> graph_out;
    for (auto& name : ctx->graph_outputs)
        if (tensor_t* t = ctx->find(name)) graph_out.insert(t);
    int fused = 0, moved = 0;
    for (int i = 0; i < n; ++i) {
        operator_t* add = nodes[i];
        if (!active(add) || add->op_type != "QLinearAdd" || add->inputs.size() != 8) continue;
        tensor_t *a = add->inputs[0], *b = add->inputs[3];
        if (!a || !b || a->dims != b->dims || a->format != b->format) continue;
        auto prod = [&](tensor_t* t) {
            auto it = producer.find(t);
            return it == producer.end() ? -1 : it->second;
        };
        int pa = prod(a), pb = prod(b);
        int moved_at = -1, moved_from = -1;
        // both operands from convolutions, the later one strided or spatial
        // and the earlier one a dense 1x1 (a bottleneck's downsample and
        // last conv): the later one moves before the earlier one when its
        // inputs exist by then, so that the dense conv, now later, takes the
        // add (its kernel streams the residual at HBM rate)
        if (pa >= 0 && pb >= 0 && pa != pb) {
            const int lo = std::min(pa, pb), hi = std::max(pa, pb);
            operator_t *early = nodes[lo], *late = nodes[hi];
            bool movable = early->op_type == "QLinearConv" && late->op_type == "QLinearConv" &&
                           early->dense_pointwise() && !late->dense_pointwise() && !early->fused_add &&
                           !late->fused_add;
            for (auto* t : late->inputs)
                if (movable && t && prod(t) >= lo) movable = false;
            for (int j = lo; movable && j < hi; ++j) {
                if (!active(nodes[j])) continue;
                for (auto* t : nodes[j]->inputs)
                    for (auto* o : late->outputs)
                        if (t && t == o) movable = false;
            }
            if (movable) {
                nodes.erase(nodes.begin() + hi);
                nodes.insert(nodes.begin() + lo, late);
                rebuild_producer();
                pa = prod(a);
                pb = prod(b);
                moved_at = lo;
                moved_from = hi;
            }
        }
        // try the later producer first: the other operand then already exists
        int order[2][2] = {{pa, 0}, {pb, 3}};
        if (pb > pa) { std::swap(order[0][0], order[1][0]); std::swap(order[0][1], order[1][1]); }
        for (auto& o : order) {
            const int pi = o[0], side = o[1];
            if (pi < 0) continue;
            operator_t* conv = nodes[pi];
            tensor_t* t = side == 0 ? a : b;
            tensor_t* other = side == 0 ? b : a;
            if (conv->op_type != "QLinearConv" || conv->fused_add || conv->outputs.size() != 1) continue;
            if (prod(other) >= pi) continue;
            if (graph_out.count(t) || count_consumers(ctx, t, -1) != 1) continue;
            if (!conv->fuse_residual_add(add, side)) continue;
            conv->fused_add = add;
            conv->fused_other = other;
            conv->outputs[0] = add->outputs[0];
            add->skip = true;
            producer[add->outputs[0]] = pi;
            ++fused;
            break;
        }
        if (moved_at >= 0) {
            if (add->skip) {
                ++moved;
            } else {
                // the dense conv did not take the add: the original order back
                operator_t* late = nodes[moved_at];
                nodes.erase(nodes.begin() + moved_at);
                nodes.insert(nodes.begin() + moved_from, late);
                rebuild_producer();
            }
        }
    }
    ctx->fusion_stats["conv_add"] = fused;
    ctx->fusion_stats["conv_add_reordered"] = moved;
}

// ---------------------------------------------------------------------------
// QLinearMatMul -> DequantizeLinear (the output's own scale / zero point) ->
// Add(constant vector over the last axis). Runs after the operators are built.
void fuse_matmul_dq_bias(context_t* ctx) {
    auto& nodes = ctx->nodes;
    const int n = (int)nodes.size();
    std::unordered_set<tensor_t*> graph_out;
    for (auto& name : ctx->graph_outputs)
        if (tensor_t* t = ctx->find(name)) graph_out.insert(t);
    auto sole_consumer = [&](tensor_t* t) -> operator_t* {
        operator_t* c = nullptr;
        for (auto* op : nodes) {
            if (!active(op)) continue;
            for (auto* x : op->inputs)
                if (x == t) {
                    if (c && c != op) return nullptr;
                    c = op;
                }
        }
        return c;
    };
    auto same_scalar = [](tensor_t* a, tensor_t* b) {
        if (!a || !b || !a->has_host() || !b->has_host() || a->ndata != 1 || b->ndata != 1) return false;
        return a->type == b->type && a->host == b->host;
    };
    int fused = 0, gelu = 0;
    for (int i = 0; i < n; ++i) {
        operator_t* mm = nodes[i];
        if (!active(mm) || mm->op_type != "QLinearMatMul" || mm->outputs.size() != 1) continue;
        tensor_t* q = mm->outputs[0];
        if (graph_out.count(q)) continue;
        operator_t* dq = sole_consumer(q);
        if (!dq || dq->op_type != "DequantizeLinear" || dq->inputs.size() < 2 || dq->inputs[0] != q) continue;
        if (!same_scalar(dq->inputs[1], mm->inputs[6])) continue;
        tensor_t* dz = dq->inputs.size() > 2 ? dq->inputs[2] : nullptr;
        if (!same_scalar(dz, mm->inputs[7])) continue;
        tensor_t* f = dq->outputs[0];
        if (graph_out.count(f)) continue;
        operator_t* add = sole_consumer(f);
        if (!add || add->op_type != "Add" || add->inputs.size() != 2) continue;
        tensor_t* bias = add->inputs[0] == f ? add->inputs[1] : add->inputs[0];
        if (!bias || !bias->has_host() || bias->type != NNR_DATA_TYPE_FLOAT32) continue;
        if (!mm->fuse_dq_bias(dq, add)) continue;
        mm->fused_chain = {dq, add};
        mm->outputs[0] = add->outputs[0];
        dq->skip = true;
        add->skip = true;
        ++fused;
        // then a Gelu of the biased value
        tensor_t* fb = add->outputs[0];
        if (graph_out.count(fb)) continue;
        operator_t* ge = sole_consumer(fb);
        if (!ge || ge->op_type != "Gelu" || ge->inputs.size() != 1 || ge->outputs.size() != 1) continue;
        if (!mm->fuse_gelu(ge)) continue;
        mm->fused_chain.push_back(ge);
        mm->outputs[0] = ge->outputs[0];
        ge->skip = true;
        ++gelu;
    }
    ctx->fusion_stats["matmul_dq_bias"] = fused;
    ctx->fusion_stats["matmul_gelu"] = gelu;
}

// ---------------------------------------------------------------------------
// MatMulInteger (constant B) -> Cast(to float) -> Mul(., S) [-> Add(bias)]
// [-> Gelu] with S = Mul(a_scale, w_scale) of the activation's scalar scale
// and a constant per-column weight scale: the per-channel form of dynamic
// quantization. The GEMM forms fl(fl(float(acc) * fl(a_scale * w_scale[n]))
// + bias[n]) itself, so the chain, and the scale product when nothing else
// reads it, are skipped; the chain is recorded in the order its values are
// formed (Cast, the scale product, the Mul, the Add, the Gelu).
void fuse_matmul_integer_scale(context_t* ctx) {
    auto& nodes = ctx->nodes;
    std::unordered_set<tensor_t*> graph_out;
    for (auto& name : ctx->graph_outputs)
        if (tensor_t* t = ctx->find(name)) graph_out.insert(t);
    std::unordered_map<tensor_t*, operator_t*> producer;
    std::unordered_map<tensor_t*, int> uses;
    for (auto* op : nodes) {
        if (!active(op)) continue;
        for (auto* t : op->outputs)
            if (t) producer[t] = op;
        for (auto* t : op->inputs)
            if (t) uses[t]++;
    }
    auto sole_consumer = [&](tensor_t* t) -> operator_t* {
        if (!t || graph_out.count(t) || uses[t] != 1) return nullptr;
        for (auto* op : nodes)
            if (active(op))
                for (auto* x : op->inputs)
                    if (x == t) return op;
        return nullptr;
    };
    auto is_vector = [](tensor_t* t, int n) {
        if (!t || !t->has_host() || t->type != NNR_DATA_TYPE_FLOAT32 || t->ndata != (size_t)n) return false;
        for (int i = 0; i + 1 < t->ndim(); ++i)
            if (t->dims[i] != 1) return false;
        return true;
    };
    int fused = 0, gelu = 0;
    for (auto* mm : nodes) {
        if (!active(mm) || mm->op_type != "MatMulInteger" || mm->outputs.size() != 1) continue;
        tensor_t* acc = mm->outputs[0];
        const int n = acc->ndim() ? acc->dims.back() : 0;
        operator_t* cast = sole_consumer(acc);
        if (!cast || cast->op_type != "Cast" || cast->attribute("to", 0) != 1) continue;
        operator_t* mul = sole_consumer(cast->outputs[0]);
        if (!mul || mul->op_type != "Mul" || mul->inputs.size() != 2) continue;
        tensor_t* sp = mul->inputs[0] == cast->outputs[0] ? mul->inputs[1] : mul->inputs[0];
        auto pit = producer.find(sp);
        if (pit == producer.end()) continue;
        operator_t* smul = pit->second;   // the scale product Mul(a_scale, w_scale)
        if (smul->op_type != "Mul" || smul->inputs.size() != 2 || graph_out.count(sp)) continue;
        tensor_t *a_s = smul->inputs[0], *w_s = smul->inputs[1];
        if (is_vector(a_s, n)) std::swap(a_s, w_s);
        if (!is_vector(w_s, n) || !a_s || a_s->ndata != 1 || a_s->type != NNR_DATA_TYPE_FLOAT32) continue;
        tensor_t* y = mul->outputs[0];
        operator_t* add = sole_consumer(y);
        tensor_t* bias = nullptr;
        if (add && add->op_type == "Add" && add->inputs.size() == 2) {
            bias = add->inputs[0] == y ? add->inputs[1] : add->inputs[0];
            if (!is_vector(bias, n) || add->outputs[0]->dims != y->dims) {
                add = nullptr;
                bias = nullptr;
            }
        } else {
            add = nullptr;
        }
        if (y->dims != acc->dims) continue;
        if (!mm->fuse_int_scale(a_s, w_s, bias)) continue;
        mm->fused_chain = {cast, smul, mul};
        cast->skip = true;
        mul->skip = true;
        if (uses[sp] == 1) smul->skip = true;   // else it still runs for its other readers
        mm->outputs[0] = y;
        if (add) {
            mm->fused_chain.push_back(add);
            mm->outputs[0] = add->outputs[0];
            add->skip = true;
        }
        ++fused;
        operator_t* ge = sole_consumer(mm->outputs[0]);
        if (!ge || ge->op_type != "Gelu" || ge->inputs.size() != 1 || ge->outputs.size() != 1) continue;
        if (!mm->fuse_gelu(ge)) continue;
        mm->fused_chain.push_back(ge);
        mm->outputs[0] = ge->outputs[0];
        ge->skip = true;
        ++gelu;
    }
    ctx->fusion_stats["matmul_integer_scale"] = fused;
    ctx->fusion_stats["matmul_integer_gelu"] = gelu;
}

// ---------------------------------------------------------------------------
// QuantizeLinear / DequantizeLinear whose only consumer is an operator that
// can read their input directly (the first-layer conv's layout kernel, the
// global average pool): the consumer does the (de)quantization itself.
void fuse_quant_prefix(context_t* ctx) {
    auto& nodes = ctx->nodes;
    std::unordered_set<tensor_t*> graph_out;
    for (auto& name : ctx->graph_outputs)
        if (tensor_t* t = ctx->find(name)) graph_out.insert(t);
    std::unordered_map<tensor_t*, operator_t*> producer;
    std::unordered_map<tensor_t*, int> uses;
    for (auto* op : nodes) {
        if (!active(op)) continue;
        for (auto* t : op->outputs)
            if (t) producer[t] = op;
        for (auto* t : op->inputs)
            if (t) uses[t]++;
    }
    int nq = 0, ndq = 0;
    for (auto* op : nodes) {
        if (!active(op) || op->inputs.empty() || !op->inputs[0]) continue;
        const bool conv = op->op_type == "QLinearConv", gap = op->op_type == "GlobalAveragePool";
        if (!conv && !gap) continue;
        tensor_t* x = op->inputs[0];
        auto it = producer.find(x);
        if (it == producer.end() || graph_out.count(x) || uses[x] != 1) continue;
        operator_t* p = it->second;
        bool done = false;
        if (conv && p->op_type == "QuantizeLinear") done = op->fuse_quantize_input(p);
        if (gap && p->op_type == "DequantizeLinear") done = op->fuse_dequantize_input(p);
        if (!done) continue;
        op->fused_pre = {p};
        op->inputs[0] = p->inputs[0];
        p->skip = true;
        (conv ? nq : ndq)++;
    }
    ctx->fusion_stats["quantize_first_conv"] = nq;
    ctx->fusion_stats["dequantize_gap"] = ndq;
}

// ---------------------------------------------------------------------------
// QLinearMatMuls with a fused dequantize + bias that read the same input with
// the same quantization (a transformer layer's Q, K and V projections): up
// to 4 run as one launch, issued by the first in graph order. The others stay
// in the plan (their outputs and chains unchanged) and do nothing at exec.
void fuse_matmul_group(context_t* ctx) {
    int groups = 0;
    std::unordered_set<operator_t*> taken;
    auto& nodes = ctx->nodes;
    for (size_t i = 0; i < nodes.size(); ++i) {
        operator_t* lead = nodes[i];
        if (!active(lead) || !lead->groupable() || taken.count(lead)) continue;
        std::vector<operator_t*> members;
        for (size_t j = i + 1; j < nodes.size() && members.size() < 3; ++j) {
            operator_t* op = nodes[j];
            if (!active(op) || op->op_type != lead->op_type || !op->groupable() || taken.count(op)) continue;
            if (!lead->same_group_input(op)) continue;
            members.push_back(op);
        }
        if (members.empty() || !lead->fuse_group(members)) continue;
        lead->group_leader = lead;
        lead->group_members = members;
        taken.insert(lead);
        for (auto* op : members) {
            op->group_leader = lead;
            taken.insert(op);
        }
        ++groups;
    }
    ctx->fusion_stats["matmul_group"] = groups;
}

// ---------------------------------------------------------------------------
// Add(a, b) of two same-shape fp32 tensors whose only consumer is a
// LayerNormalization (BERT's residual connections): the normalization reads
// a and b and forms fl(a + b) itself, so the sum is never stored.
// ---------------------------------------------------------------------------
// Runs after every operator is built: a QLinearConv whose output feeds only a
// MaxPool (and is not a graph output) takes the pool into its kernel when it
// can; the MaxPool is skipped and its output becomes the conv's.
void fuse_conv_maxpool(context_t* ctx) {
    std::unordered_set<tensor_t*> graph_out;
    for (auto& name : ctx->graph_outputs)
        if (tensor_t* t = ctx->find(name)) graph_out.insert(t);
    int fused = 0;
    for (auto* conv : ctx->nodes) {
        if (!active(conv) || conv->op_type != "QLinearConv" || conv->fused_add || !conv->fused_chain.empty() ||
            conv->outputs.size() != 1)
            continue;
        tensor_t* t = conv->outputs[0];
        if (!t || graph_out.count(t) || count_consumers(ctx, t, -1) != 1) continue;
        operator_t* pool = nullptr;
        for (auto* op : ctx->nodes)
            if (active(op) && op != conv && op->op_type == "MaxPool" && !op->inputs.empty() && op->inputs[0] == t)
                pool = op;
        if (!pool || pool->outputs.size() != 1) continue;
        int k[2], st[2], pads[4];
        if (!pool->pool_params(k, st, pads) || !conv->fuse_maxpool(pool, k, st, pads)) continue;
        conv->fused_chain.push_back(pool);
        conv->outputs[0] = pool->outputs[0];
        pool->skip = true;
        ++fused;
    }
    ctx->fusion_stats["conv_maxpool"] = fused;
}

void fuse_add_layernorm(context_t* ctx) {
    std::unordered_set<tensor_t*> graph_out;
    for (auto& name : ctx->graph_outputs)
        if (tensor_t* t = ctx->find(name)) graph_out.insert(t);
    std::unordered_map<tensor_t*, operator_t*> producer;
    std::unordered_map<tensor_t*, int> uses;
    for (auto* op : ctx->nodes) {
        if (!active(op)) continue;
        for (auto* t : op->outputs)
            if (t) producer[t] = op;
        for (auto* t : op->inputs)
            if (t) uses[t]++;
    }
    int fused = 0;
    for (auto* op : ctx->nodes) {
        if (!active(op) || op->op_type != "LayerNormalization" || !op->fused_pre.empty()) continue;
        tensor_t* x = op->inputs[0];
        auto it = producer.find(x);
        if (it == producer.end() || graph_out.count(x) || uses[x] != 1) continue;
        operator_t* add = it->second;
        if (add->op_type != "Add" || add->inputs.size() != 2 || add->outputs.size() != 1) continue;
        tensor_t *a = add->inputs[0], *b = add->inputs[1];
        if (!a || !b || a->type != NNR_DATA_TYPE_FLOAT32 || b->type != NNR_DATA_TYPE_FLOAT32) continue;
        if (a->dims != x->dims || b->dims != x->dims) continue;
        if (!op->fuse_residual_input(add)) continue;
        op->fused_pre = {add};
        op->inputs[0] = a;
        op->fused_other = b;
        add->skip = true;
        ++fused;
    }
    ctx->fusion_stats["add_layernorm"] = fused;
}

// ---------------------------------------------------------------------------
// DynamicQuantizeLinear whose input's producer can write the input's
// (min, max) pairs as it stores it: the producer gets a buffer for them and
// the quantizer skips its own min / max pass. The producer still writes the
// whole tensor; any other consumer reads it as before.
void fuse_dynq_minmax(context_t* ctx) {
    std::unordered_map<tensor_t*, operator_t*> producer;
    for (auto* op : ctx->nodes) {
        if (!active(op)) continue;
        for (auto* t : op->outputs)
            if (t) producer[t] = op;
    }
    int fused = 0;
    for (auto* op : ctx->nodes) {
        if (!active(op) || op->op_type != "DynamicQuantizeLinear" || op->minmax_src) continue;
        auto it = producer.find(op->inputs[0]);
        if (it == producer.end()) continue;
        operator_t* p = it->second;
        if (p->outputs.empty() || p->outputs[0] != op->inputs[0]) continue;
        if (!p->minmax_parts) {
            const int pairs = p->minmax_pairs();
            if (pairs <= 0) continue;
            float* buf = (float*)ctx->device_alloc(sizeof(float) * 2 * (size_t)pairs);
            if (!buf) continue;
            if (!p->set_minmax_out(buf, pairs)) continue;
            p->minmax_parts = buf;
            p->minmax_count = pairs;
        }
        op->minmax_src = p;
        ++fused;
    }
    ctx->fusion_stats["dynq_minmax"] = fused;
}

// ---------------------------------------------------------------------------
// DynamicQuantizeLinear reading min / max pairs from a producer whose output
// it alone reads (no other operator, no fused chain, not a graph output): a
// producer that can (a fused QLinearMatMul -> DequantizeLinear -> Add [->
// Gelu], not grouped) stores the uint8 QLinearMatMul bytes instead of the
// fp32 chain values, the tensor becomes uint8 (a quarter of the bytes), and
// the quantizer rebuilds each value's byte from the bytes through a table per
// column. Runs after fuse_dynq_minmax and fuse_matmul_group.
void fuse_dynq_codes(context_t* ctx) {
    std::unordered_set<tensor_t*> graph_out;
    for (auto& name : ctx->graph_outputs)
        if (tensor_t* t = ctx->find(name)) graph_out.insert(t);
    std::unordered_map<tensor_t*, int> uses;
    for (auto* op : ctx->nodes) {
        if (op->folded) continue;
        for (auto* t : op->inputs)
            if (t) uses[t]++;
        if (op->fused_other) uses[op->fused_other]++;
    }
    int fused = 0;
    for (auto* op : ctx->nodes) {
        if (!active(op) || op->op_type != "DynamicQuantizeLinear" || !op->minmax_src || op->codes_src) continue;
        tensor_t* t = op->inputs[0];
        if (!t || uses[t] != 1 || graph_out.count(t) || t->type != NNR_DATA_TYPE_FLOAT32) continue;
        operator_t* p = op->minmax_src;
        if (p->group_leader || !p->set_codes_out(true)) continue;
        const std::vector<int> dims = t->dims;
        t->reshape(dims, NNR_DATA_TYPE_UINT8);
        op->codes_src = p;
        ++fused;
    }
    ctx->fusion_stats["dynq_codes"] = fused;
}

// ---------------------------------------------------------------------------
// fp32 results of fused QLinearMatMul -> DequantizeLinear -> Add(bias)
// chains (no Gelu) whose only reader at run time can form each value from the
// chain's uint8 QLinearMatMul byte with the GEMM epilogue's two operations:
// a LayerNormalization (either operand of its residual Add), or the fused
// MultiHeadAttention (q, k and v together, from ungrouped chains or from one
// grouped launch of exactly those three). The chains store their bytes, the
// tensors become uint8 (a quarter of the bytes), the readers record the
// chains' parameters. Runs after fuse_dynq_codes.
void fuse_codes_readers(context_t* ctx) {
    std::unordered_set<tensor_t*> graph_out;
    for (auto& name : ctx->graph_outputs)
        if (tensor_t* t = ctx->find(name)) graph_out.insert(t);
    // readers at run time: the active operators' inputs and fused operands
    std::unordered_map<tensor_t*, int> uses;
    std::unordered_map<tensor_t*, operator_t*> producer;
    for (auto* op : ctx->nodes) {
        if (!active(op)) continue;
        for (auto* t : op->inputs)
            if (t) uses[t]++;
        if (op->fused_other) uses[op->fused_other]++;
        if (!op->outputs.empty() && op->outputs[0]) producer[op->outputs[0]] = op;
    }
    // the chain producing t, when t can be stored as its bytes for one reader
    auto chain_of = [&](tensor_t* t) -> operator_t* {
        if (!t || t->type != NNR_DATA_TYPE_FLOAT32 || graph_out.count(t) || uses[t] != 1) return nullptr;
        auto it = producer.find(t);
        if (it == producer.end()) return nullptr;
        operator_t* p = it->second;
        int zp = 0;
        float sc = 0.0f;
        const float* b = nullptr;
        if (p->op_type != "QLinearMatMul" || p->fused_chain.size() != 2 || !p->codes_params(&zp, &sc, &b))
            return nullptr;
        return p;
    };
    auto to_bytes = [](tensor_t* t) {
        const std::vector<int> dims = t->dims;
        t->reshape(dims, NNR_DATA_TYPE_UINT8);
    };
    int ln = 0, mha = 0;
    for (auto* op : ctx->nodes) {
        if (!active(op)) continue;
        if (op->op_type == "LayerNormalization") {
            tensor_t* cand[2] = {op->inputs[0], op->fused_other};
            for (int w = 0; w < 2; ++w) {
                operator_t* p = chain_of(cand[w]);
                if (!p || p->group_leader || !op->set_codes_input(w, p)) continue;
                if (!p->set_codes_out(true)) {
                    op->set_codes_input(w, nullptr);
                    continue;
                }
                to_bytes(cand[w]);
                ++ln;
                break;
            }
        } else if (op->op_type == "MultiHeadAttention" && op->inputs.size() >= 3) {
            operator_t* ps[3];
            bool all = op->inputs[0] != op->inputs[1] && op->inputs[0] != op->inputs[2] &&
                       op->inputs[1] != op->inputs[2];
            for (int i = 0; i < 3; ++i) {
                ps[i] = chain_of(op->inputs[i]);
                all = all && ps[i];
            }
            if (!all) continue;
            operator_t* lead = ps[0]->group_leader;
            if (lead) {
                // one launch writes exactly these three
                std::unordered_set<operator_t*> grp(lead->group_members.begin(), lead->group_members.end());
                grp.insert(lead);
                bool same = grp.size() == 3;
                for (int i = 0; i < 3; ++i) same = same && ps[i]->group_leader == lead && grp.count(ps[i]);
                if (!same) continue;
            } else if (ps[1]->group_leader || ps[2]->group_leader) {
                continue;
            }
            int rec = 0;
            while (rec < 3 && op->set_codes_input(rec, ps[rec])) ++rec;
            bool good = rec == 3;
            // the launch that writes the bytes first: the group's leader
            std::vector<operator_t*> order;
            if (lead) order.push_back(lead);
            for (int i = 0; i < 3; ++i)
                if (ps[i] != lead) order.push_back(ps[i]);
            size_t set = 0;
            while (good && set < order.size() && order[set]->set_codes_out(true)) ++set;
            good = good && set == order.size();
            if (!good) {
                for (size_t i = 0; i < set; ++i) order[i]->set_codes_out(false);
                for (int i = 0; i < rec; ++i) op->set_codes_input(i, nullptr);
                continue;
            }
            for (int i = 0; i < 3; ++i) to_bytes(op->inputs[i]);
            ++mha;
        }
    }
    ctx->fusion_stats["codes_layernorm"] = ln;
    ctx->fusion_stats["codes_attention"] = mha;
}

// ---------------------------------------------------------------------------
// Reshape([B,S,nh,hd]) -> Transpose(0,2,1,3) of q and v, Transpose(0,2,3,1) of
// k, MatMul(q, k^T) -> Mul(scalar) -> Softmax(last axis) -> MatMul(., v) ->
// Transpose(0,2,1,3) -> Reshape([B,S,nh*hd])  ==>  MultiHeadAttention(q, k, v)
// with num_heads = nh and scale = the Mul's constant. Every intermediate has
// one consumer and is not a graph output. Runs before shape inference: the
// pattern is read from constant shapes and attributes only.
void fuse_attention(context_t* ctx) {
    auto& nodes = ctx->nodes;
    const int n = (int)nodes.size();
    std::unordered_set<tensor_t*> graph_out;
    for (auto& name : ctx->graph_outputs)
        if (tensor_t* t = ctx->find(name)) graph_out.insert(t);
    std::unordered_map<tensor_t*, int> producer, uses;
    for (int i = 0; i < n; ++i) {
        if (!active(nodes[i])) continue;
        for (auto* t : nodes[i]->outputs)
            if (t) producer[t] = i;
        for (auto* t : nodes[i]->inputs)
            if (t) uses[t]++;
    }
    auto only_use = [&](tensor_t* t) { return t && uses[t] == 1 && !graph_out.count(t); };
    auto prod = [&](tensor_t* t, const char* type) -> operator_t* {
        auto it = producer.find(t);
        if (it == producer.end() || nodes[it->second]->op_type != type) return nullptr;
        return nodes[it->second];
    };
    auto perm_is = [](operator_t* op, std::vector<int64_t> p) { return op->attribute_ints("perm") == p; };
    auto shape_of = [](operator_t* r) -> std::vector<int64_t> {
        tensor_t* s = r->inputs.size() > 1 ? r->inputs[1] : nullptr;
        if (!s || !s->has_host() || s->type != NNR_DATA_TYPE_INT64) return {};
        return std::vector<int64_t>(s->h<int64_t>(), s->h<int64_t>() + s->ndata);
    };
    // Reshape(x, [B,S,nh,hd]) -> Transpose(perm) feeding `t`: returns x
    auto head_split = [&](tensor_t* t, std::vector<int64_t> perm, std::vector<int64_t>& shape,
                          std::vector<operator_t*>& eaten) -> tensor_t* {
        operator_t* tr = prod(t, "Transpose");
        if (!tr || !only_use(t) || !perm_is(tr, perm)) return nullptr;
        operator_t* rs = prod(tr->inputs[0], "Reshape");
        if (!rs || !only_use(tr->inputs[0])) return nullptr;
        std::vector<int64_t> sh = shape_of(rs);
        if (sh.size() != 4) return nullptr;
        for (auto d : sh)
            if (d <= 0) return nullptr;
        if (!shape.empty() && sh != shape) return nullptr;
        shape = sh;
        eaten.push_back(rs);
        eaten.push_back(tr);
        return rs->inputs[0];
    };
    int fused = 0;
    for (int i = 0; i < n; ++i) {
        operator_t* sm = nodes[i];
        if (!active(sm) || sm->op_type != "Softmax" || sm->inputs.empty() || sm->outputs.empty()) continue;
        if (sm->attribute("axis", -1) != -1) continue;
        std::vector<operator_t*> eaten;
        // Mul(scores, c) -> Softmax
        operator_t* mul = prod(sm->inputs[0], "Mul");
        if (!mul || !only_use(sm->inputs[0]) || mul->inputs.size() != 2) continue;
        tensor_t *a = mul->inputs[0], *b = mul->inputs[1];
        tensor_t* c = (b && b->has_host()) ? b : ((a && a->has_host()) ? a : nullptr);
        tensor_t* scores = c == b ? a : b;
        if (!c || c->ndata != 1 || c->type != NNR_DATA_TYPE_FLOAT32 || !only_use(scores)) continue;
        operator_t* mm1 = prod(scores, "MatMul");
        if (!mm1 || mm1->inputs.size() != 2) continue;
        // Softmax -> MatMul(p, v4) -> Transpose(0,2,1,3) -> Reshape([B,S,H])
        tensor_t* p = sm->outputs[0];
        if (!only_use(p)) continue;
        operator_t* mm2 = nullptr;
        for (auto* op : nodes)
            if (active(op) && op->op_type == "MatMul" && op->inputs.size() == 2 && op->inputs[0] == p) mm2 = op;
        if (!mm2 || !only_use(mm2->outputs[0])) continue;
        operator_t* tc = nullptr;
        for (auto* op : nodes)
            if (active(op) && op->op_type == "Transpose" && !op->inputs.empty() && op->inputs[0] == mm2->outputs[0])
                tc = op;
        if (!tc || !perm_is(tc, {0, 2, 1, 3}) || !only_use(tc->outputs[0])) continue;
        int rc_i = -1;
        for (int j = 0; j < n; ++j)
            if (active(nodes[j]) && nodes[j]->op_type == "Reshape" && !nodes[j]->inputs.empty() &&
                nodes[j]->inputs[0] == tc->outputs[0])
                rc_i = j;
        if (rc_i < 0) continue;
        operator_t* rc = nodes[rc_i];
        std::vector<int64_t> shape;
        tensor_t* q = head_split(mm1->inputs[0], {0, 2, 1, 3}, shape, eaten);
        tensor_t* k = q ? head_split(mm1->inputs[1], {0, 2, 3, 1}, shape, eaten) : nullptr;
        tensor_t* v = k ? head_split(mm2->inputs[1], {0, 2, 1, 3}, shape, eaten) : nullptr;
        if (!v) continue;
        std::vector<int64_t> merged = shape_of(rc);
        if (merged != std::vector<int64_t>{shape[0], shape[1], shape[2] * shape[3]}) continue;
        operator_t* f = solve_operator("MultiHeadAttention", sm->opset, ctx->attr_pool, ctx->preferred_backend);
        if (!f) continue;
        f->ctx = ctx;
        f->opset = sm->opset;
        f->op_type = "MultiHeadAttention";
        f->node_name = sm->node_name;
        f->inputs = {q, k, v};
        f->outputs = {rc->outputs[0]};
        attr_t heads, scale;
        heads.kind = attr_t::kind_t::INT;
        heads.i = shape[2];
        scale.kind = attr_t::kind_t::FLOAT;
        scale.f = c->scalar_f32();
        f->attrs = {{"num_heads", heads}, {"scale", scale}};
        if (!f->init()) {
            destroy_op(f);
            continue;
        }
        for (auto* op : eaten) op->skip = true;
        mm1->skip = mul->skip = sm->skip = mm2->skip = tc->skip = true;
        nodes[rc_i] = f;
        destroy_op(rc);
        ++fused;
    }
    ctx->fusion_stats["attention"] = fused;
}

}  // namespace nnr

namespace nnr {

namespace {

// a per-tensor fp32 scale held on the host
bool host_scale(const tensor_t* t, float& v) {
    if (!t || t->ndata != 1 || t->type != NNR_DATA_TYPE_FLOAT32 || !t->has_host()) return false;
    v = t->scalar_f32();
    return true;
}
// a uint8 / int8 zero point (absent: 0); fold_bn_qdq.cpp:91-95
int host_zp(const operator_t* op, size_t i) {
    const tensor_t* z = op->inputs.size() > i ? op->inputs[i] : nullptr;
    if (!z || z->ndata == 0 || !z->has_host()) return 0;
    if (z->type == NNR_DATA_TYPE_UINT8) return *z->h<uint8_t>();
    if (z->type == NNR_DATA_TYPE_INT8) return *z->h<int8_t>();
    return 0;
}
// the only active consumer of t, if it is of op_type and reads t as input 0
operator_t* sole_consumer(context_t* ctx, tensor_t* t, int skip_idx, const char* op_type) {
    if (count_consumers(ctx, t, skip_idx) != 1) return nullptr;
    for (auto* op : ctx->nodes)
        if (active(op) && op->op_type == op_type && !op->inputs.empty() && op->inputs[0] == t) return op;
    return nullptr;
}
// operators of this backend whose outputs are fp32
bool fp32_source(context_t* ctx, tensor_t* t) {
    if (t->type == NNR_DATA_TYPE_FLOAT32) return true;
    static const char* const f32_ops[] = {"DequantizeLinear", "Add", "Sub", "Mul", "Div", "Relu", "Clip", "Gelu",
                                          "Softmax", "LayerNormalization", "MatMul", "Gemm", "GlobalAveragePool",
                                          "Transpose", "BatchNormalization"};
    for (auto* op : ctx->nodes) {
        if (!active(op) || op->outputs.empty() || op->outputs[0] != t) continue;
        for (const char* s : f32_ops)
            if (op->op_type == s) return true;
    }
    return false;
}

}  // namespace

// fold_bn_qdq (src/graph_optimizer/fold_bn_qdq.cpp:23-259): DQ -> BN -> Q
// (each link the only consumer) becomes a BatchNormalization reading the
// DQ's uint8 input and writing the Q's uint8 output, its scale / bias
// replaced by the combined per-channel
//   A = dq_s * gamma / q_s,  B = (beta - dq_zp * dq_s * gamma) / q_s + q_zp
// with gamma = scale / sqrtf(var + eps), beta = bias - gamma * mean (float,
// this expression order); then BN -> Q with fp32 input becomes
//   A = gamma / q_s,  B = beta / q_s + q_zp.
// Scales must be per tensor and BN's parameters fp32 initializers. The
// combined A / B go to new initializers (the reference overwrites BN's own
// scale / bias, which another node may share). The folded DQ and Q are kept
// as fused_pre / fused_chain for the plan's readers.
void fold_bn_qdq(context_t* ctx) {
    auto& nodes = ctx->nodes;
    const int n = (int)nodes.size();
    int folded = 0, folded_bnq = 0;
    auto bn_params = [&](operator_t* bn, std::vector<const float*>& p) {
        if (bn->inputs.size() < 5 || bn->outputs.empty() || !bn->fold_affine_u8_possible()) return false;
        const tensor_t* s0 = bn->inputs[1];
        if (!s0) return false;
        p.clear();
        for (int k = 1; k <= 4; ++k) {
            const tensor_t* t = bn->inputs[k];
            if (!t || t->ndata == 0 || t->ndata != s0->ndata || t->type != NNR_DATA_TYPE_FLOAT32 ||
                !t->has_host() || !ctx->initializer_names.count(t->name))
                return false;
            p.push_back(t->h<float>());
        }
        return true;
    };
    auto apply = [&](operator_t* bn, operator_t* dq, operator_t* q, const std::vector<const float*>& p, float dq_s,
                     int dq_zp, float q_s, int q_zp) {
        const int C = (int)bn->inputs[1]->ndata;
        const float eps = bn->attribute_f("epsilon", 1e-5f);
        std::vector<float> A(C), B(C);
        for (int c = 0; c < C; ++c) {
            const float gamma = p[0][c] / sqrtf(p[3][c] + eps);
            const float beta = p[1][c] - gamma * p[2][c];
            if (dq) {
                A[c] = dq_s * gamma / q_s;
                B[c] = (beta - (float)dq_zp * dq_s * gamma) / q_s + (float)q_zp;
            } else {
                A[c] = gamma / q_s;
                B[c] = beta / q_s + (float)q_zp;
            }
        }
        const std::string a_name = bn->node_name + "_fold_A", b_name = bn->node_name + "_fold_B";
        ctx->add_initializer(a_name, NNR_DATA_TYPE_FLOAT32, {C}, A.data());
        ctx->add_initializer(b_name, NNR_DATA_TYPE_FLOAT32, {C}, B.data());
        bn->inputs[1] = ctx->find(a_name);
        bn->inputs[2] = ctx->find(b_name);
        if (dq) {
            bn->inputs[0] = dq->inputs[0];
            bn->fused_pre = {dq};
            dq->skip = true;
        }
        bn->outputs[0] = q->outputs[0];
        bn->fused_chain = {q};
        q->skip = true;
        bn->fold_affine_u8();
    };
    std::vector<const float*> p;
    for (int i = 0; i < n; ++i) {
        operator_t* dq = nodes[i];
        if (!active(dq) || dq->op_type != "DequantizeLinear" || dq->outputs.empty() || dq->inputs.size() < 2) continue;
        operator_t* bn = sole_consumer(ctx, dq->outputs[0], i, "BatchNormalization");
        if (!bn || !bn_params(bn, p)) continue;
        int bn_idx = -1;
        for (int j = 0; j < n; ++j)
            if (nodes[j] == bn) bn_idx = j;
        operator_t* q = sole_consumer(ctx, bn->outputs[0], bn_idx, "QuantizeLinear");
        float dq_s, q_s;
        if (!q || q->inputs.size() < 2 || !host_scale(dq->inputs[1], dq_s) || !host_scale(q->inputs[1], q_s)) continue;
        // uint8 in and out: the folded kernel writes uint8
        const tensor_t* qz = q->inputs.size() > 2 ? q->inputs[2] : nullptr;
        if (qz && qz->type != NNR_DATA_TYPE_UINT8) continue;
        if (dq->inputs[0]->type != NNR_DATA_TYPE_UINT8 && dq->inputs[0]->type != NNR_DATA_TYPE_UNDEFINED) continue;
        const tensor_t* dz = dq->inputs.size() > 2 ? dq->inputs[2] : nullptr;
        if (dz && dz->type != NNR_DATA_TYPE_UINT8) continue;
        apply(bn, dq, q, p, dq_s, host_zp(dq, 2), q_s, host_zp(q, 2));
        folded++;
    }
    for (int i = 0; i < n; ++i) {
        operator_t* bn = nodes[i];
        if (!active(bn) || bn->op_type != "BatchNormalization" || !bn->fused_chain.empty()) continue;
        if (!bn_params(bn, p) || !bn->inputs[0] || !fp32_source(ctx, bn->inputs[0])) continue;
        operator_t* q = sole_consumer(ctx, bn->outputs[0], i, "QuantizeLinear");
        float q_s;
        if (!q || q->inputs.size() < 2 || !host_scale(q->inputs[1], q_s)) continue;
        const tensor_t* qz = q->inputs.size() > 2 ? q->inputs[2] : nullptr;
        if (qz && qz->type != NNR_DATA_TYPE_UINT8) continue;
        apply(bn, nullptr, q, p, 0.f, 0, q_s, host_zp(q, 2));
        folded_bnq++;
    }
    ctx->fusion_stats["bn_qdq"] += folded;
    ctx->fusion_stats["bn_q"] += folded_bnq;
}

}  // namespace nnr
