// memory_planner.cpp -- lifetimes, slot sharing, in-place and concat aliasing
// over device memory (the reference's src/memory_planner.cpp:33-337).
#include "memory_planner.h"

#include <algorithm>
#include <functional>
#include <unordered_map>
#include <unordered_set>

#include "../../include/nnr_hip.h"
#include "nnr.h"

namespace nnr {

namespace {

constexpr size_t kAlign = 256;   // slot alignment in the arena
constexpr size_t kTiny = 256;    // tensors below this keep their own allocation (:81)

size_t round_up(size_t b) { return (b + kAlign - 1) & ~(kAlign - 1); }

// operators whose HIP kernel reads each output element's operands at the same
// index it writes, so the output may overwrite a same-size input
// (is_inplace_safe, memory_planner.cpp:10-29, restricted to the operators
// this backend registers)
bool inplace_safe(const std::string& op) {
    static const char* const safe[] = {"QLinearAdd", "QLinearMul", "Add", "Sub", "Mul",
                                       "Div",        "Relu",       "Clip", "Gelu"};
    for (const char* s : safe)
        if (op == s) return true;
    return false;
}

// an operator whose exec is exactly its own kernel on its own tensors
bool plain(const operator_t* op) {
    return op->fused_chain.empty() && op->fused_pre.empty() && !op->fused_add && !op->fused_other &&
           op->group_members.empty() && !op->group_leader && op->minmax_count == 0 && !op->minmax_src;
}

bool active(const operator_t* op) { return !op->skip && !op->folded; }

}  // namespace

void touched_tensors(const operator_t* op, std::vector<tensor_t*>& out) {
    auto add_op = [&](const operator_t* o) {
        for (auto* t : o->inputs)
            if (t) out.push_back(t);
        for (auto* t : o->outputs)
            if (t) out.push_back(t);
    };
    add_op(op);
    if (op->fused_other) out.push_back(op->fused_other);
    if (op->fused_add) add_op(op->fused_add);
    if (!op->fused_chain.empty()) {
        // the values a chain passes from stage to stage exist only inside the
        // kernel: the producer's own result (the first stage's first input)
        // and every stage's output, unless it is this operator's output (a
        // post-op applied in place). What else a stage reads -- a bias, the
        // activation scale of a scale product -- the kernel reads itself.
        auto is_out = [&](const tensor_t* t) {
            return std::find(op->outputs.begin(), op->outputs.end(), t) != op->outputs.end();
        };
        std::unordered_set<const tensor_t*> inner;
        const operator_t* first = op->fused_chain.front();
        if (!first->inputs.empty() && first->inputs[0] && !is_out(first->inputs[0])) inner.insert(first->inputs[0]);
        for (auto* o : op->fused_chain)
            for (auto* t : o->outputs)
                if (t && !is_out(t)) inner.insert(t);
        for (auto* o : op->fused_chain) {
            for (auto* t : o->inputs)
                if (t && !inner.count(t)) out.push_back(t);
            for (auto* t : o->outputs)
                if (t && !inner.count(t)) out.push_back(t);
        }
    }
    for (auto* o : op->fused_pre) add_op(o);
    for (auto* o : op->group_members) add_op(o);
}

void memory_planner_t::analyze(context_t* ctx) {
    release();
    ctx_ = ctx;
    lifetimes.clear();
    slots.clear();
    auto& nodes = ctx->nodes;

    // views (Flatten / Reshape): the output borrows its source's memory, so a
    // touch of a view is a touch of the source (:49-67)
    std::unordered_map<tensor_t*, tensor_t*> view_source;
    auto root = [&](tensor_t* t) {
        while (true) {
            if (t->alias_of) { t = t->alias_of; continue; }
            auto it = view_source.find(t);
            if (it == view_source.end()) return t;
            t = it->second;
        }
    };
    for (auto* op : nodes) {
        if (!active(op)) continue;
        const int vi = op->view_input_index();
        if (vi >= 0 && vi < (int)op->inputs.size() && op->inputs[vi] && !op->outputs.empty() && op->outputs[0])
            view_source[op->outputs[0]] = op->inputs[vi];
    }
    // never pooled: graph inputs and outputs (and what a graph output views),
    // initializers and folded constants, memory an operator set up itself
    std::unordered_set<tensor_t*> excluded;
    for (auto& n : ctx->graph_inputs)
        if (tensor_t* t = ctx->find(n)) excluded.insert(root(t));
    for (auto& n : ctx->graph_outputs)
        if (tensor_t* t = ctx->find(n)) {
            excluded.insert(t);
            excluded.insert(root(t));
        }
    for (auto& n : ctx->initializer_names)
        if (tensor_t* t = ctx->find(n)) excluded.insert(t);
    auto poolable = [&](tensor_t* t) {
        return !excluded.count(t) && !t->has_host() && !t->data && t->nbytes() >= kTiny;
    };

    std::unordered_map<tensor_t*, int> index;
    std::vector<tensor_t*> ts;
    for (int i = 0; i < (int)nodes.size(); ++i) {
        operator_t* op = nodes[i];
        if (!active(op)) continue;
        ts.clear();
        touched_tensors(op, ts);
        for (auto* t : ts) {
            tensor_t* r = root(t);
            auto it = index.find(r);
            if (it != index.end()) {
                lifetimes[it->second].last = i;
                continue;
            }
            if (!poolable(r)) continue;
            lifetime_t lt;
            lt.tensor = r;
            lt.first = lt.last = i;
            lt.bytes = r->nbytes();
            index[r] = (int)lifetimes.size();
            lifetimes.push_back(lt);
        }
    }
    num_intermediates = (int)lifetimes.size();
    total_unpooled_bytes = 0;
    for (auto& lt : lifetimes) total_unpooled_bytes += round_up(lt.bytes);
}

void memory_planner_t::plan() {
    auto& nodes = ctx_->nodes;
    std::unordered_map<tensor_t*, int> index;
    for (int i = 0; i < (int)lifetimes.size(); ++i) index[lifetimes[i].tensor] = i;

    // 1. in place: a plain elementwise operator whose same-size input is read
    //    for the last time by it writes over that input (:120-148)
    for (int i = 0; i < (int)lifetimes.size(); ++i) {
        lifetime_t& lt = lifetimes[i];
        operator_t* op = nodes[lt.first];
        if (!active(op) || !plain(op) || !inplace_safe(op->op_type)) continue;
        if (op->outputs.empty() || op->outputs[0] != lt.tensor) continue;
        for (auto* in : op->inputs) {
            if (!in) continue;
            auto it = index.find(in);
            if (it == index.end() || it->second == i) continue;
            lifetime_t& p = lifetimes[it->second];
            if (p.last != lt.first || p.bytes != lt.bytes || in->format != lt.tensor->format) continue;
            lt.kind = INPLACE;
            lt.parent = it->second;
            for (int k = it->second; k >= 0; k = lifetimes[k].kind == INPLACE ? lifetimes[k].parent : -1)
                lifetimes[k].last = std::max(lifetimes[k].last, lt.last);
            break;
        }
    }

    // 2. concat aliasing: the parts of a QLinearConcat that copies every part
    //    (scale, zero point and type equal to the output's), along an axis
    //    with only unit dimensions before it, live inside the output; their
    //    producers write there and the copy is skipped (:150-212). Every part
    //    offset must keep the slot alignment.
    for (int i = 0; i < (int)lifetimes.size(); ++i) {
        lifetime_t& lt = lifetimes[i];
        operator_t* op = nodes[lt.first];
        if (!active(op) || !plain(op) || op->op_type != "QLinearConcat") continue;
        if (op->outputs.empty() || op->outputs[0] != lt.tensor || lt.kind != SLOT) continue;
        tensor_t* y = lt.tensor;
        if (y->format != memory_layout_t::NCHW || y->ndim() < 2 || op->inputs.size() < 5) continue;
        int axis = (int)op->attribute("axis", 0);
        if (axis < 0) axis += y->ndim();
        if (axis < 0 || axis >= y->ndim()) continue;
        long long outer = 1;
        for (int d = 0; d < axis; ++d) outer *= y->dims[d];
        if (outer != 1) continue;
        tensor_t *ys = op->inputs[0], *yz = op->inputs[1];
        if (!ys || !yz || !ys->has_host() || !yz->has_host()) continue;
        const int nt = (int)(op->inputs.size() - 2) / 3;
        bool ok = true;
        size_t off = 0;
        std::unordered_set<tensor_t*> seen;
        std::vector<std::pair<int, size_t>> parts;
        for (int k = 0; k < nt && ok; ++k) {
            tensor_t *x = op->inputs[2 + 3 * k], *xs = op->inputs[3 + 3 * k], *xz = op->inputs[4 + 3 * k];
            auto it = x ? index.find(x) : index.end();
            if (it == index.end() || !seen.insert(x).second) { ok = false; break; }
            lifetime_t& p = lifetimes[it->second];
            if (p.kind != SLOT || p.last != lt.first || x->type != y->type || x->ndim() != y->ndim()) {
                ok = false;
                break;
            }
            for (int d = 0; d < y->ndim(); ++d)
                if (d != axis && x->dims[d] != y->dims[d]) ok = false;
            if (!xs || !xz || !xs->has_host() || !xz->has_host() || xs->scalar_f32() != ys->scalar_f32() ||
                xz->scalar_int() != yz->scalar_int())
                ok = false;
            if (off % kAlign) ok = false;
            parts.emplace_back(it->second, off);
            off += p.bytes;
        }
        if (!ok || off != lt.bytes) continue;
        for (auto& [pi, po] : parts) {
            lifetime_t& p = lifetimes[pi];
            p.kind = CONCAT;
            p.parent = i;
            p.concat_offset = po;
            lt.first = std::min(lt.first, p.first);
            lt.last = std::max(lt.last, p.last);
        }
    }

    // 3. slots, best fit by decreasing size: a slot is free for a tensor
    //    produced after the last use of the slot's latest tenant; it grows
    //    by at most the tensor's own size, else a new slot (:214-262)
    std::vector<int> order;
    for (int i = 0; i < (int)lifetimes.size(); ++i)
        if (lifetimes[i].kind == SLOT) order.push_back(i);
    std::stable_sort(order.begin(), order.end(),
                     [&](int a, int b) { return lifetimes[a].bytes > lifetimes[b].bytes; });
    slots.clear();
    for (int idx : order) {
        lifetime_t& lt = lifetimes[idx];
        int best = -1;
        size_t best_cost = SIZE_MAX;
        for (int s = 0; s < (int)slots.size(); ++s) {
            if (slots[s].free_after >= lt.first) continue;
            const size_t cost = lt.bytes > slots[s].size ? lt.bytes - slots[s].size : 0;
            if (cost < best_cost) {
                best = s;
                best_cost = cost;
            }
        }
        if (best >= 0 && best_cost <= lt.bytes) {
            lt.slot = best;
            slots[best].size = std::max(slots[best].size, lt.bytes);
            slots[best].free_after = lt.last;
        } else {
            lt.slot = (int)slots.size();
            slots.push_back({lt.bytes, lt.last, 0});
        }
    }
    size_t at = 0;
    for (auto& s : slots) {
        s.offset = at;
        at += round_up(s.size);
    }
    total_pool_bytes = at;

    // 4. in-place tensors take their parent's slot (:264-275); concat parts
    //    sit at their offset inside the output
    std::function<size_t(int)> offset_of = [&](int i) -> size_t {
        lifetime_t& lt = lifetimes[i];
        if (lt.kind == INPLACE) {
            lt.slot = lifetimes[lt.parent].slot;
            return offset_of(lt.parent);
        }
        if (lt.kind == CONCAT) return offset_of(lt.parent) + lt.concat_offset;
        return slots[lt.slot].offset;
    };
    for (int i = 0; i < (int)lifetimes.size(); ++i) {
        lifetimes[i].offset = offset_of(i);
        if (lifetimes[i].kind == CONCAT) lifetimes[i].slot = lifetimes[lifetimes[i].parent].slot;
    }
    num_slots = (int)slots.size();
    num_inplace = num_concat = 0;
    for (auto& lt : lifetimes) {
        num_inplace += lt.kind == INPLACE;
        num_concat += lt.kind == CONCAT;
    }
}

bool memory_planner_t::apply() {
    if (total_pool_bytes == 0) return true;
    if (nnrh_malloc(&arena, total_pool_bytes) != NNRH_OK) {
        arena = nullptr;
        return ctx_->fail(std::string("memory planner: arena allocation failed: ") + nnrh_last_error());
    }
    for (auto& lt : lifetimes) {
        lt.tensor->data = (char*)arena + lt.offset;
        lt.tensor->owns_data = false;
    }
    return true;
}

void memory_planner_t::release() {
    if (arena) nnrh_free(arena);
    arena = nullptr;
}

}  // namespace nnr
