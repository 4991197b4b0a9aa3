// memory_planner.h -- device-memory planner of the HIP backend.
//
// The reference's planner (src/memory_planner.h, src/memory_planner.cpp:33-337)
// shares host buffers between intermediate tensors whose lifetimes do not
// overlap, runs elementwise operators in place, and lets the inputs of a
// Concat live inside its output. This planner keeps those three ideas and
// their rules, on device memory:
//   - one arena (a single device allocation) holds every slot, each slot at a
//     256-byte-aligned offset, so every pooled tensor keeps the alignment the
//     vector kernels check for;
//   - lifetimes are taken over the executed plan: a fused or grouped
//     operator touches, at its own position, every tensor of the nodes whose
//     work it does (those nodes are skipped and never run);
//   - the pool is not cleared between runs (the reference's zero_pool,
//     :333-337): every HIP kernel writes each byte of its output.
#pragma once

#include <cstddef>
#include <string>
#include <vector>

namespace nnr {

struct tensor_t;
struct context_t;
struct operator_t;

struct memory_planner_t {
    enum kind_t : int { SLOT = 0, INPLACE = 1, CONCAT = 2 };
    struct lifetime_t {
        tensor_t* tensor = nullptr;
        int first = 0;              // position of the first node that touches it (its producer)
        int last = 0;               // position of the last node that touches it
        size_t bytes = 0;
        int slot = -1;
        kind_t kind = SLOT;
        int parent = -1;            // INPLACE: the input it overwrites; CONCAT: the Concat output
        size_t concat_offset = 0;   // CONCAT: byte offset inside the parent
        size_t offset = 0;          // byte offset in the arena (after plan)
    };
    struct slot_t {
        size_t size = 0;
        int free_after = -1;        // position of the last use of its current tenant
        size_t offset = 0;
    };

    // lifetime analysis (memory_planner.cpp:33-106)
    void analyze(context_t* ctx);
    // in-place, concat aliasing, best-fit-decreasing slots (:108-280)
    void plan();
    // one device allocation; pooled tensors point into it (:282-331).
    // false (with ctx->last_error set) if the allocation fails
    bool apply();
    void release();
    ~memory_planner_t() { release(); }

    std::vector<lifetime_t> lifetimes;
    std::vector<slot_t> slots;
    int num_intermediates = 0;
    int num_slots = 0;
    int num_inplace = 0;
    int num_concat = 0;
    size_t total_pool_bytes = 0;       // the arena
    size_t total_unpooled_bytes = 0;   // the same tensors one allocation each
    void* arena = nullptr;

private:
    context_t* ctx_ = nullptr;
};

// every tensor an active operator's exec may read or write: its own, and
// those of the nodes fused into it (fused_add, fused_chain, fused_pre,
// fused_other) or launched by it (group_members)
void touched_tensors(const operator_t* op, std::vector<tensor_t*>& out);

}  // namespace nnr
