// registry.h -- operator registry with per-backend resolvers.
//
// Same contract as the reference (src/registry.h:8-28, src/registry.cpp:5-27):
// a resolver takes (opset, pool) and placement-news its operator into the
// pool; resolve tries the preferred backend first and falls back to CPU when
// that resolver is missing or returns nullptr. This build registers its operators
// under backend_t::HIP only; there is no CPU implementation in the product,
// so a nullptr from every resolver means "unsupported here".
#pragma once

#include <functional>
#include <map>
#include <new>
#include <string>

#include "nnr.h"

namespace nnr {

using resolver_fn = operator_t* (*)(int opset, pool_t& pool);

struct registry_t {
    void register_op(const std::string& name, backend_t backend, resolver_fn fn);
    operator_t* solve(const std::string& op_type, int opset, pool_t& pool,
                      backend_t preferred = backend_t::CPU);
    bool has(const std::string& name, backend_t backend) const;

private:
    std::map<std::pair<std::string, backend_t>, resolver_fn> ops_;
};

registry_t& global_registry();

// static registration helper (src/backend/cpu/solve_operator.cpp:18-26)
template <typename T>
T* pool_new(pool_t& pool) {
    return new (pool.alloc(sizeof(T), alignof(T))) T();
}

struct op_registrar_t {
    op_registrar_t(const char* name, backend_t b, resolver_fn fn) {
        global_registry().register_op(name, b, fn);
    }
};

}  // namespace nnr
