// onnx_loader.cpp -- ONNX ModelProto -> context_t (the reference's
// src/format/onnx/onnx_loader.cpp:491-732 over its own protobuf reader,
// src/format/onnx/pb.h, onnx_pb.cpp).
//
// A protobuf wire-format reader of its own (varint / 64-bit / length-
// delimited / 32-bit records; repeated scalars packed or not) decodes the
// messages the graph needs; the graph is then built through the same
// context_t calls in-process builders use (add_initializer / add_input /
// add_node / add_output), so the passes, the registry and the HIP operators
// see a loaded model exactly as they see a built one.
//
// Behaviour kept from the reference:
//   - the default-domain opset ("" or "ai.onnx") is the operators' opset
//     (:690-696);
//   - graph inputs that are initializers are not graph inputs (:702-708);
//   - a symbolic or non-positive dimension becomes 1 (tensor_from_value_info,
//     :394-409), unless the caller passes another value for symbolic ones;
//   - initializer data from raw_data (little-endian) or the typed fields,
//     sub-32-bit types one value per int32_data element (:65-200);
//   - external data: "location" relative to the model's directory, "offset",
//     "length" (:250-300);
//   - an operator no backend resolves becomes a placeholder whose exec fails
//     (:597-602).
// Constant nodes become initializers at load (NNR runs them once in
// fold_run; the value is the same).
#include <algorithm>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <string>
#include <vector>

#include "nnr.h"

namespace nnr {

namespace {

// ---- wire format ------------------------------------------------------------
struct reader_t {
    const uint8_t* p;
    const uint8_t* end;
    bool ok = true;

    bool more() const { return ok && p < end; }
    uint64_t varint() {
        uint64_t v = 0;
        for (int shift = 0; shift < 64; shift += 7) {
            if (p >= end) { ok = false; return 0; }
            const uint8_t b = *p++;
            v |= (uint64_t)(b & 0x7f) << shift;
            if (!(b & 0x80)) return v;
        }
        ok = false;
        return 0;
    }
    uint32_t fixed32() {
        if (end - p < 4) { ok = false; return 0; }
        uint32_t v;
        std::memcpy(&v, p, 4);
        p += 4;
        return v;
    }
    uint64_t fixed64() {
        if (end - p < 8) { ok = false; return 0; }
        uint64_t v;
        std::memcpy(&v, p, 8);
        p += 8;
        return v;
    }
    // a length-delimited record as a sub-reader
    reader_t bytes() {
        const uint64_t n = varint();
        if (!ok || n > (uint64_t)(end - p)) {
            ok = false;
            return {end, end, false};
        }
        reader_t r{p, p + n};
        p += n;
        return r;
    }
    std::string str() {
        reader_t r = bytes();
        return ok ? std::string((const char*)r.p, (size_t)(r.end - r.p)) : std::string();
    }
    // key: field number and wire type
    bool key(int& field, int& wt) {
        const uint64_t k = varint();
        field = (int)(k >> 3);
        wt = (int)(k & 7);
        return ok && field > 0;
    }
    void skip(int wt) {
        switch (wt) {
        case 0: varint(); break;
        case 1: if (end - p < 8) ok = false; else p += 8; break;
        case 2: bytes(); break;
        case 5: if (end - p < 4) ok = false; else p += 4; break;
        default: ok = false;
        }
    }
};

// repeated scalar fields (scalar wire type swt), packed (wire type 2) or one
// record each; any other wire type is skipped
template <typename T, typename F>
void repeated(reader_t& r, int wt, int swt, std::vector<T>& out, F one) {
    if (wt == 2) {
        reader_t s = r.bytes();
        while (s.more()) out.push_back(one(s));
        if (!s.ok) r.ok = false;
    } else if (wt == swt) {
        out.push_back(one(r));
    } else {
        r.skip(wt);
    }
}
// a field of the expected wire type; otherwise it is skipped
bool want(reader_t& r, int wt, int expected) {
    if (wt == expected) return true;
    r.skip(wt);
    return false;
}
int64_t as_i64(reader_t& r) { return (int64_t)r.varint(); }
int32_t as_i32(reader_t& r) { return (int32_t)r.varint(); }
float as_f32(reader_t& r) {
    const uint32_t u = r.fixed32();
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
double as_f64(reader_t& r) {
    const uint64_t u = r.fixed64();
    double d;
    std::memcpy(&d, &u, 8);
    return d;
}
uint64_t as_u64(reader_t& r) { return r.varint(); }

// ---- messages (the fields the graph build reads) ---------------------------
struct tensor_pb {
    std::vector<int64_t> dims;         // 1
    int32_t data_type = 0;             // 2
    std::vector<float> float_data;     // 4
    std::vector<int32_t> int32_data;   // 5
    std::vector<int64_t> int64_data;   // 7
    std::string name;                  // 8
    const uint8_t* raw = nullptr;      // 9
    size_t raw_size = 0;
    bool has_raw = false;
    std::vector<double> double_data;   // 10
    std::vector<uint64_t> uint64_data; // 11
    std::vector<std::pair<std::string, std::string>> external;   // 13
    int32_t data_location = 0;         // 14
};

struct attr_pb {
    std::string name;                  // 1
    float f = 0;                       // 2
    int64_t i = 0;                     // 3
    std::string s;                     // 4
    tensor_pb t;                       // 5
    bool has_t = false, has_f = false, has_i = false, has_s = false;
    std::vector<float> floats;         // 7
    std::vector<int64_t> ints;         // 8
    std::vector<std::string> strings;  // 9
    int32_t type = 0;                  // 20
};

struct node_pb {
    std::vector<std::string> input, output;   // 1, 2
    std::string name, op_type, domain;        // 3, 4, 7
    std::vector<attr_pb> attribute;           // 5
};

struct value_info_pb {
    std::string name;            // 1
    int32_t elem_type = 0;       // type(2).tensor_type(1).elem_type(1)
    std::vector<int64_t> dims;   // ...shape(2).dim(1): dim_value(1), or -1 for dim_param(2)
    bool has_shape = false;
};

struct graph_pb {
    std::vector<node_pb> node;             // 1
    std::vector<tensor_pb> initializer;    // 5
    std::vector<value_info_pb> input;      // 11
    std::vector<value_info_pb> output;     // 12
};

struct model_pb {
    int64_t ir_version = 0;                               // 1
    std::vector<std::pair<std::string, int64_t>> opset;   // 8: domain(1), version(2)
    graph_pb graph;                                       // 7
    bool has_graph = false;
};

void parse_kv(reader_t r, std::pair<std::string, std::string>& kv, bool& ok) {
    int f, wt;
    while (r.more() && r.key(f, wt)) {
        if (f == 1 && wt == 2) kv.first = r.str();
        else if (f == 2 && wt == 2) kv.second = r.str();
        else r.skip(wt);
    }
    ok = ok && r.ok;
}

bool parse_tensor(reader_t r, tensor_pb& t) {
    int f, wt;
    bool ok = true;
    while (r.more() && r.key(f, wt)) {
        switch (f) {
        case 1: repeated(r, wt, 0, t.dims, as_i64); break;
        case 2: if (want(r, wt, 0)) t.data_type = as_i32(r); break;
        case 4: repeated(r, wt, 5, t.float_data, as_f32); break;
        case 5: repeated(r, wt, 0, t.int32_data, as_i32); break;
        case 7: repeated(r, wt, 0, t.int64_data, as_i64); break;
        case 8: if (want(r, wt, 2)) t.name = r.str(); break;
        case 9: {
            if (!want(r, wt, 2)) break;
            reader_t s = r.bytes();
            t.raw = s.p;
            t.raw_size = (size_t)(s.end - s.p);
            t.has_raw = true;
            break;
        }
        case 10: repeated(r, wt, 1, t.double_data, as_f64); break;
        case 11: repeated(r, wt, 0, t.uint64_data, as_u64); break;
        case 13: {
            if (!want(r, wt, 2)) break;
            std::pair<std::string, std::string> kv;
            parse_kv(r.bytes(), kv, ok);
            t.external.push_back(kv);
            break;
        }
        case 14: if (want(r, wt, 0)) t.data_location = as_i32(r); break;
        default: r.skip(wt);
        }
    }
    return ok && r.ok;
}

bool parse_attr(reader_t r, attr_pb& a) {
    int f, wt;
    bool ok = true;
    while (r.more() && r.key(f, wt)) {
        switch (f) {
        case 1: if (want(r, wt, 2)) a.name = r.str(); break;
        case 2: if (want(r, wt, 5)) { a.f = as_f32(r); a.has_f = true; } break;
        case 3: if (want(r, wt, 0)) { a.i = as_i64(r); a.has_i = true; } break;
        case 4: if (want(r, wt, 2)) { a.s = r.str(); a.has_s = true; } break;
        case 5: if (want(r, wt, 2)) { ok = parse_tensor(r.bytes(), a.t) && ok; a.has_t = true; } break;
        case 7: repeated(r, wt, 5, a.floats, as_f32); break;
        case 8: repeated(r, wt, 0, a.ints, as_i64); break;
        case 9: if (want(r, wt, 2)) a.strings.push_back(r.str()); break;
        case 20: if (want(r, wt, 0)) a.type = as_i32(r); break;
        default: r.skip(wt);
        }
    }
    return ok && r.ok;
}

bool parse_node(reader_t r, node_pb& n) {
    int f, wt;
    bool ok = true;
    while (r.more() && r.key(f, wt)) {
        switch (f) {
        case 1: if (want(r, wt, 2)) n.input.push_back(r.str()); break;
        case 2: if (want(r, wt, 2)) n.output.push_back(r.str()); break;
        case 3: if (want(r, wt, 2)) n.name = r.str(); break;
        case 4: if (want(r, wt, 2)) n.op_type = r.str(); break;
        case 5: if (want(r, wt, 2)) { n.attribute.emplace_back(); ok = parse_attr(r.bytes(), n.attribute.back()) && ok; } break;
        case 7: if (want(r, wt, 2)) n.domain = r.str(); break;
        default: r.skip(wt);
        }
    }
    return ok && r.ok;
}

bool parse_shape(reader_t r, value_info_pb& v) {
    int f, wt;
    v.has_shape = true;
    while (r.more() && r.key(f, wt)) {
        if (f == 1 && wt == 2) {   // Dimension
            reader_t d = r.bytes();
            int64_t value = -1;
            int g, wt2;
            while (d.more() && d.key(g, wt2)) {
                if (g == 1 && wt2 == 0) value = as_i64(d);
                else d.skip(wt2);
            }
            if (!d.ok) return false;
            v.dims.push_back(value);
        } else {
            r.skip(wt);
        }
    }
    return r.ok;
}

bool parse_value_info(reader_t r, value_info_pb& v) {
    int f, wt;
    bool ok = true;
    while (r.more() && r.key(f, wt)) {
        if (f == 1 && wt == 2) {
            v.name = r.str();
        } else if (f == 2 && wt == 2) {   // TypeProto
            reader_t tp = r.bytes();
            int g, wt2;
            while (tp.more() && tp.key(g, wt2)) {
                if (g == 1 && wt2 == 2) {   // tensor_type
                    reader_t tt = tp.bytes();
                    int h, wt3;
                    while (tt.more() && tt.key(h, wt3)) {
                        if (h == 1 && wt3 == 0) v.elem_type = as_i32(tt);
                        else if (h == 2 && wt3 == 2) ok = parse_shape(tt.bytes(), v) && ok;
                        else tt.skip(wt3);
                    }
                    ok = ok && tt.ok;
                } else {
                    tp.skip(wt2);
                }
            }
            ok = ok && tp.ok;
        } else {
            r.skip(wt);
        }
    }
    return ok && r.ok;
}

bool parse_graph(reader_t r, graph_pb& g) {
    int f, wt;
    bool ok = true;
    while (r.more() && r.key(f, wt)) {
        switch (f) {
        case 1: if (want(r, wt, 2)) { g.node.emplace_back(); ok = parse_node(r.bytes(), g.node.back()) && ok; } break;
        case 5: if (want(r, wt, 2)) { g.initializer.emplace_back(); ok = parse_tensor(r.bytes(), g.initializer.back()) && ok; } break;
        case 11: if (want(r, wt, 2)) { g.input.emplace_back(); ok = parse_value_info(r.bytes(), g.input.back()) && ok; } break;
        case 12: if (want(r, wt, 2)) { g.output.emplace_back(); ok = parse_value_info(r.bytes(), g.output.back()) && ok; } break;
        default: r.skip(wt);
        }
    }
    return ok && r.ok;
}

bool parse_model(reader_t r, model_pb& m) {
    int f, wt;
    bool ok = true;
    while (r.more() && r.key(f, wt)) {
        switch (f) {
        case 1: if (want(r, wt, 0)) m.ir_version = as_i64(r); break;
        case 7: if (want(r, wt, 2)) { ok = parse_graph(r.bytes(), m.graph) && ok; m.has_graph = true; } break;
        case 8: {
            if (!want(r, wt, 2)) break;
            reader_t s = r.bytes();
            std::string domain;
            int64_t version = 0;
            int g, wt2;
            while (s.more() && s.key(g, wt2)) {
                if (g == 1 && wt2 == 2) domain = s.str();
                else if (g == 2 && wt2 == 0) version = as_i64(s);
                else s.skip(wt2);
            }
            ok = ok && s.ok;
            m.opset.emplace_back(domain, version);
            break;
        }
        default: r.skip(wt);
        }
    }
    return ok && r.ok;
}

// ---- tensor data --------------------------------------------------------------
bool supported_type(data_type_t dt) {
    switch (dt) {
    case NNR_DATA_TYPE_FLOAT32: case NNR_DATA_TYPE_UINT8: case NNR_DATA_TYPE_INT8:
    case NNR_DATA_TYPE_UINT16: case NNR_DATA_TYPE_INT16: case NNR_DATA_TYPE_INT32:
    case NNR_DATA_TYPE_INT64: case NNR_DATA_TYPE_BOOL: case NNR_DATA_TYPE_FLOAT16:
        return true;
    default:
        return false;
    }
}

// largest initializer the loader will hold on the host (a larger one is a
// malformed or hostile file, not a model this backend can place in HBM)
constexpr size_t MAX_INITIALIZER_BYTES = (size_t)64 << 30;

// host bytes of a TensorProto (onnx_tensor_copy_from_proto, :65-200; external
// data :250-300). Fewer stored values than elements leave zeros, as the
// reference's copy does.
bool tensor_bytes(const tensor_pb& t, const std::string& model_dir, std::vector<uint8_t>& out,
                  std::string& err) {
    const data_type_t dt = data_type_from_onnx(t.data_type);
    if (!supported_type(dt)) {
        err = "tensor " + t.name + ": unsupported data type " + std::to_string(t.data_type);
        return false;
    }
    std::vector<int> dims;
    for (int64_t d : t.dims) {
        if (d < 0 || d > INT32_MAX) {
            err = "tensor " + t.name + ": bad dimension";
            return false;
        }
        dims.push_back((int)d);
    }
    const size_t sz = data_type_sizeof(dt);
    size_t n = 0;
    if (!checked_count(dims, sz, &n) || n * sz > MAX_INITIALIZER_BYTES) {
        err = "tensor " + t.name + ": element count too large";
        return false;
    }
    out.assign(n * sz, 0);
    if (t.data_location == 1) {   // EXTERNAL
        std::string location;
        long long offset = 0, length = -1;
        for (auto& kv : t.external) {
            if (kv.first == "location") location = kv.second;
            else if (kv.first == "offset") offset = std::atoll(kv.second.c_str());
            else if (kv.first == "length") length = std::atoll(kv.second.c_str());
        }
        if (location.empty()) {
            err = "tensor " + t.name + ": external data without a location";
            return false;
        }
        if (offset < 0) {
            err = "tensor " + t.name + ": negative external data offset";
            return false;
        }
        const std::string path = model_dir + location;
        std::ifstream f(path, std::ios::binary);
        if (!f) {
            err = "tensor " + t.name + ": external data file not found: " + path;
            return false;
        }
        const size_t want = length > 0 ? std::min((size_t)length, out.size()) : out.size();
        f.seekg(offset);
        f.read((char*)out.data(), (std::streamsize)want);
        if ((size_t)f.gcount() != want) {
            err = "tensor " + t.name + ": external data file too short: " + path;
            return false;
        }
        return true;
    }
    if (t.has_raw) {
        std::memcpy(out.data(), t.raw, std::min(t.raw_size, out.size()));
        return true;
    }
    switch (dt) {
    case NNR_DATA_TYPE_FLOAT32:
        std::memcpy(out.data(), t.float_data.data(), std::min(n, t.float_data.size()) * 4);
        break;
    case NNR_DATA_TYPE_INT32:
        std::memcpy(out.data(), t.int32_data.data(), std::min(n, t.int32_data.size()) * 4);
        break;
    case NNR_DATA_TYPE_INT64:
        std::memcpy(out.data(), t.int64_data.data(), std::min(n, t.int64_data.size()) * 8);
        break;
    default:   // uint8 / int8 / uint16 / int16 / bool / float16: one value per int32 element
        for (size_t i = 0; i < std::min(n, t.int32_data.size()); ++i)
            std::memcpy(out.data() + i * sz, &t.int32_data[i], sz);
    }
    return true;
}

std::vector<int> dims_of(const tensor_pb& t) {
    std::vector<int> d;
    for (int64_t v : t.dims) d.push_back((int)v);
    return d;
}

}  // namespace

bool load_onnx(context_t* ctx, const void* data, size_t size, const std::string& model_dir, int sym_dim) {
    if (!ctx || !data) return ctx ? ctx->fail("load_onnx: NULL data") : false;
    if (!ctx->nodes.empty() || !ctx->graph_inputs.empty()) return ctx->fail("load_onnx: context is not empty");
    model_pb m;
    reader_t r{(const uint8_t*)data, (const uint8_t*)data + size};
    if (!parse_model(r, m) || !m.has_graph) return ctx->fail("load_onnx: not a valid ONNX ModelProto");
    std::string dir = model_dir;
    if (!dir.empty() && dir.back() != '/') dir += '/';

    for (auto& o : m.opset)
        if (o.first.empty() || o.first == "ai.onnx") {
            ctx->opset = (int)o.second;
            break;
        }
    const graph_pb& g = m.graph;
    std::string err;
    std::vector<uint8_t> bytes;
    for (auto& t : g.initializer) {
        if (t.name.empty()) continue;
        if (!tensor_bytes(t, dir, bytes, err)) return ctx->fail("load_onnx: " + err);
        if (!ctx->add_initializer(t.name, data_type_from_onnx(t.data_type), dims_of(t), bytes.data()))
            return false;
    }
    for (auto& v : g.input) {
        if (v.name.empty() || ctx->initializer_names.count(v.name)) continue;
        if (!supported_type(data_type_from_onnx(v.elem_type)))
            return ctx->fail("load_onnx: input " + v.name + ": unsupported element type");
        std::vector<int> d;
        for (int64_t x : v.dims) d.push_back(x > 0 ? (int)x : (sym_dim > 0 ? sym_dim : 1));
        if (!ctx->add_input(v.name, data_type_from_onnx(v.elem_type), d)) return false;
    }
    int unnamed = 0;
    for (auto& n : g.node) {
        if (n.op_type == "Constant" && (n.domain.empty() || n.domain == "ai.onnx")) {
            // value (tensor) / value_float(s) / value_int(s) -> an initializer
            if (n.output.empty() || n.output[0].empty()) continue;
            bool done = false;
            for (auto& a : n.attribute) {
                if (a.name == "value" && a.has_t) {
                    if (!tensor_bytes(a.t, dir, bytes, err)) return ctx->fail("load_onnx: " + err);
                    done = ctx->add_initializer(n.output[0], data_type_from_onnx(a.t.data_type), dims_of(a.t), bytes.data());
                } else if (a.name == "value_float") {
                    done = ctx->add_initializer(n.output[0], NNR_DATA_TYPE_FLOAT32, {}, &a.f);
                } else if (a.name == "value_int") {
                    done = ctx->add_initializer(n.output[0], NNR_DATA_TYPE_INT64, {}, &a.i);
                } else if (a.name == "value_floats") {
                    done = ctx->add_initializer(n.output[0], NNR_DATA_TYPE_FLOAT32, {(int)a.floats.size()},
                                                a.floats.data());
                } else if (a.name == "value_ints") {
                    done = ctx->add_initializer(n.output[0], NNR_DATA_TYPE_INT64, {(int)a.ints.size()},
                                                a.ints.data());
                }
                if (done) break;
            }
            if (!done) return ctx->fail("load_onnx: Constant " + n.name + ": no value this loader reads");
            continue;
        }
        std::vector<std::pair<std::string, attr_t>> attrs;
        for (auto& a : n.attribute) {
            if (a.name.empty()) continue;
            // the discriminator (:419-489); files without it: the field present
            int type = a.type;
            if (type == 0)
                type = a.has_f ? 1 : a.has_i ? 2 : a.has_s ? 3 : a.has_t ? 4 : !a.floats.empty() ? 6
                     : !a.ints.empty() ? 7 : !a.strings.empty() ? 8 : 0;
            attr_t v;
            switch (type) {
            case 1: v.kind = attr_t::kind_t::FLOAT; v.f = a.f; break;
            case 2: v.kind = attr_t::kind_t::INT; v.i = a.i; break;
            case 3: v.kind = attr_t::kind_t::STRING; v.s = a.s; break;
            case 6: v.kind = attr_t::kind_t::FLOATS; v.floats = a.floats; break;
            case 7: v.kind = attr_t::kind_t::INTS; v.ints = a.ints; break;
            default: continue;   // tensors, graphs, string lists: not read by this backend's operators
            }
            attrs.emplace_back(a.name, std::move(v));
        }
        const std::string name = n.name.empty() ? n.op_type + "_" + std::to_string(unnamed++) : n.name;
        if (!ctx->add_node(n.op_type, name, n.input, n.output, std::move(attrs))) return false;
    }
    for (auto& v : g.output)
        if (!v.name.empty() && !ctx->add_output(v.name)) return false;
    return true;
}

bool load_onnx_file(context_t* ctx, const std::string& path, int sym_dim) {
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) return ctx->fail("load_onnx: cannot open " + path);
    const std::streamsize n = f.tellg();
    std::vector<uint8_t> buf((size_t)std::max<std::streamsize>(n, 0));
    f.seekg(0);
    if (n > 0 && !f.read((char*)buf.data(), n)) return ctx->fail("load_onnx: cannot read " + path);
    const size_t slash = path.find_last_of('/');
    const std::string dir = slash == std::string::npos ? std::string() : path.substr(0, slash + 1);
    return load_onnx(ctx, buf.data(), buf.size(), dir, sym_dim);
}

}  // namespace nnr
