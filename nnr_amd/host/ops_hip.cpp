// ops_hip.cpp -- operators of the HIP backend, registered under
// backend_t::HIP. Each one keeps the reference operator's inputs, attributes,
// shape rules and error behaviour (init/reshape return false, exec returns
// false on a device error) and crosses into device code only through the C
// ABI of include/nnr_hip.h on the context's stream.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>

#include "nnr.h"
#include "nnr_hip.h"
#include "registry.h"

namespace nnr {
namespace {

bool ok(operator_t* op, int rc) {
    if (rc != NNRH_OK) {
        op->ctx->last_error = nnrh_last_error();
        return false;
    }
    return true;
}
bool bad(operator_t* op, const std::string& msg) {
    op->ctx->last_error = op->op_type + " " + op->node_name + ": " + msg;
    return false;
}
int qdtype(data_type_t t) {
    return t == NNR_DATA_TYPE_UINT8 ? NNRH_U8 : t == NNR_DATA_TYPE_INT8 ? NNRH_S8
         : t == NNR_DATA_TYPE_INT32 ? NNRH_I32 : -1;
}
tensor_t* in(const operator_t* op, size_t i) { return op->inputs.size() > i ? op->inputs[i] : nullptr; }
bool has_zp(tensor_t* t) { return t && t->ndata > 0; }
int32_t zp_value(tensor_t* t) { return has_zp(t) ? t->scalar_int() : 0; }

// ===========================================================================
// QuantizeLinear (src/backend/cpu/QuantizeLinear.cpp), per-tensor
struct QuantizeLinear_hip : operator_t {
    bool init() override {
        layout_mask = LAYOUT_ALL;
        return inputs.size() >= 2 && outputs.size() == 1;
    }
    bool reshape() override {
        tensor_t *x = inputs[0], *s = inputs[1], *z = in(this, 2), *y = outputs[0];
        data_type_t t = z ? z->type : NNR_DATA_TYPE_UINT8;
        if (t != NNR_DATA_TYPE_UINT8 && t != NNR_DATA_TYPE_INT8) return bad(this, "only uint8/int8 output");
        if (!s->has_host() || s->ndata != 1) return bad(this, "only a constant per-tensor scale");
        y->format = x->format;
        return y->reshape(x->dims, t);
    }
    bool exec() override {
        tensor_t* y = outputs[0];
        return ok(this, nnrh_quantize_linear((const float*)inputs[0]->data, inputs[0]->ndata,
                                             inputs[1]->scalar_f32(), zp_value(in(this, 2)),
                                             qdtype(y->type), y->data, ctx->stream));
    }
};

// DequantizeLinear (src/backend/cpu/DequantizeLinear.cpp), per-tensor
struct DequantizeLinear_hip : operator_t {
    bool init() override {
        layout_mask = LAYOUT_ALL;
        return inputs.size() >= 2 && outputs.size() == 1;
    }
    bool reshape() override {
        tensor_t *x = inputs[0], *s = inputs[1], *y = outputs[0];
        if (!s->has_host() || s->ndata != 1) return bad(this, "only a constant per-tensor scale");
        if (qdtype(x->type) < 0) return bad(this, "input must be uint8/int8/int32");
        y->format = x->format;
        return y->reshape(x->dims, NNR_DATA_TYPE_FLOAT32);
    }
    bool exec() override {
        tensor_t* x = inputs[0];
        return ok(this, nnrh_dequantize_linear(x->data, qdtype(x->type), x->ndata,
                                               inputs[1]->scalar_f32(), zp_value(in(this, 2)),
                                               (float*)outputs[0]->data, ctx->stream));
    }
};

// DynamicQuantizeLinear (src/backend/cpu/DynamicQuantizeLinear.cpp)
struct DynamicQuantizeLinear_hip : operator_t {
    bool init() override {
        layout_mask = LAYOUT_ALL;
        return inputs.size() == 1 && outputs.size() == 3;
    }
    bool reshape() override {
        tensor_t* x = inputs[0];
        outputs[0]->format = x->format;
        outputs[0]->reshape(x->dims, NNR_DATA_TYPE_UINT8);
        outputs[1]->reshape({}, NNR_DATA_TYPE_FLOAT32);
        outputs[2]->reshape({}, NNR_DATA_TYPE_UINT8);
        outputs[1]->device_only = outputs[2]->device_only = true;
        return true;
    }
    // the (min, max) partials of the two-pass quantize; the producer's pairs
    // or bytes replace them when a fusion set minmax_src / codes_src
    size_t workspace_size() const override {
        return codes_src || minmax_src ? 0 : nnrh_dynamic_quantize_workspace();
    }
    std::string variant() const override { return codes_src ? "Codes" : minmax_src ? "MinMaxIn" : ""; }
    bool exec() override {
        if (codes_src) return codes_src->quantize_codes(outputs[0], outputs[1], outputs[2]);
        if (minmax_src)
            return ok(this, nnrh_dynamic_quantize_linear_parts(
                                (const float*)inputs[0]->data, inputs[0]->ndata, minmax_src->minmax_parts,
                                minmax_src->minmax_count, (uint8_t*)outputs[0]->data,
                                (float*)outputs[1]->data, (uint8_t*)outputs[2]->data, ctx->stream));
        return ok(this, nnrh_dynamic_quantize_linear(
                            (const float*)inputs[0]->data, inputs[0]->ndata, (uint8_t*)outputs[0]->data,
                            (float*)outputs[1]->data, (uint8_t*)outputs[2]->data, ctx->workspace, ctx->stream));
    }
};

// ===========================================================================
// QLinearConv (src/backend/cpu/QLinearConv.cpp)
struct QLinearConv_hip : operator_t {
    int auto_pad = 0;   // NOTSET, SAME_UPPER, SAME_LOWER, VALID
    int group = 1;
    std::vector<int> kernels, dilations, pads, strides;
    int cpads[4] = {0, 0, 0, 0};
    nnrh_qconv_t h = nullptr;
    int branch = 0;
    ~QLinearConv_hip() override { nnrh_qconv_destroy(h); }

    bool init() override {
        if (!(inputs.size() >= 8 && inputs.size() <= 9 && outputs.size() == 1)) return false;
        std::string ap = attribute_s("auto_pad", "NOTSET");
        auto_pad = ap == "SAME_UPPER" ? 1 : ap == "SAME_LOWER" ? 2 : ap == "VALID" ? 3 : 0;
        group = (int)attribute("group", 1);
        for (auto v : attribute_ints("kernel_shape")) kernels.push_back((int)v);
        if (kernels.empty() && inputs[3])
            for (int i = 2; i < inputs[3]->ndim(); ++i) kernels.push_back(inputs[3]->dims[i]);
        auto d = attribute_ints("dilations"), p = attribute_ints("pads"), s = attribute_ints("strides");
        dilations.assign(kernels.size(), 1);
        strides.assign(kernels.size(), 1);
        pads.assign(kernels.size() * 2, 0);
        for (size_t i = 0; i < d.size() && i < dilations.size(); ++i) dilations[i] = (int)d[i];
        for (size_t i = 0; i < s.size() && i < strides.size(); ++i) strides[i] = (int)s[i];
        for (size_t i = 0; i < p.size() && i < pads.size(); ++i) pads[i] = (int)p[i];
        return true;
    }
    bool dense_pointwise() const override {
        if (group != 1 || kernels.size() != 2 || auto_pad == 1 || auto_pad == 2) return false;
        for (size_t i = 0; i < 2; ++i)
            if (kernels[i] != 1 || strides[i] != 1 || dilations[i] != 1 || pads[i] != 0 || pads[i + 2] != 0)
                return false;
        return true;
    }
    bool per_channel_zp() const {
        tensor_t* z = in((operator_t*)this, 5);
        if (!z || z->ndata <= 1 || !z->has_host()) return false;
        for (size_t i = 1; i < z->ndata; ++i)
            if (z->host[i] != z->host[0]) return true;
        return false;
    }
    // 3-D tensors: the reference's exec_typed path (QLinearConv.cpp:286-334)
    bool conv1d() const { return inputs[0]->ndim() == 3; }
    bool reshape() override {
        tensor_t *x = inputs[0], *w = inputs[3], *y = outputs[0];
        if (x->ndim() == 3) {
            if (w->ndim() != 3 || kernels.size() != 1) return bad(this, "1-D convolution needs 3-D weights");
            // conv_shape.h:21-81 along the single spatial axis
            const int ek = (kernels[0] - 1) * dilations[0] + 1, xd = x->dims[2];
            int o;
            if (auto_pad == 1 || auto_pad == 2) {
                int pad = (int)(ceilf(xd / (float)strides[0]) - 1) * strides[0] + ek - xd;
                if (auto_pad == 1) { cpads[0] = pad / 2; cpads[1] = pad - cpads[0]; }
                else { cpads[1] = pad / 2; cpads[0] = pad - cpads[1]; }
                o = (int)ceilf(xd / (float)strides[0]);
            } else if (auto_pad == 3) {
                cpads[0] = cpads[1] = 0;
                o = (int)ceilf((xd - ek + 1) / (float)strides[0]);
            } else {
                cpads[0] = pads[0];
                cpads[1] = pads[1];
                o = (int)floorf((xd + cpads[0] + cpads[1] - ek) / (float)strides[0] + 1);
            }
            layout_mask = LAYOUT_NCHW;
            if (!y->reshape({x->dims[0], w->dims[0], o}, x->type)) return false;
            if (ctx->shape_only) return describe(true);
            return build();
        }
        if (x->ndim() != 4 || w->ndim() != 4 || kernels.size() != 2)
            return bad(this, "only 1-D and 2-D convolution (3-D and 4-D tensors)");
        // conv_shape.h:21-81
        int out[2];
        for (int i = 0; i < 2; ++i) {
            int ek = (kernels[i] - 1) * dilations[i] + 1;
            int xd = x->dims[i + 2];
            if (auto_pad == 1 || auto_pad == 2) {
                int pad = (int)(ceilf(xd / (float)strides[i]) - 1) * strides[i] + ek - xd;
                if (auto_pad == 1) { cpads[i] = pad / 2; cpads[i + 2] = pad - cpads[i]; }
                else { cpads[i + 2] = pad / 2; cpads[i] = pad - cpads[i + 2]; }
                out[i] = (int)ceilf(xd / (float)strides[i]);
            } else if (auto_pad == 3) {
                cpads[i] = cpads[i + 2] = 0;
                out[i] = (int)ceilf((xd - ek + 1) / (float)strides[i]);
            } else {
                cpads[i] = pads[i];
                cpads[i + 2] = pads[i + 2];
                out[i] = (int)floorf((xd + cpads[i] + cpads[i + 2] - ek) / (float)strides[i] + 1);
            }
        }
        // QLinearConv_reshape.h:36-46: NHWC-capable for uint8, group 1 or depthwise
        const bool dw = group == w->dims[0] && w->dims[1] == 1;
        layout_mask = LAYOUT_NCHW;
        if (x->type == NNR_DATA_TYPE_UINT8 && !per_channel_zp() && (dw || group == 1))
            layout_mask = LAYOUT_NCHW | LAYOUT_NHWC;
        if (!y->reshape({x->dims[0], w->dims[0], out[0], out[1]}, x->type)) return false;
        if (ctx->shape_only) return describe(true);
        return build();
    }
    nnrh_qconv_desc d{};
    // fill the C-ABI descriptor; with dispatch_only, only resolve the branch
    bool describe(bool dispatch_only) {
        tensor_t *x = inputs[0], *w = inputs[3], *y = outputs[0];
        tensor_t *xs = inputs[1], *xz = inputs[2], *ws = inputs[4], *wz = inputs[5];
        tensor_t *ys = inputs[6], *yz = inputs[7], *b = in(this, 8);
        if (w->type != NNR_DATA_TYPE_INT8 || !w->has_host()) return bad(this, "weights must be constant int8");
        if (!xs->has_host() || !ws->has_host() || !ys->has_host()) return bad(this, "scales must be constant");
        if ((xz && xz->ndata && !xz->has_host()) || (yz && yz->ndata && !yz->has_host()) ||
            (wz && wz->ndata && !wz->has_host()) || (b && !b->has_host()))
            return bad(this, "zero points / bias must be constant");
        d = nnrh_qconv_desc{};
        if (conv1d()) {
            d.N = x->dims[0]; d.C = x->dims[1]; d.H = 1; d.W = x->dims[2];
            d.OC = w->dims[0]; d.kH = 1; d.kW = w->dims[2]; d.group = group;
            d.sH = 1; d.sW = strides[0]; d.dH = 1; d.dW = dilations[0];
            d.pad_l = cpads[0]; d.pad_r = cpads[1];
            d.oH = 1; d.oW = y->dims[2];
            d.spatial_dims = 1;
        } else {
            d.N = x->dims[0]; d.C = x->dims[1]; d.H = x->dims[2]; d.W = x->dims[3];
            d.OC = w->dims[0]; d.kH = w->dims[2]; d.kW = w->dims[3]; d.group = group;
            d.sH = strides[0]; d.sW = strides[1]; d.dH = dilations[0]; d.dW = dilations[1];
            d.pad_t = cpads[0]; d.pad_l = cpads[1]; d.pad_b = cpads[2]; d.pad_r = cpads[3];
            d.oH = y->dims[2]; d.oW = y->dims[3];
            d.x_nhwc = x->format == memory_layout_t::NHWC;
            d.y_nhwc = y->format == memory_layout_t::NHWC;
        }
        d.post_fn = post_fn ? 1 : 0;
        d.act_dtype = qdtype(x->type);
        d.x_scale = xs->scalar_f32();
        d.x_zp = zp_value(xz);
        d.w_scale_host = ws->h<float>();
        d.w_scale_count = (int)ws->ndata;
        d.w_zp_host = (wz && wz->ndata) ? wz->h<int8_t>() : nullptr;
        d.w_zp_count = wz ? (int)wz->ndata : 0;
        d.y_scale = ys->scalar_f32();
        d.y_zp = zp_value(yz);
        d.w_host = w->h<int8_t>();
        d.bias_host = (b && b->ndata) ? b->h<int32_t>() : nullptr;
        if (dispatch_only) return ok(this, nnrh_qconv_dispatch(&d, &branch));
        return true;
    }
    bool build() {
        if (!describe(false)) return false;
        nnrh_qconv_destroy(h);
        h = nullptr;
        if (!ok(this, nnrh_qconv_create(&h, &d))) return false;
        nnrh_qconv_branch(h, &branch);
        return true;
    }
    bool fused_quant = false;   // input is the fp32 tensor of a fused QuantizeLinear
    tensor_t* conv_out = nullptr;   // a fused MaxPool's input (the conv's own result)
    // the MaxPool after this first-layer conv runs in its kernel
    bool fuse_maxpool(operator_t* pool, const int* k, const int* st, const int* pads) override {
        if (!h || fused_add || conv_out || pool->outputs.empty()) return false;
        tensor_t *y = outputs[0], *py = pool->outputs[0];
        if (y->type != NNR_DATA_TYPE_UINT8 || y->format != memory_layout_t::NHWC || py->format != y->format)
            return false;
        if (nnrh_qconv_fuse_maxpool(h, k[0], k[1], st[0], st[1], pads[0], pads[1], pads[2], pads[3]) != NNRH_OK)
            return false;
        conv_out = y;
        return true;
    }
    bool exec() override {
        if (fused_add)
            return ok(this, nnrh_qconv_run_add(h, inputs[0]->data, fused_other->data, outputs[0]->data,
                                               ctx->stream));
        if (fused_quant)
            return ok(this, nnrh_qconv_run_f32(h, (const float*)inputs[0]->data, outputs[0]->data, ctx->stream));
        return ok(this, nnrh_qconv_run(h, inputs[0]->data, outputs[0]->data, ctx->stream));
    }
    // the QuantizeLinear producing this first-layer conv's input (per-tensor
    // fp32 scale, uint8 zero point, fp32 NCHW input) runs in its layout kernel
    bool fuse_quantize_input(operator_t* q) override {
        if (!h || fused_add || q->inputs.size() < 2 || q->outputs.empty()) return false;
        tensor_t *qx = q->inputs[0], *qs = q->inputs[1], *qz = in(q, 2), *qy = q->outputs[0];
        if (!qx || qx->type != NNR_DATA_TYPE_FLOAT32 || qx->format != memory_layout_t::NCHW) return false;
        if (qy->type != NNR_DATA_TYPE_UINT8 || !qs->has_host() || qs->ndata != 1 || qs->type != NNR_DATA_TYPE_FLOAT32)
            return false;
        if (qz && (!qz->has_host() || qz->ndata != 1 || qz->type != NNR_DATA_TYPE_UINT8)) return false;
        if (nnrh_qconv_fuse_quantize(h, qs->scalar_f32(), zp_value(qz)) != NNRH_OK) return false;
        fused_quant = true;
        return true;
    }
    bool fuse_residual_add(operator_t* add, int conv_side) override {
        if (!h || add->inputs.size() != 8) return false;
        for (int i : {1, 2, 4, 5, 6, 7})
            if (add->inputs[i] && add->inputs[i]->ndata && !add->inputs[i]->has_host()) return false;
        tensor_t* y = outputs[0];
        tensor_t* ay = add->outputs[0];
        if (!ay || ay->dims != y->dims || ay->type != y->type || ay->format != y->format) return false;
        nnrh_qadd_fuse_desc fd{};
        fd.conv_is_a = conv_side == 0;
        fd.a_scale = add->inputs[1]->scalar_f32();
        fd.a_zp = zp_value(add->inputs[2]);
        fd.b_scale = add->inputs[4]->scalar_f32();
        fd.b_zp = zp_value(add->inputs[5]);
        fd.y_scale = add->inputs[6]->scalar_f32();
        fd.y_zp = zp_value(add->inputs[7]);
        return nnrh_qconv_fuse_add(h, &fd) == NNRH_OK;
    }
    double num_ops() const override {
        const tensor_t *w = inputs[3], *y = conv_out ? conv_out : outputs[0];
        if (y->ndim() == 3 && w->ndim() == 3)
            return 2.0 * y->dims[0] * y->dims[1] * y->dims[2] * (double)w->dims[1] * w->dims[2];
        if (y->ndim() != 4 || w->ndim() != 4) return 0;
        return 2.0 * y->dims[0] * y->dims[1] * y->dims[2] * y->dims[3] * (double)w->dims[1] * w->dims[2] *
               w->dims[3];
    }
    double num_bytes() const override {
        const tensor_t *x = inputs[0], *w = inputs[3], *y = outputs[0];
        double other = fused_other ? (double)fused_other->nbytes() : 0.0;
        return (double)x->nbytes() + (double)y->nbytes() + (double)w->nbytes() + 8.0 * w->dims[0] + other;
    }
    std::string variant() const override {
        static const char* names[] = {"?", "DW", "FIRST", "DIRECT", "PACKED", "NR16", "IM2COL_S1", "IM2COL", "FLOAT",
                                      "TYPED"};
        std::string v = branch >= 0 && branch <= 9 ? names[branch] : "?";
        return fused_add ? v + "+Add" : conv_out ? v + "+MaxPool" : v;
    }
};

// ===========================================================================
// QLinearMatMul (src/backend/cpu/QLinearMatMul.cpp), constant B
struct QLinearMatMul_hip : operator_t {
    nnrh_qmatmul_t h = nullptr;
    nnrh_qmatmul_group_t grp = nullptr;   // leader of a grouped launch
    int m = 0, n = 0, k = 0, batch = 1;
    bool codes = false;   // set_codes_out: output 0 holds the uint8 bytes of the chain
    ~QLinearMatMul_hip() override {
        nnrh_qmatmul_group_destroy(grp);
        nnrh_qmatmul_destroy(h);
    }
    bool init() override {
        layout_mask = LAYOUT_NCHW;
        return inputs.size() == 8 && outputs.size() == 1;
    }
    bool reshape() override {
        tensor_t *a = inputs[0], *b = inputs[3], *y = outputs[0];
        if (a->ndim() < 2 || b->ndim() != 2) return bad(this, "B must be a 2-D matrix");
        m = a->dims[a->ndim() - 2];
        k = a->dims[a->ndim() - 1];
        if (b->dims[0] != k) return bad(this, "inner dimensions differ");
        n = b->dims[1];
        batch = 1;
        std::vector<int> d(a->dims.begin(), a->dims.end() - 1);
        for (int i = 0; i + 2 < a->ndim(); ++i) batch *= a->dims[i];
        d.push_back(n);
        if (!y->reshape(d, inputs[7]->type)) return false;
        if (ctx->shape_only) return true;
        if (!b->has_host()) return bad(this, "B must be a constant initializer");
        nnrh_qmatmul_desc dsc{};
        dsc.m = m; dsc.n = n; dsc.k = k;
        dsc.a_dtype = qdtype(a->type);
        dsc.b_dtype = qdtype(b->type);
        dsc.y_dtype = qdtype(inputs[7]->type);
        dsc.scale_dtype = inputs[1]->type == NNR_DATA_TYPE_FLOAT16 ? NNRH_F16 : NNRH_F32;
        static const float one = 1.0f;
        static const uint8_t zero_u8 = 0;
        dsc.a_scale_host = inputs[1]->has_host() ? (const void*)inputs[1]->host.data() : (const void*)&one;
        dsc.a_zp_host = inputs[2]->has_host() ? (const void*)inputs[2]->host.data() : (const void*)&zero_u8;
        dsc.b_scale_host = inputs[4]->host.data();
        dsc.b_zp_host = inputs[5] && inputs[5]->has_host() ? (const void*)inputs[5]->host.data() : (const void*)&zero_u8;
        dsc.y_scale_host = inputs[6]->host.data();
        dsc.y_zp_host = inputs[7]->host.data();
        dsc.b_host = b->host.data();
        if (!inputs[4]->has_host() || !inputs[6]->has_host() || !inputs[7]->has_host())
            return bad(this, "b/y quantization must be constant");
        nnrh_qmatmul_destroy(h);
        h = nullptr;
        return ok(this, nnrh_qmatmul_create(&h, &dsc));
    }
    bool fuse_dq_bias(operator_t* dq, operator_t* add) override {
        if (!h) return false;
        tensor_t* f = dq->outputs[0];
        tensor_t* bias = add->inputs[0] == f ? add->inputs[1] : add->inputs[0];
        tensor_t* y = add->outputs[0];
        // the bias must be a vector over the last axis of the result
        if (bias->ndata != (size_t)n) return false;
        for (int i = 0; i + 1 < bias->ndim(); ++i)
            if (bias->dims[i] != 1) return false;
        if (y->dims != f->dims || y->type != NNR_DATA_TYPE_FLOAT32) return false;
        return nnrh_qmatmul_fuse_dq_bias(h, dq->inputs[1]->scalar_f32(), zp_value(in(dq, 2)),
                                         bias->h<float>()) == NNRH_OK;
    }
    bool fuse_gelu(operator_t* ge) override {
        if (ge->attribute_s("approximate", "none") != "none") return false;
        if (ge->outputs[0]->dims != ge->inputs[0]->dims) return false;
        return nnrh_qmatmul_fuse_gelu(h) == NNRH_OK;
    }
    int minmax_pairs() const override {
        int c = 0;
        if (!h || fused_chain.empty() || nnrh_qmatmul_minmax_count(h, batch, &c) != NNRH_OK) return 0;
        return c;
    }
    bool set_minmax_out(float* parts, int pairs) override {
        return nnrh_qmatmul_set_minmax_out(h, parts, pairs) == NNRH_OK;
    }
    bool set_codes_out(bool on) override {
        if (!h || fused_chain.empty()) return false;
        if (group_leader && group_leader != this) {
            codes = on;   // its bytes come from the leader's launch
            return true;
        }
        const int rc = grp ? nnrh_qmatmul_group_set_codes_out(grp, on ? 1 : 0) : nnrh_qmatmul_set_codes_out(h, on ? 1 : 0);
        if (rc != NNRH_OK) return false;
        codes = on;
        return true;
    }
    bool codes_params(int* zp, float* scale, const float** bias) const override {
        return h && nnrh_qmatmul_dq_params(h, zp, scale, bias) == NNRH_OK;
    }
    bool quantize_codes(tensor_t* y, tensor_t* y_scale, tensor_t* y_zp) override {
        return ok(this, nnrh_qmatmul_dynamic_quantize_codes(h, outputs[0]->data, batch, (uint8_t*)y->data,
                                                            (float*)y_scale->data, (uint8_t*)y_zp->data,
                                                            ctx->stream));
    }
    bool groupable() const override { return h && fused_chain.size() == 2 && !codes; }
    bool same_group_input(const operator_t* o) const override {
        return dynamic_cast<const QLinearMatMul_hip*>(o) && o->inputs[0] == inputs[0] &&
               o->inputs[1] == inputs[1] && o->inputs[2] == inputs[2];
    }
    bool fuse_group(const std::vector<operator_t*>& members) override {
        if (!h || fused_chain.size() != 2) return false;
        std::vector<nnrh_qmatmul_t> hs{h};
        for (auto* op : members) {
            auto* o = dynamic_cast<QLinearMatMul_hip*>(op);
            if (!o || !o->h || o->fused_chain.size() != 2 || o->m != m || o->n != n || o->k != k ||
                o->batch != batch)
                return false;
            hs.push_back(o->h);
        }
        return nnrh_qmatmul_group_create(&grp, hs.data(), (int)hs.size()) == NNRH_OK;
    }
    std::string variant() const override {
        if (fused_chain.empty()) return "";
        std::string v = fused_chain.size() > 2 ? "+DQ+Bias+Gelu" : "+DQ+Bias";
        if (grp) v += "+Group" + std::to_string(group_members.size() + 1);
        else if (group_leader) v += "(grouped)";
        if (codes) v += "+Codes";
        return v;
    }
    bool exec() override {
        if (group_leader && group_leader != this) return true;   // written by the leader's launch
        const float* a_s_dev = inputs[1]->has_host() ? nullptr : (const float*)inputs[1]->data;
        const void* a_z_dev = inputs[2]->has_host() ? nullptr : inputs[2]->data;
        if (grp) {
            std::vector<void*> ys{outputs[0]->data};
            for (auto* op : group_members) ys.push_back(op->outputs[0]->data);
            return ok(this, nnrh_qmatmul_group_run(grp, inputs[0]->data, batch * m, ys.data(), a_s_dev, a_z_dev,
                                                   ctx->stream));
        }
        return exec_single(a_s_dev, a_z_dev);
    }
    bool exec_single(const float* a_s_dev, const void* a_z_dev) {
        return ok(this, nnrh_qmatmul_run(h, inputs[0]->data, batch > 1 ? (long long)m * k : 0,
                                         outputs[0]->data, batch, a_s_dev, a_z_dev, ctx->stream));
    }
    // a grouped launch's work is counted on its leader (members run nothing)
    double num_ops() const override {
        if (group_leader && group_leader != this) return 0.0;
        return 2.0 * batch * m * (double)n * k * (double)(grp ? group_members.size() + 1 : 1);
    }
};

// MatMulInteger (src/backend/cpu/MatMulInteger.cpp). With a constant B and
// the per-channel dynamic-quantization chain after it (Cast -> Mul by the
// scale product Mul(a_scale, w_scale) -> Add(bias) [-> Gelu], fused by
// fuse_matmul_integer_scale), the whole chain runs in one GEMM (sh).
struct MatMulInteger_hip : operator_t {
    nnrh_matmul_integer_t h = nullptr;
    nnrh_qmatmul_t sh = nullptr;            // fused chain
    nnrh_qmatmul_group_t grp = nullptr;     // leader of a grouped launch
    tensor_t* a_scale = nullptr;            // fused chain: the activation scale
    int m = 0, n = 0, k = 0, batch = 1;
    bool b_batched = false;
    ~MatMulInteger_hip() override {
        nnrh_qmatmul_group_destroy(grp);
        nnrh_qmatmul_destroy(sh);
        nnrh_matmul_integer_destroy(h);
    }
    bool init() override { return inputs.size() >= 2 && inputs.size() <= 4 && outputs.size() == 1; }
    bool reshape() override {
        tensor_t *a = inputs[0], *b = inputs[1], *y = outputs[0];
        if (a->ndim() < 2 || b->ndim() < 2) return bad(this, "operands must be at least 2-D");
        m = a->dims[a->ndim() - 2];
        k = a->dims[a->ndim() - 1];
        n = b->dims[b->ndim() - 1];
        if (b->dims[b->ndim() - 2] != k) return bad(this, "inner dimensions differ");
        batch = 1;
        for (int i = 0; i + 2 < a->ndim(); ++i) batch *= a->dims[i];
        int bb = 1;
        for (int i = 0; i + 2 < b->ndim(); ++i) bb *= b->dims[i];
        if (bb != 1 && bb != batch) return bad(this, "only equal or broadcast B batches");
        b_batched = bb > 1;
        std::vector<int> d(a->dims.begin(), a->dims.end() - 1);
        d.push_back(n);
        if (!y->reshape(d, NNR_DATA_TYPE_INT32)) return false;
        if (ctx->shape_only) return true;
        // A's zero point may come from the device (DynamicQuantizeLinear);
        // B's must be a constant
        if (in(this, 2) && in(this, 2)->ndata > 1) return bad(this, "per-row A zero points");
        if (in(this, 3) && in(this, 3)->ndata && !in(this, 3)->has_host())
            return bad(this, "B's zero point must be constant");
        if (in(this, 3) && in(this, 3)->ndata > 1) return bad(this, "per-column B zero points");
        nnrh_matmul_integer_destroy(h);
        h = nullptr;
        return ok(this, nnrh_matmul_integer_create(&h, m, n, k, qdtype(a->type), qdtype(b->type), batch));
    }
    // the chain Cast -> Mul(scale product) [-> Add(bias)] after a constant B
    bool fuse_int_scale(tensor_t* a_s, tensor_t* w_scale, tensor_t* bias) override {
        tensor_t* b = inputs[1];
        if (!b->has_host() || b->ndim() != 2 || b_batched) return false;
        if (!w_scale->has_host() || w_scale->type != NNR_DATA_TYPE_FLOAT32 || w_scale->ndata != (size_t)n) return false;
        if (bias && (!bias->has_host() || bias->type != NNR_DATA_TYPE_FLOAT32 || bias->ndata != (size_t)n)) return false;
        if (a_s->ndata != 1 || a_s->type != NNR_DATA_TYPE_FLOAT32) return false;
        nnrh_mmi_scaled_desc d{};
        d.m = m; d.n = n; d.k = k;
        d.a_dtype = qdtype(inputs[0]->type);
        d.b_dtype = qdtype(b->type);
        d.b_host = b->host.data();
        d.a_zp = in(this, 2) && in(this, 2)->has_host() ? zp_value(in(this, 2)) : 0;
        d.b_zp = zp_value(in(this, 3));
        d.a_scale = a_s->has_host() ? a_s->scalar_f32() : 1.0f;
        d.w_scale_host = w_scale->h<float>();
        d.bias_host = bias ? bias->h<float>() : nullptr;
        nnrh_qmatmul_destroy(sh);
        sh = nullptr;
        if (nnrh_matmul_integer_scaled_create(&sh, &d) != NNRH_OK) return false;
        a_scale = a_s;
        return true;
    }
    bool fuse_gelu(operator_t* ge) override {
        if (!sh || ge->attribute_s("approximate", "none") != "none") return false;
        if (ge->outputs[0]->dims != ge->inputs[0]->dims) return false;
        return nnrh_qmatmul_fuse_gelu(sh) == NNRH_OK;
    }
    int minmax_pairs() const override {
        int c = 0;
        if (!sh || nnrh_qmatmul_minmax_count(sh, batch, &c) != NNRH_OK) return 0;
        return c;
    }
    bool set_minmax_out(float* parts, int pairs) override {
        return sh && nnrh_qmatmul_set_minmax_out(sh, parts, pairs) == NNRH_OK;
    }
    bool groupable() const override {
        return sh && !fused_chain.empty() && fused_chain.back()->op_type != "Gelu";
    }
    bool same_group_input(const operator_t* o) const override {
        auto* x = dynamic_cast<const MatMulInteger_hip*>(o);
        return x && x->inputs[0] == inputs[0] && in(x, 2) == in(this, 2) && x->a_scale == a_scale;
    }
    bool fuse_group(const std::vector<operator_t*>& members) override {
        if (!groupable()) return false;
        std::vector<nnrh_qmatmul_t> hs{sh};
        for (auto* op : members) {
            auto* o = dynamic_cast<MatMulInteger_hip*>(op);
            if (!o || !o->groupable() || o->m != m || o->n != n || o->k != k || o->batch != batch) return false;
            hs.push_back(o->sh);
        }
        return nnrh_qmatmul_group_create(&grp, hs.data(), (int)hs.size()) == NNRH_OK;
    }
    std::string variant() const override {
        if (!sh) return "";
        std::string v = "+Cast+Scale";
        for (auto* op : fused_chain) {
            if (op->op_type == "Add") v += "+Bias";
            if (op->op_type == "Gelu") v += "+Gelu";
        }
        if (grp) v += "+Group" + std::to_string(group_members.size() + 1);
        else if (group_leader) v += "(grouped)";
        return v;
    }
    bool exec() override {
        tensor_t* az = in(this, 2);
        const void* az_dev = az && az->ndata && !az->has_host() ? az->data : nullptr;
        if (sh) {
            if (group_leader && group_leader != this) return true;   // written by the leader's launch
            const float* as_dev = a_scale->has_host() ? nullptr : (const float*)a_scale->data;
            if (grp) {
                std::vector<void*> ys{outputs[0]->data};
                for (auto* op : group_members) ys.push_back(op->outputs[0]->data);
                return ok(this, nnrh_qmatmul_group_run(grp, inputs[0]->data, batch * m, ys.data(), as_dev, az_dev,
                                                       ctx->stream));
            }
            return ok(this, nnrh_qmatmul_run(sh, inputs[0]->data, batch > 1 ? (long long)m * k : 0,
                                             outputs[0]->data, batch, as_dev, az_dev, ctx->stream));
        }
        if (az_dev)
            return ok(this, nnrh_matmul_integer_run_dev_zp(h, inputs[0]->data, batch > 1 ? (long long)m * k : 0,
                                                           inputs[1]->data, b_batched ? (long long)k * n : 0, az_dev,
                                                           zp_value(in(this, 3)), (int32_t*)outputs[0]->data,
                                                           batch, ctx->stream));
        return ok(this, nnrh_matmul_integer_run(h, inputs[0]->data, batch > 1 ? (long long)m * k : 0,
                                                inputs[1]->data, b_batched ? (long long)k * n : 0,
                                                zp_value(in(this, 2)), zp_value(in(this, 3)),
                                                (int32_t*)outputs[0]->data, batch, ctx->stream));
    }
    double num_ops() const override {
        if (group_leader && group_leader != this) return 0.0;
        return 2.0 * batch * m * (double)n * k * (double)(grp ? group_members.size() + 1 : 1);
    }
};

// Cast to float (src/backend/cpu/Cast.cpp) from int32 / uint8 / int8
struct Cast_hip : operator_t {
    bool init() override {
        layout_mask = LAYOUT_ALL;
        return inputs.size() == 1 && outputs.size() == 1;
    }
    bool reshape() override {
        if (attribute("to", 0) != 1) return bad(this, "only Cast to float (to = 1)");
        const data_type_t t = inputs[0]->type;
        if (t != NNR_DATA_TYPE_INT32 && t != NNR_DATA_TYPE_UINT8 && t != NNR_DATA_TYPE_INT8)
            return bad(this, "Cast from int32 / uint8 / int8 only");
        outputs[0]->format = inputs[0]->format;
        return outputs[0]->reshape(inputs[0]->dims, NNR_DATA_TYPE_FLOAT32);
    }
    bool exec() override {
        const data_type_t t = inputs[0]->type;
        const int dt = t == NNR_DATA_TYPE_INT32 ? NNRH_I32 : t == NNR_DATA_TYPE_UINT8 ? NNRH_U8 : NNRH_S8;
        return ok(this, nnrh_cast_to_f32(inputs[0]->data, dt, (float*)outputs[0]->data, inputs[0]->ndata,
                                         ctx->stream));
    }
};

// ===========================================================================
// QLinearAdd (src/backend/cpu/QLinearAdd.cpp)
struct QLinearAdd_hip : operator_t {
    int kind = 0;
    bool swap = false;
    int C = 0, HW = 0;
    bool init() override {
        layout_mask = LAYOUT_ALL;
        return inputs.size() == 8 && outputs.size() == 1;
    }
    bool reshape() override {
        tensor_t *a = inputs[0], *b = inputs[3], *y = outputs[0];
        const tensor_t* full = a->ndata >= b->ndata ? a : b;
        const tensor_t* other = a->ndata >= b->ndata ? b : a;
        swap = false;
        if (a->dims == b->dims) {
            kind = 0;
        } else if (b->ndata == 1) {
            kind = 1;
        } else if (a->ndata == 1) {
            kind = 2;
        } else if (full->ndim() == 4 && other->ndata == (size_t)full->dims[1] &&
                   (other->ndim() == 1 || (other->ndim() == 4 && other->dims[0] == 1 && other->dims[2] == 1 &&
                                           other->dims[3] == 1))) {
            kind = 3;
            swap = full == b;
            C = full->dims[1];
            HW = full->dims[2] * full->dims[3];
        } else {
            return bad(this, "general broadcasting is not supported");
        }
        y->format = full->format;
        return y->reshape(full->dims, a->type);
    }
    bool exec() override {
        tensor_t *a = inputs[0], *b = inputs[3];
        float as = inputs[1]->scalar_f32(), bs = inputs[4]->scalar_f32(), ys = inputs[6]->scalar_f32();
        int az = zp_value(inputs[2]), bz = zp_value(inputs[5]), yz = zp_value(inputs[7]);
        if (swap)
            return ok(this, nnrh_qlinear_add(3, b->data, a->data, outputs[0]->data, outputs[0]->ndata, C, HW,
                                             outputs[0]->format == memory_layout_t::NHWC, qdtype(a->type),
                                             bs, bz, as, az, ys, yz, ctx->stream));
        return ok(this, nnrh_qlinear_add(kind, a->data, b->data, outputs[0]->data, outputs[0]->ndata, C, HW,
                                         outputs[0]->format == memory_layout_t::NHWC, qdtype(a->type), as,
                                         az, bs, bz, ys, yz, ctx->stream));
    }
};

// QLinearMul (src/backend/cpu/QLinearMul.cpp:17-231): the broadcast kinds of
// classify_broadcast (util.h:50-67) but the general one
struct QLinearMul_hip : operator_t {
    int kind = 0;
    bool swap = false;
    int C = 0, HW = 0;
    bool init() override {
        layout_mask = LAYOUT_ALL;
        return inputs.size() == 8 && outputs.size() == 1;
    }
    bool reshape() override {
        tensor_t *a = inputs[0], *b = inputs[3], *y = outputs[0];
        const tensor_t* full = a->ndata >= b->ndata ? a : b;
        const tensor_t* other = a->ndata >= b->ndata ? b : a;
        swap = false;
        if (a->dims == b->dims) {
            kind = 0;
        } else if (a->ndata == 1) {     // A_SCALAR is tested first (util.h:56)
            kind = 2;
        } else if (b->ndata == 1) {
            kind = 1;
        } else if (full->ndim() == 4 && other->ndata == (size_t)full->dims[1] &&
                   (other->ndim() == 1 || (other->ndim() == 4 && other->dims[0] == 1 && other->dims[2] == 1 &&
                                           other->dims[3] == 1) ||
                    (other->ndim() == 3 && other->dims[1] == 1 && other->dims[2] == 1))) {
            kind = 3;
            swap = full == b;
            C = full->dims[1];
            HW = full->dims[2] * full->dims[3];
        } else {
            return bad(this, "general broadcasting is not supported");
        }
        y->format = full->format;
        return y->reshape(full->dims, a->type);
    }
    bool exec() override {
        tensor_t *a = inputs[0], *b = inputs[3];
        float as = inputs[1]->scalar_f32(), bs = inputs[4]->scalar_f32(), ys = inputs[6]->scalar_f32();
        int az = zp_value(inputs[2]), bz = zp_value(inputs[5]), yz = zp_value(inputs[7]);
        const int nhwc = outputs[0]->format == memory_layout_t::NHWC;
        if (swap)   // per channel with A the [C] operand (QLinearMul.cpp:127-131)
            return ok(this, nnrh_qlinear_mul(3, b->data, a->data, outputs[0]->data, outputs[0]->ndata, C, HW, nhwc,
                                             qdtype(a->type), bs, bz, as, az, ys, yz, ctx->stream));
        return ok(this, nnrh_qlinear_mul(kind, a->data, b->data, outputs[0]->data, outputs[0]->ndata, C, HW, nhwc,
                                         qdtype(a->type), as, az, bs, bz, ys, yz, ctx->stream));
    }
};

// QLinearGlobalAveragePool (src/backend/cpu/QLinearGlobalAveragePool.cpp):
// the kernel reads NCHW or NHWC (the same integer sums), y is [N][C][1..]
struct QLinearGlobalAveragePool_hip : operator_t {
    bool init() override {
        layout_mask = LAYOUT_ALL;
        return inputs.size() == 5 && outputs.size() == 1;
    }
    bool reshape() override {
        tensor_t* x = inputs[0];
        if (x->ndim() < 3) return bad(this, "needs at least 3 dimensions");
        std::vector<int> d(x->dims.size(), 1);
        d[0] = x->dims[0];
        d[1] = x->dims[1];
        outputs[0]->format = x->format;
        return outputs[0]->reshape(d, x->type);
    }
    bool exec() override {
        tensor_t* x = inputs[0];
        const int N = x->dims[0], C = x->dims[1];
        const int sp = (int)(x->ndata / ((size_t)N * C));
        return ok(this, nnrh_qlinear_global_avgpool(x->data, outputs[0]->data, N, C, sp,
                                                    x->format == memory_layout_t::NHWC, qdtype(x->type),
                                                    inputs[1]->scalar_f32(), zp_value(inputs[2]),
                                                    inputs[3]->scalar_f32(), zp_value(inputs[4]), ctx->stream));
    }
};

// QLinearAveragePool (src/backend/cpu/QLinearAveragePool.cpp): 2-D, the
// reference's attributes (kernel_shape, strides, pads, ceil_mode; no
// count_include_pad); NCHW or NHWC
struct QLinearAveragePool_hip : operator_t {
    std::vector<int> kernels, pads, strides;
    int ceil_mode = 0;
    bool init() override {
        layout_mask = LAYOUT_ALL;
        if (inputs.size() != 5 || outputs.size() != 1) return false;
        for (auto v : attribute_ints("kernel_shape")) kernels.push_back((int)v);
        if (kernels.size() != 2) return false;   // :28
        auto s = attribute_ints("strides"), p = attribute_ints("pads");
        strides = {s.size() > 0 ? (int)s[0] : 1, s.size() > 1 ? (int)s[1] : 1};
        pads = {0, 0, 0, 0};
        for (size_t i = 0; i < p.size() && i < 4; ++i) pads[i] = (int)p[i];
        ceil_mode = (int)attribute("ceil_mode", 0);
        return true;
    }
    bool reshape() override {
        tensor_t* x = inputs[0];
        if (x->ndim() != 4) return bad(this, "4-D input only");
        const int N = x->dims[0], C = x->dims[1], H = x->dims[2], W = x->dims[3];
        int oH, oW;
        if (ceil_mode) {   // :55-57
            oH = (int)ceilf((H + pads[0] + pads[2] - kernels[0]) / (float)strides[0] + 1);
            oW = (int)ceilf((W + pads[1] + pads[3] - kernels[1]) / (float)strides[1] + 1);
        } else {
            oH = (H + pads[0] + pads[2] - kernels[0]) / strides[0] + 1;
            oW = (W + pads[1] + pads[3] - kernels[1]) / strides[1] + 1;
        }
        outputs[0]->format = x->format;
        return outputs[0]->reshape({N, C, oH, oW}, x->type);
    }
    bool exec() override {
        tensor_t *x = inputs[0], *y = outputs[0];
        return ok(this, nnrh_qlinear_avgpool(x->data, y->data, x->dims[0], x->dims[1], x->dims[2], x->dims[3],
                                             y->dims[2], y->dims[3], kernels[0], kernels[1], strides[0], strides[1],
                                             pads[0], pads[1], x->format == memory_layout_t::NHWC, qdtype(x->type),
                                             inputs[1]->scalar_f32(), zp_value(inputs[2]), inputs[3]->scalar_f32(),
                                             zp_value(inputs[4]), ctx->stream));
    }
};

// QLinearConcat (src/backend/cpu/QLinearConcat.cpp): inputs (Y_scale, Y_zp,
// then X, X_scale, X_zp per tensor). Chunks as the reference forms them: the
// logical NCHW rows (:119-166), or each pixel's channels when all 4-D inputs
// are NHWC and the axis is 1 (:170-236)
struct QLinearConcat_hip : operator_t {
    int axis = 0;
    bool init() override {
        layout_mask = LAYOUT_NCHW;
        if (inputs.size() < 5 || outputs.size() != 1 || (inputs.size() - 2) % 3) return false;
        axis = (int)attribute("axis", 0);
        return true;
    }
    int ntens() const { return (int)(inputs.size() - 2) / 3; }
    bool reshape() override {
        tensor_t* t0 = inputs[2];
        const int nd = t0->ndim();
        const int a = axis < 0 ? axis + nd : axis;
        if (a < 0 || a >= nd) return bad(this, "axis");
        std::vector<int> d(t0->dims.begin(), t0->dims.end());
        for (int i = 1; i < ntens(); ++i) {
            tensor_t* t = inputs[2 + 3 * i];
            if (t->ndim() != nd) return bad(this, "ranks differ");
            for (int k = 0; k < nd; ++k) {
                if (k == a) d[k] += t->dims[k];
                else if (t->dims[k] != t0->dims[k]) return bad(this, "shapes differ");
            }
        }
        // NHWC only along channels of 4-D int8 tensors (:58-62)
        layout_mask = (nd == 4 && a == 1) ? (LAYOUT_NCHW | LAYOUT_NHWC) : LAYOUT_NCHW;
        bool nhwc = true;
        for (int i = 0; i < ntens(); ++i) nhwc &= inputs[2 + 3 * i]->format == memory_layout_t::NHWC;
        if (!nhwc)
            for (int i = 0; i < ntens(); ++i)
                if (inputs[2 + 3 * i]->format == memory_layout_t::NHWC)
                    return bad(this, "inputs mix NCHW and NHWC");
        if (nhwc && !(nd == 4 && a == 1)) return bad(this, "NHWC inputs concatenated along a non-channel axis");
        outputs[0]->format = nhwc ? memory_layout_t::NHWC : memory_layout_t::NCHW;
        return outputs[0]->reshape(d, t0->type);
    }
    bool exec() override {
        tensor_t* y = outputs[0];
        const int nd = y->ndim();
        const int a = axis < 0 ? axis + nd : axis;
        const bool nhwc = y->format == memory_layout_t::NHWC;
        long long outer = 1, inner = 1;
        if (nhwc) {
            outer = (long long)y->dims[0] * y->dims[2] * y->dims[3];
        } else {
            for (int k = 0; k < a; ++k) outer *= y->dims[k];
            for (int k = a + 1; k < nd; ++k) inner *= y->dims[k];
        }
        const long long row = nhwc ? y->dims[1] : (long long)y->dims[a] * inner;
        const float ys = inputs[0]->scalar_f32();
        const int yz = zp_value(inputs[1]);
        // one launch for all parts, unless the memory planner placed parts
        // inside y (then only the others are copied, part by part)
        bool aliased = false;
        {
            long long o2 = 0;
            for (int i = 0; i < ntens(); ++i) {
                tensor_t* t = inputs[2 + 3 * i];
                aliased |= outer == 1 && (const char*)t->data == (const char*)y->data + o2;
                o2 += nhwc ? t->dims[1] : (long long)t->dims[a] * inner;
            }
        }
        if (!aliased) {
            std::vector<const void*> xs;
            std::vector<long long> cnts;
            std::vector<float> scs;
            std::vector<int> zps;
            for (int i = 0; i < ntens(); ++i) {
                tensor_t* t = inputs[2 + 3 * i];
                xs.push_back(t->data);
                cnts.push_back(nhwc ? t->dims[1] : (long long)t->dims[a] * inner);
                scs.push_back(inputs[3 + 3 * i]->scalar_f32());
                zps.push_back(zp_value(inputs[4 + 3 * i]));
            }
            return ok(this, nnrh_qlinear_concat(ntens(), xs.data(), cnts.data(), scs.data(), zps.data(), outer,
                                                qdtype(inputs[2]->type), ys, yz, y->data, ctx->stream));
        }
        long long off = 0;
        for (int i = 0; i < ntens(); ++i) {
            tensor_t* t = inputs[2 + 3 * i];
            const long long cnt = nhwc ? t->dims[1] : (long long)t->dims[a] * inner;
            // the memory planner placed this part inside y (its producer
            // wrote it there): nothing to copy
            if (outer == 1 && (const char*)t->data == (const char*)y->data + off) {
                off += cnt;
                continue;
            }
            if (!ok(this, nnrh_qlinear_concat_part(t->data, y->data, outer, cnt, row, off, qdtype(t->type),
                                                   inputs[3 + 3 * i]->scalar_f32(), zp_value(inputs[4 + 3 * i]), ys,
                                                   yz, ctx->stream)))
                return false;
            off += cnt;
        }
        return true;
    }
};

// ===========================================================================
// ConvInteger (src/backend/cpu/ConvInteger.cpp): 4-D, int32 NCHW output.
// Attributes and output extents as :30-143 (auto_pad NOTSET / SAME_UPPER /
// SAME_LOWER / VALID with the reference's float ceil / floor formulas); the
// convolution reads the begin pads (:185). x_zero_point scalar, w_zero_point
// scalar or per output channel (:150-176). Exact int32 (see nnrh_conv_integer).
struct ConvInteger_hip : operator_t {
    std::vector<int> kernels, dilations, pads, strides;
    std::string auto_pad;
    int group = 1;
    int cp[4] = {0, 0, 0, 0};
    nnrh_conv_integer_t h = nullptr;
    int32_t* wzp_dev = nullptr;
    ~ConvInteger_hip() override {
        if (h) nnrh_conv_integer_destroy(h);
    }
    bool init() override {
        if (inputs.size() < 2 || outputs.size() != 1) return false;
        auto_pad = attribute_s("auto_pad", "NOTSET");
        group = (int)attribute("group", 1);
        for (auto v : attribute_ints("kernel_shape")) kernels.push_back((int)v);
        for (auto v : attribute_ints("dilations")) dilations.push_back((int)v);
        for (auto v : attribute_ints("pads")) pads.push_back((int)v);
        for (auto v : attribute_ints("strides")) strides.push_back((int)v);
        return true;
    }
    int zp_at(size_t i, int idx) const {
        const tensor_t* z = inputs.size() > i ? inputs[i] : nullptr;
        if (!z || !z->has_host()) return 0;
        if (z->type == NNR_DATA_TYPE_UINT8) return z->h<uint8_t>()[idx];
        if (z->type == NNR_DATA_TYPE_INT8) return z->h<int8_t>()[idx];
        return 0;
    }
    bool reshape() override {
        tensor_t *x = inputs[0], *w = inputs[1];
        if (x->ndim() != 4 || w->ndim() != 4) return bad(this, "4-D input and weights only");
        if (x->type != NNR_DATA_TYPE_UINT8 && x->type != NNR_DATA_TYPE_INT8) return bad(this, "uint8 / int8 input");
        if (kernels.empty()) kernels = {w->dims[2], w->dims[3]};
        if (dilations.empty()) dilations = {1, 1};
        if (strides.empty()) strides = {1, 1};
        if (pads.empty()) pads = {0, 0, 0, 0};
        if (kernels.size() != 2 || dilations.size() != 2 || strides.size() != 2 || pads.size() != 4)
            return bad(this, "2-D attributes");
        int dims[2];
        for (int i = 0; i < 2; ++i) {
            const int in = x->dims[2 + i], ke = (kernels[i] - 1) * dilations[i] + 1, st = strides[i];
            if (auto_pad == "SAME_UPPER" || auto_pad == "SAME_LOWER") {
                const int pad = (int)(ceilf(in / (float)st) - 1) * st + ke - in;
                const int small = pad / 2, large = pad - small;
                cp[i] = auto_pad == "SAME_UPPER" ? small : large;
                cp[i + 2] = auto_pad == "SAME_UPPER" ? large : small;
                dims[i] = (int)ceilf(in / (float)st);
            } else if (auto_pad == "VALID") {
                cp[i] = cp[i + 2] = 0;
                dims[i] = (int)ceilf((in - ke + 1) / (float)st);
            } else {
                cp[i] = pads[i];
                cp[i + 2] = pads[i + 2];
                dims[i] = (int)floorf((in + cp[i] + cp[i + 2] - ke) / (float)st + 1);
            }
        }
        outputs[0]->format = memory_layout_t::NCHW;
        if (!outputs[0]->reshape({x->dims[0], w->dims[0], dims[0], dims[1]}, NNR_DATA_TYPE_INT32)) return false;
        if (ctx->shape_only || h) return true;
        const int OC = w->dims[0];
        if (x->dims[1] != w->dims[1] * group) return bad(this, "channels != weight channels * group");
        if (nnrh_conv_integer_create(&h, x->dims[0], x->dims[1], x->dims[2], x->dims[3], OC, kernels[0], kernels[1],
                                     strides[0], strides[1], cp[0], cp[1], dilations[0], dilations[1], dims[0],
                                     dims[1], group, qdtype(x->type), qdtype(w->type)) != NNRH_OK)
            return bad(this, nnrh_last_error());
        const tensor_t* wz = inputs.size() > 3 ? inputs[3] : nullptr;
        if (wz && wz->ndata > 1) {
            if (!wz->has_host() || (int)wz->ndata != OC) return bad(this, "w_zero_point: constant [OC] expected");
            std::vector<int32_t> v(OC);
            for (int c = 0; c < OC; ++c) v[c] = zp_at(3, c);
            wzp_dev = (int32_t*)ctx->device_alloc(v.size() * sizeof(int32_t));
            if (!wzp_dev || nnrh_memcpy(wzp_dev, v.data(), v.size() * sizeof(int32_t), 0, ctx->stream) != NNRH_OK ||
                nnrh_stream_synchronize(ctx->stream) != NNRH_OK)
                return bad(this, "w_zero_point upload failed");
        }
        return true;
    }
    bool exec() override {
        return ok(this, nnrh_conv_integer_run(h, inputs[0]->data, inputs[1]->data, zp_at(2, 0), wzp_dev ? 0 : zp_at(3, 0),
                                              wzp_dev, (int32_t*)outputs[0]->data, ctx->stream));
    }
    double num_ops() const override {
        const tensor_t* w = inputs[1];
        return 2.0 * (double)outputs[0]->ndata * w->dims[1] * w->dims[2] * w->dims[3];
    }
};

// ===========================================================================
// BatchNormalization (src/backend/cpu/BatchNormalization.cpp), inference.
// After fold_bn_qdq its scale / bias inputs hold the combined A / B and it
// writes uint8 from uint8 (DQ -> BN -> Q) or fp32 (BN -> Q) input
// (:246-376); otherwise fp32 -> fp32 with alpha = scale / sqrt(var + eps) in
// double and beta = bias - alpha * mean (:126-134), uploaded at reshape.
// NCHW or NHWC for 4-D inputs (:30-40).
struct BatchNormalization_hip : operator_t {
    float eps = 1e-5f;
    bool folded_u8 = false;
    float* ab = nullptr;   // fp32 path: alpha[C] | beta[C] on the device
    bool init() override {
        if (inputs.size() < 5 || outputs.empty()) return false;
        eps = attribute_f("epsilon", 1e-5f);
        return attribute("training_mode", 0) == 0;   // inference only
    }
    bool fold_affine_u8() override {
        folded_u8 = true;
        return true;
    }
    bool fold_affine_u8_possible() const override { return true; }
    bool reshape() override {
        tensor_t* x = inputs[0];
        if (x->ndim() < 2) return bad(this, "needs at least 2 dimensions");
        layout_mask = x->ndim() == 4 ? (LAYOUT_NCHW | LAYOUT_NHWC) : LAYOUT_NCHW;
        outputs[0]->format = x->format;
        const int C = x->dims[1];
        for (int k = 1; k <= 4; ++k)
            if (!inputs[k] || (int)inputs[k]->ndata != C || inputs[k]->type != NNR_DATA_TYPE_FLOAT32)
                return bad(this, "scale / bias / mean / var must be fp32 [C]");
        if (folded_u8) {
            if (x->type != NNR_DATA_TYPE_UINT8 && x->type != NNR_DATA_TYPE_FLOAT32)
                return bad(this, "folded: uint8 or fp32 input");
            return outputs[0]->reshape(x->dims, NNR_DATA_TYPE_UINT8);
        }
        if (x->type != NNR_DATA_TYPE_FLOAT32) return bad(this, "fp32 input only");
        if (!ctx->shape_only && !ab) {
            for (int k = 1; k <= 4; ++k)
                if (!inputs[k]->has_host()) return bad(this, "scale / bias / mean / var must be constants");
            const float *sc = inputs[1]->h<float>(), *bi = inputs[2]->h<float>();
            const float *me = inputs[3]->h<float>(), *va = inputs[4]->h<float>();
            std::vector<float> h(2 * (size_t)C);
            for (int c = 0; c < C; ++c) {
                const float a = (float)(sc[c] / std::sqrt((double)va[c] + eps));
                h[c] = a;
                h[C + c] = bi[c] - a * me[c];
            }
            ab = (float*)ctx->device_alloc(h.size() * sizeof(float));
            if (!ab) return bad(this, "device allocation failed");
            if (nnrh_memcpy(ab, h.data(), h.size() * sizeof(float), 0, ctx->stream) != NNRH_OK ||
                nnrh_stream_synchronize(ctx->stream) != NNRH_OK)
                return bad(this, nnrh_last_error());
        }
        return outputs[0]->reshape(x->dims, NNR_DATA_TYPE_FLOAT32);
    }
    bool exec() override {
        tensor_t* x = inputs[0];
        const long long N = x->dims[0];
        const int C = x->dims[1];
        const long long HW = (long long)(x->ndata / ((size_t)N * C));
        const int nhwc = x->format == memory_layout_t::NHWC;
        if (folded_u8)
            return ok(this, nnrh_batchnorm_u8(x->data, x->type == NNR_DATA_TYPE_FLOAT32, (uint8_t*)outputs[0]->data,
                                              (const float*)inputs[1]->data, (const float*)inputs[2]->data, N, C, HW,
                                              nhwc, ctx->stream));
        return ok(this, nnrh_batchnorm_f32((const float*)x->data, (float*)outputs[0]->data, ab, ab + C, N, C, HW, nhwc,
                                           ctx->stream));
    }
    std::string variant() const override {
        if (!folded_u8) return std::string();
        return inputs[0]->type == NNR_DATA_TYPE_UINT8 ? "DQ-BN-Q" : "BN-Q";
    }
};

// ===========================================================================
// MaxPool (src/backend/cpu/MaxPool.cpp); uint8 NHWC after fuse_qdq
struct MaxPool_hip : operator_t {
    std::vector<int> kernels, pads, strides;
    int auto_pad = 0;
    int cp[4] = {0, 0, 0, 0};
    // after reshape(): the resolved window, strides and pads
    bool pool_params(int* k, int* s, int* p) const override {
        if (kernels.size() != 2 || strides.size() != 2) return false;
        for (int i = 0; i < 2; ++i) { k[i] = kernels[i]; s[i] = strides[i]; }
        for (int i = 0; i < 4; ++i) p[i] = cp[i];
        return true;
    }
    bool init() override {
        for (auto v : attribute_ints("kernel_shape")) kernels.push_back((int)v);
        if (kernels.size() != 2) return false;
        auto p = attribute_ints("pads"), s = attribute_ints("strides"), d = attribute_ints("dilations");
        for (auto v : d)
            if (v != 1) return false;
        if (attribute("ceil_mode", 0) != 0 || outputs.size() != 1) return false;
        std::string ap = attribute_s("auto_pad", "NOTSET");
        auto_pad = ap == "SAME_UPPER" ? 1 : ap == "SAME_LOWER" ? 2 : ap == "VALID" ? 3 : 0;
        pads.assign(4, 0);
        strides.assign(2, 1);
        for (size_t i = 0; i < p.size() && i < 4; ++i) pads[i] = (int)p[i];
        for (size_t i = 0; i < s.size() && i < 2; ++i) strides[i] = (int)s[i];
        return true;
    }
    bool reshape() override {
        tensor_t *x = inputs[0], *y = outputs[0];
        if (x->ndim() != 4) return bad(this, "only 2-D pooling");
        int out[2];
        for (int i = 0; i < 2; ++i) {
            int xd = x->dims[i + 2];
            if (auto_pad == 1 || auto_pad == 2) {
                int pad = (int)(ceilf(xd / (float)strides[i]) - 1) * strides[i] + kernels[i] - xd;
                if (auto_pad == 1) { cp[i] = pad / 2; cp[i + 2] = pad - cp[i]; }
                else { cp[i + 2] = pad / 2; cp[i] = pad - cp[i + 2]; }
                out[i] = (int)ceilf(xd / (float)strides[i]);
            } else if (auto_pad == 3) {
                out[i] = (int)ceilf((xd - kernels[i] + 1) / (float)strides[i]);
            } else {
                cp[i] = pads[i];
                cp[i + 2] = pads[i + 2];
                out[i] = (int)floorf((xd + cp[i] + cp[i + 2] - kernels[i]) / (float)strides[i] + 1);
            }
        }
        layout_mask = x->type == NNR_DATA_TYPE_UINT8 ? (LAYOUT_NCHW | LAYOUT_NHWC) : LAYOUT_NCHW;
        y->format = x->format;
        if (x->is_quantized()) y->set_quant(x->quant_scale, x->quant_zero_point);
        if (!ctx->shape_only && !(x->type == NNR_DATA_TYPE_UINT8 && x->format == memory_layout_t::NHWC))
            return bad(this, "only uint8 NHWC pooling is implemented on the HIP backend");
        return y->reshape({x->dims[0], x->dims[1], out[0], out[1]}, x->type);
    }
    bool exec() override {
        tensor_t *x = inputs[0], *y = outputs[0];
        return ok(this, nnrh_maxpool_u8_nhwc((const uint8_t*)x->data, (uint8_t*)y->data, x->dims[0], x->dims[1],
                                             x->dims[2], x->dims[3], y->dims[2], y->dims[3], kernels[0], kernels[1],
                                             strides[0], strides[1], cp[0], cp[1], ctx->stream));
    }
};

// GlobalAveragePool (src/backend/cpu/global_pool.cpp), fp32
struct GlobalAveragePool_hip : operator_t {
    bool init() override {
        layout_mask = LAYOUT_NCHW | LAYOUT_NHWC;
        return inputs.size() == 1 && outputs.size() == 1;
    }
    bool reshape() override {
        tensor_t *x = inputs[0], *y = outputs[0];
        if (x->ndim() != 4 || x->type != NNR_DATA_TYPE_FLOAT32) return bad(this, "fp32 4-D input");
        return y->reshape({x->dims[0], x->dims[1], 1, 1}, x->type);
    }
    // a per-tensor DequantizeLinear of an 8-bit tensor folded into the pool
    bool fused_dq = false;
    float dq_scale = 1.0f;
    int dq_zp = 0, dq_type = 0;
    bool exec() override {
        tensor_t* x = inputs[0];
        if (fused_dq)
            return ok(this, nnrh_global_avgpool_dequant(x->data, (float*)outputs[0]->data, x->dims[0], x->dims[1],
                                                        x->dims[2] * x->dims[3], x->format == memory_layout_t::NHWC,
                                                        dq_type, dq_scale, dq_zp, ctx->stream));
        return ok(this, nnrh_global_avgpool_f32((const float*)x->data, (float*)outputs[0]->data, x->dims[0],
                                                x->dims[1], x->dims[2] * x->dims[3],
                                                x->format == memory_layout_t::NHWC, ctx->stream));
    }
    bool fuse_dequantize_input(operator_t* dq) override {
        if (dq->inputs.size() < 2 || dq->outputs.empty()) return false;
        tensor_t *x = dq->inputs[0], *s = dq->inputs[1], *z = in(dq, 2);
        if (!x || (x->type != NNR_DATA_TYPE_UINT8 && x->type != NNR_DATA_TYPE_INT8) || x->ndim() != 4) return false;
        if (x->format != dq->outputs[0]->format) return false;
        if (!s->has_host() || s->ndata != 1 || s->type != NNR_DATA_TYPE_FLOAT32) return false;
        if (z && (!z->has_host() || z->ndata != 1 || z->type != x->type)) return false;
        dq_scale = s->scalar_f32();
        dq_zp = zp_value(z);
        dq_type = qdtype(x->type);
        fused_dq = true;
        return true;
    }
    double num_bytes() const override {
        return (double)inputs[0]->nbytes() + (double)outputs[0]->nbytes();
    }
};

// Flatten / Reshape: views of their input (src/backend/cpu/Flatten.cpp, Reshape.cpp)
struct Flatten_hip : operator_t {
    bool init() override { return inputs.size() >= 1 && outputs.size() == 1; }
    int view_input_index() const override { return 0; }
    bool reshape() override {
        tensor_t *x = inputs[0], *y = outputs[0];
        int axis = (int)attribute("axis", 1);
        if (axis < 0) axis += x->ndim();
        if (x->format == memory_layout_t::NHWC && x->ndim() == 4 && x->dims[2] * x->dims[3] > 1)
            return bad(this, "NHWC input with spatial extent > 1");
        int a = 1, b = 1;
        for (int i = 0; i < x->ndim(); ++i) (i < axis ? a : b) *= x->dims[i];
        return y->reshape({a, b}, x->type);
    }
    bool exec() override { return true; }
};

struct Reshape_hip : operator_t {
    bool init() override { return inputs.size() >= 2 && outputs.size() == 1; }
    int view_input_index() const override { return 0; }
    bool reshape() override {
        tensor_t *x = inputs[0], *s = inputs[1], *y = outputs[0];
        if (!s->has_host() || s->type != NNR_DATA_TYPE_INT64) return bad(this, "shape must be a constant int64");
        if (x->format == memory_layout_t::NHWC && x->ndim() == 4 && x->dims[2] * x->dims[3] > 1)
            return bad(this, "NHWC input with spatial extent > 1");
        std::vector<int> d;
        const int64_t* sh = s->h<int64_t>();
        int neg = -1;
        size_t known = 1;
        for (size_t i = 0; i < s->ndata; ++i) {
            int v = (int)sh[i];
            if (v == 0 && i < (size_t)x->ndim()) v = x->dims[i];
            if (v == -1) { neg = (int)i; v = 1; }
            else known *= (size_t)v;
            d.push_back(v);
        }
        if (neg >= 0) d[neg] = known ? (int)(x->ndata / known) : 0;
        return y->reshape(d, x->type);
    }
    bool exec() override { return true; }
};

// Gemm (src/backend/cpu/Gemm.cpp), fp32
struct Gemm_hip : operator_t {
    int M = 0, N = 0, K = 0, c_mode = 0;
    bool init() override { return inputs.size() >= 2 && outputs.size() == 1; }
    bool reshape() override {
        tensor_t *a = inputs[0], *b = inputs[1], *c = in(this, 2), *y = outputs[0];
        if (a->ndim() != 2 || b->ndim() != 2 || a->type != NNR_DATA_TYPE_FLOAT32) return bad(this, "fp32 2-D only");
        int ta = (int)attribute("transA", 0), tb = (int)attribute("transB", 0);
        M = ta ? a->dims[1] : a->dims[0];
        K = ta ? a->dims[0] : a->dims[1];
        N = tb ? b->dims[0] : b->dims[1];
        if ((tb ? b->dims[1] : b->dims[0]) != K) return bad(this, "inner dimensions differ");
        c_mode = 0;
        if (c) {
            if (c->ndata == 1) c_mode = 1;
            else if (c->ndata == (size_t)N && (c->ndim() == 1 || c->dims[0] == 1)) c_mode = 2;
            else if (c->ndata == (size_t)M * N) c_mode = 3;
            else if (c->ndata == (size_t)M) c_mode = 4;
            else return bad(this, "bias shape");
        }
        return y->reshape({M, N}, NNR_DATA_TYPE_FLOAT32);
    }
    bool exec() override {
        tensor_t* c = in(this, 2);
        if (!ok(this, nnrh_gemm_f32((const float*)inputs[0]->data, (const float*)inputs[1]->data,
                                    c ? (const float*)c->data : nullptr, (float*)outputs[0]->data, M, N, K,
                                    (int)attribute("transA", 0), (int)attribute("transB", 0),
                                    attribute_f("alpha", 1.0f), attribute_f("beta", 1.0f), c_mode, ctx->stream)))
            return false;
        // a fused Relu / Clip / HardSwish runs over the whole output (Gemm.cpp:146-151)
        return !(post_fn && fused_op) || fused_op->apply_post(outputs[0]->data, outputs[0]->ndata);
    }
    double num_ops() const override { return 2.0 * M * (double)N * K; }
};

// Relu / Clip, fp32; fusable into a preceding producer (post_fn)
struct Clip_hip : operator_t {
    bool relu = false;
    bool init() override {
        layout_mask = LAYOUT_ALL;
        fusable_unary = true;
        return inputs.size() >= 1 && outputs.size() == 1;
    }
    bool reshape() override {
        if (inputs[0]->type != NNR_DATA_TYPE_FLOAT32 && !ctx->shape_only && !skip)
            return bad(this, "only fp32 (int8 Relu/Clip are fused or absorbed into Q)");
        return operator_t::reshape();
    }
    bool exec() override {
        float lo = relu ? 0.0f : -INFINITY, hi = INFINITY;
        if (!relu) {
            if (in(this, 1) && in(this, 1)->has_host()) lo = in(this, 1)->scalar_f32();
            if (in(this, 2) && in(this, 2)->has_host()) hi = in(this, 2)->scalar_f32();
        }
        return ok(this, nnrh_clip_f32((const float*)inputs[0]->data, (float*)outputs[0]->data, inputs[0]->ndata,
                                      lo, hi, ctx->stream));
    }
    // fused after an fp32 producer: with no bias the reference runs the same
    // clip over the output in place (Relu.cpp:36-70, Clip.cpp:20-57)
    bool apply_post(void* data, size_t n) override {
        float lo = relu ? 0.0f : -INFINITY, hi = INFINITY;
        if (!relu) {
            if (in(this, 1) && in(this, 1)->has_host()) lo = in(this, 1)->scalar_f32();
            if (in(this, 2) && in(this, 2)->has_host()) hi = in(this, 2)->scalar_f32();
        }
        return ok(this, nnrh_clip_f32((const float*)data, (float*)data, n, lo, hi, ctx->stream));
    }
};

// HardSwish (src/backend/cpu/HardSwish.cpp:18-50), fp32. Not quant-capable
// (fuse_qdq.cpp:96-100), so DQ -> HardSwish -> Q runs it on fp32 tensors;
// fusable into a preceding producer like Relu / Clip (on QLinearConv the
// fusion only sets qmin, QLinearConv.cpp:419).
struct HardSwish_hip : operator_t {
    bool init() override {
        layout_mask = LAYOUT_ALL;
        fusable_unary = true;
        return inputs.size() == 1 && outputs.size() == 1;
    }
    bool reshape() override {
        if (inputs[0]->type != NNR_DATA_TYPE_FLOAT32 && !ctx->shape_only && !skip)
            return bad(this, "fp32 only (a fused HardSwish on QLinearConv only raises qmin)");
        return operator_t::reshape();
    }
    bool exec() override {
        return ok(this, nnrh_hardswish_f32((const float*)inputs[0]->data, (float*)outputs[0]->data,
                                           inputs[0]->ndata, 0, ctx->stream));
    }
    // bias_hardswish with a zero bias over the producer's output as one row
    // (Gemm.cpp:146-151, vec_ops_avx512.h:74-94)
    bool apply_post(void* data, size_t n) override {
        return ok(this, nnrh_hardswish_f32((const float*)data, (float*)data, n, 1, ctx->stream));
    }
};

// ===========================================================================
// fp32 glue of the transformer encoder

// Add / Mul / Sub / Div (src/backend/cpu/binary_math.cpp) with the broadcasts
// the graphs use: same shape, a scalar operand, or a vector over the last axis
struct Binary_hip : operator_t {
    int op = 0;   // 0 add, 1 mul, 2 sub, 3 div
    int b_mode = 0, D = 1;
    bool swap = false;
    bool init() override { return inputs.size() == 2 && outputs.size() == 1; }
    static bool is_last_axis_vector(const tensor_t* v, const tensor_t* full) {
        if (full->ndim() < 1 || v->ndata != (size_t)full->dims.back()) return false;
        for (int i = 0; i + 1 < v->ndim(); ++i)
            if (v->dims[i] != 1) return false;
        return v->ndim() >= 1 && v->dims.back() == full->dims.back();
    }
    bool reshape() override {
        tensor_t *a = inputs[0], *b = inputs[1], *y = outputs[0];
        if (a->type != NNR_DATA_TYPE_FLOAT32 || b->type != NNR_DATA_TYPE_FLOAT32)
            return bad(this, "fp32 only (int8 additions are fused to QLinearAdd)");
        swap = a->ndata < b->ndata;
        const tensor_t* full = swap ? b : a;
        const tensor_t* other = swap ? a : b;
        if (full->dims == other->dims) b_mode = 0;
        else if (other->ndata == 1) b_mode = 1;
        else if (is_last_axis_vector(other, full)) { b_mode = 2; D = full->dims.back(); }
        else return bad(this, "unsupported broadcast");
        return y->reshape(full->dims, NNR_DATA_TYPE_FLOAT32);
    }
    bool exec() override {
        tensor_t *a = inputs[0], *b = inputs[1];
        const float* full = (const float*)(swap ? b : a)->data;
        const float* other = (const float*)(swap ? a : b)->data;
        return ok(this, nnrh_binary_f32(op, full, other, (float*)outputs[0]->data, outputs[0]->ndata, D, b_mode,
                                        swap ? 1 : 0, ctx->stream));
    }
};
template <int OP>
operator_t* make_binary(int, pool_t& pool) {
    auto* b = pool_new<Binary_hip>(pool);
    b->op = OP;
    return b;
}

// Softmax over the last axis (src/backend/cpu/Softmax.cpp, opset 13)
struct Softmax_hip : operator_t {
    bool init() override { return inputs.size() == 1 && outputs.size() == 1; }
    bool reshape() override {
        tensor_t* x = inputs[0];
        int axis = (int)attribute("axis", -1);
        if (axis < 0) axis += x->ndim();
        if (axis != x->ndim() - 1 || x->type != NNR_DATA_TYPE_FLOAT32)
            return bad(this, "fp32 softmax over the last axis only");
        return outputs[0]->reshape(x->dims, x->type);
    }
    bool exec() override {
        tensor_t* x = inputs[0];
        const int D = x->dims.back();
        return ok(this, nnrh_softmax_f32((const float*)x->data, (float*)outputs[0]->data, x->ndata / D, D,
                                         ctx->stream));
    }
};

// com.microsoft MultiHeadAttention (src/backend/cpu/MultiHeadAttention.cpp)
// on fp32 [B][S][hidden] q, k, v without masks; created by fuse_attention
struct MultiHeadAttention_hip : operator_t {
    int num_heads = 0;
    float scale = 0.0f;
    size_t ws_need = 0;   // score matrix of the general path; 0 on the fused head-64 path
    bool init() override {
        num_heads = (int)attribute("num_heads", 0);
        scale = attribute_f("scale", 0.0f);
        return inputs.size() >= 3 && outputs.size() == 1 && num_heads > 0;
    }
    bool reshape() override {
        tensor_t *q = inputs[0], *k = inputs[1], *v = inputs[2];
        if (q->ndim() != 3 || q->type != NNR_DATA_TYPE_FLOAT32 || k->dims != q->dims || v->dims != q->dims ||
            k->type != q->type || v->type != q->type)
            return bad(this, "q, k, v must be fp32 [B][S][hidden] of one shape");
        for (size_t i = 3; i < inputs.size(); ++i)
            if (inputs[i] && inputs[i]->ndata) return bad(this, "bias / masks / past state are not supported");
        if (q->dims[2] % num_heads) return bad(this, "hidden not divisible by num_heads");
        if (!ok(this, nnrh_multihead_attention_workspace(q->dims[0], q->dims[1], q->dims[2], num_heads, &ws_need)))
            return false;
        return outputs[0]->reshape(q->dims, q->type);
    }
    size_t workspace_size() const override { return ws_need; }
    // one (min, max) pair per wave of the fused head-64 kernel, for the
    // DynamicQuantizeLinear of the output projection's input
    int minmax_pairs() const override {
        const tensor_t* q = inputs[0];
        int c = 0;
        if (q->ndim() != 3 ||
            nnrh_multihead_attention_minmax_count(q->dims[0], q->dims[1], q->dims[2], num_heads, &c) != NNRH_OK)
            return 0;
        return c;
    }
    bool set_minmax_out(float*, int) override { return true; }
    // q, k, v as chain bytes (fuse_codes_readers): the fused head-64 kernel's
    // shapes only (those with (min, max) pairs); used when all three are set
    nnrh_dq_codes cq[3] = {};
    int ncodes = 0;
    bool set_codes_input(int which, operator_t* p) override {
        if (which < 0 || which > 2) return false;
        if (!p) {
            if (cq[which].bias_dev) --ncodes;
            cq[which] = nnrh_dq_codes{};
            return true;
        }
        int zp = 0;
        float sc = 0.0f;
        const float* b = nullptr;
        if (cq[which].bias_dev || minmax_pairs() <= 0 || !p->codes_params(&zp, &sc, &b)) return false;
        cq[which] = nnrh_dq_codes{nullptr, zp, sc, b};
        ++ncodes;
        return true;
    }
    std::string variant() const override { return ncodes == 3 ? "Codes" : ""; }
    bool exec() override {
        tensor_t* q = inputs[0];
        const int B = q->dims[0], S = q->dims[1], Hd = q->dims[2];
        // contrib op default: 1 / sqrt(head_dim)
        const float sc = scale != 0.0f ? scale : 1.0f / sqrtf((float)(Hd / num_heads));
        if (ncodes == 3) {
            nnrh_dq_codes c[3];
            for (int i = 0; i < 3; ++i) {
                c[i] = cq[i];
                c[i].codes_dev = (const uint8_t*)inputs[i]->data;
            }
            return ok(this, nnrh_multihead_attention_codes_f32(&c[0], &c[1], &c[2], (float*)outputs[0]->data, B, S,
                                                               Hd, num_heads, sc, minmax_parts, ctx->stream));
        }
        return ok(this, nnrh_multihead_attention_f32((const float*)q->data, (const float*)inputs[1]->data,
                                                     (const float*)inputs[2]->data, (float*)outputs[0]->data, B, S,
                                                     Hd, num_heads, sc, minmax_parts, ctx->workspace, ctx->stream));
    }
    double num_ops() const override {
        const tensor_t* q = inputs[0];
        return 4.0 * q->dims[0] * (double)q->dims[1] * q->dims[1] * q->dims[2];
    }
};

// LayerNormalization over the last axis (src/backend/cpu/LayerNormalization.cpp)
struct LayerNormalization_hip : operator_t {
    bool init() override { return inputs.size() >= 2 && inputs.size() <= 3 && outputs.size() >= 1; }
    bool reshape() override {
        tensor_t* x = inputs[0];
        int axis = (int)attribute("axis", -1);
        if (axis < 0) axis += x->ndim();
        if (axis != x->ndim() - 1 || x->type != NNR_DATA_TYPE_FLOAT32)
            return bad(this, "fp32 layer norm over the last axis only");
        if (outputs.size() > 1 && (outputs[1] || (outputs.size() > 2 && outputs[2])))
            return bad(this, "Mean / InvStdDev outputs are not produced");
        if (inputs[1]->ndata != (size_t)x->dims.back()) return bad(this, "scale shape");
        return outputs[0]->reshape(x->dims, x->type);
    }
    bool fuse_residual_input(operator_t* add) override {
        return add->outputs[0] == inputs[0] && !fused_other;
    }
    // one pair per 4 rows
    int minmax_pairs() const override {
        const tensor_t* x = inputs[0];
        const size_t groups = (x->ndata / (size_t)x->dims.back() + 3) / 4;
        return groups <= 0x7fffffff ? (int)groups : 0;
    }
    bool set_minmax_out(float*, int) override { return true; }
    // one operand as chain bytes (fuse_codes_readers): 0 the normalized
    // input, 1 the residual Add's other operand
    int codes_which = -1;
    nnrh_dq_codes cq{};
    bool set_codes_input(int which, operator_t* p) override {
        if (!p) {
            codes_src = nullptr;
            codes_which = -1;
            return true;
        }
        int zp = 0;
        float sc = 0.0f;
        const float* b = nullptr;
        if (codes_src || which < 0 || which > 1 || (which == 1 && !fused_other) || !p->codes_params(&zp, &sc, &b))
            return false;
        cq = nnrh_dq_codes{nullptr, zp, sc, b};
        codes_src = p;
        codes_which = which;
        return true;
    }
    std::string variant() const override {
        return std::string(fused_other ? "+Add" : "") + (codes_src ? (fused_other ? "+Codes" : "Codes") : "");
    }
    bool exec() override {
        tensor_t* x = inputs[0];
        tensor_t* bias = in(this, 2);
        const int D = x->dims.back();
        if (codes_src) {
            // the sum fl(a + b) is the same either way round
            tensor_t* ct = codes_which == 0 ? x : fused_other;
            tensor_t* other = codes_which == 0 ? fused_other : x;
            nnrh_dq_codes c = cq;
            c.codes_dev = (const uint8_t*)ct->data;
            return ok(this, nnrh_add_layernorm_codes_f32(&c, other ? (const float*)other->data : nullptr,
                                                         (const float*)inputs[1]->data,
                                                         bias ? (const float*)bias->data : nullptr,
                                                         (float*)outputs[0]->data, ct->ndata / D, D,
                                                         attribute_f("epsilon", 1e-5f), minmax_parts, ctx->stream));
        }
        return ok(this, nnrh_add_layernorm_f32((const float*)x->data,
                                               fused_other ? (const float*)fused_other->data : nullptr,
                                               (const float*)inputs[1]->data,
                                               bias ? (const float*)bias->data : nullptr,
                                               (float*)outputs[0]->data, x->ndata / D, D,
                                               attribute_f("epsilon", 1e-5f), minmax_parts, ctx->stream));
    }
};

// Gelu (src/backend/cpu/Gelu.cpp), approximate = "none"
struct Gelu_hip : operator_t {
    bool init() override { return inputs.size() == 1 && outputs.size() == 1; }
    bool reshape() override {
        if (attribute_s("approximate", "none") != "none") return bad(this, "tanh approximation");
        if (inputs[0]->type != NNR_DATA_TYPE_FLOAT32) return bad(this, "fp32 only");
        return operator_t::reshape();
    }
    bool exec() override {
        return ok(this, nnrh_gelu_f32((const float*)inputs[0]->data, (float*)outputs[0]->data, inputs[0]->ndata,
                                      ctx->stream));
    }
};

// Transpose (src/backend/cpu/Transpose.cpp), fp32, up to 6 axes
struct Transpose_hip : operator_t {
    std::vector<int> perm;
    bool init() override { return inputs.size() == 1 && outputs.size() == 1; }
    bool reshape() override {
        tensor_t* x = inputs[0];
        if (x->type != NNR_DATA_TYPE_FLOAT32 || x->ndim() > 6) return bad(this, "fp32, <= 6 axes");
        perm.clear();
        for (auto v : attribute_ints("perm")) perm.push_back((int)v);
        if (perm.empty())
            for (int i = x->ndim() - 1; i >= 0; --i) perm.push_back(i);
        if ((int)perm.size() != x->ndim()) return bad(this, "perm length");
        std::vector<int> d;
        for (int p : perm) {
            if (p < 0 || p >= x->ndim()) return bad(this, "perm value");
            d.push_back(x->dims[p]);
        }
        return outputs[0]->reshape(d, x->type);
    }
    bool exec() override {
        tensor_t* x = inputs[0];
        return ok(this, nnrh_transpose_f32((const float*)x->data, (float*)outputs[0]->data, x->ndim(),
                                           x->dims.data(), perm.data(), ctx->stream));
    }
};

// MatMul (src/backend/cpu/MatMul.cpp), fp32: [..., M, K] x [..., K, N] with
// equal leading axes, or a 2-D right operand shared by every batch
struct MatMul_hip : operator_t {
    int M = 0, N = 0, K = 0, batch = 1;
    bool b_shared = false;
    bool init() override { return inputs.size() == 2 && outputs.size() == 1; }
    bool reshape() override {
        tensor_t *a = inputs[0], *b = inputs[1];
        if (a->type != NNR_DATA_TYPE_FLOAT32 || b->type != NNR_DATA_TYPE_FLOAT32)
            return bad(this, "fp32 only (int8 MatMul is fused to QLinearMatMul)");
        if (a->ndim() < 2 || b->ndim() < 2) return bad(this, "operands must have >= 2 axes");
        M = a->dims[a->ndim() - 2];
        K = a->dims[a->ndim() - 1];
        N = b->dims[b->ndim() - 1];
        if (b->dims[b->ndim() - 2] != K) return bad(this, "inner dimensions differ");
        batch = 1;
        for (int i = 0; i + 2 < a->ndim(); ++i) batch *= a->dims[i];
        b_shared = b->ndim() == 2;
        if (!b_shared) {
            if (b->ndim() != a->ndim()) return bad(this, "batch broadcast");
            for (int i = 0; i + 2 < a->ndim(); ++i)
                if (a->dims[i] != b->dims[i]) return bad(this, "batch broadcast");
        }
        std::vector<int> d(a->dims.begin(), a->dims.end() - 1);
        d.push_back(N);
        return outputs[0]->reshape(d, NNR_DATA_TYPE_FLOAT32);
    }
    bool exec() override {
        if (!ok(this, nnrh_gemm_f32_batched((const float*)inputs[0]->data, (const float*)inputs[1]->data, nullptr,
                                            (float*)outputs[0]->data, M, N, K, 0, 0, 1.0f, 0.0f, 0, batch,
                                            (long long)M * K, b_shared ? 0 : (long long)K * N,
                                            (long long)M * N, ctx->stream)))
            return false;
        // a fused Relu / Clip (position-free; a HardSwish is not fused here)
        return !(post_fn && fused_op) || fused_op->apply_post(outputs[0]->data, outputs[0]->ndata);
    }
    double num_ops() const override { return 2.0 * batch * M * (double)N * K; }
};

template <typename T>
operator_t* make(int, pool_t& pool) { return pool_new<T>(pool); }
operator_t* make_relu(int, pool_t& pool) {
    auto* c = pool_new<Clip_hip>(pool);
    c->relu = true;
    return c;
}

const op_registrar_t reg[] = {
    {"QuantizeLinear", backend_t::HIP, make<QuantizeLinear_hip>},
    {"DequantizeLinear", backend_t::HIP, make<DequantizeLinear_hip>},
    {"DynamicQuantizeLinear", backend_t::HIP, make<DynamicQuantizeLinear_hip>},
    {"QLinearConv", backend_t::HIP, make<QLinearConv_hip>},
    {"QLinearMatMul", backend_t::HIP, make<QLinearMatMul_hip>},
    {"MatMulInteger", backend_t::HIP, make<MatMulInteger_hip>},
    {"Cast", backend_t::HIP, make<Cast_hip>},
    {"QLinearAdd", backend_t::HIP, make<QLinearAdd_hip>},
    {"QLinearMul", backend_t::HIP, make<QLinearMul_hip>},
    {"QLinearGlobalAveragePool", backend_t::HIP, make<QLinearGlobalAveragePool_hip>},
    {"QLinearAveragePool", backend_t::HIP, make<QLinearAveragePool_hip>},
    {"QLinearConcat", backend_t::HIP, make<QLinearConcat_hip>},
    {"MaxPool", backend_t::HIP, make<MaxPool_hip>},
    {"BatchNormalization", backend_t::HIP, make<BatchNormalization_hip>},
    {"ConvInteger", backend_t::HIP, make<ConvInteger_hip>},
    {"GlobalAveragePool", backend_t::HIP, make<GlobalAveragePool_hip>},
    {"Flatten", backend_t::HIP, make<Flatten_hip>},
    {"Reshape", backend_t::HIP, make<Reshape_hip>},
    {"Gemm", backend_t::HIP, make<Gemm_hip>},
    {"Relu", backend_t::HIP, make_relu},
    {"Clip", backend_t::HIP, make<Clip_hip>},
    {"HardSwish", backend_t::HIP, make<HardSwish_hip>},
    {"Add", backend_t::HIP, make_binary<0>},
    {"Mul", backend_t::HIP, make_binary<1>},
    {"Sub", backend_t::HIP, make_binary<2>},
    {"Div", backend_t::HIP, make_binary<3>},
    {"Softmax", backend_t::HIP, make<Softmax_hip>},
    {"MultiHeadAttention", backend_t::HIP, make<MultiHeadAttention_hip>},
    {"LayerNormalization", backend_t::HIP, make<LayerNormalization_hip>},
    {"Gelu", backend_t::HIP, make<Gelu_hip>},
    {"Transpose", backend_t::HIP, make<Transpose_hip>},
    {"MatMul", backend_t::HIP, make<MatMul_hip>},
};

}  // namespace

// referenced by the host C ABI so the registrations above are linked in
int hip_backend_op_count() { return (int)(sizeof(reg) / sizeof(reg[0])); }

}  // namespace nnr
