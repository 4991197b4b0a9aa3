"""Synthetic int8 QDQ graphs of the benchmark configurations.

Each builder returns a `Graph` in the QDQ form the reference fuses
(fuse_qdq_compute.cpp:100-207): DequantizeLinear -> Conv / MatMul ->
QuantizeLinear, with Relu absorbed into the output quantization (zero point
0; NNR does not fuse DQ->Conv->Relu->Q, fuse_qdq_compute.cpp:128-134), and
residual additions as DQ + DQ -> Add -> Relu -> Q (fused to QLinearAdd,
fuse_qdq_compute.cpp:209-345). Weights are random-init, quantized per output
channel to int8 (symmetric, zero point 0); activation scales are drawn from
[0.01, 0.05] with a seeded generator, so every run rebuilds the same graph.
"""
from __future__ import annotations

import numpy as np

from .graph import Graph

F32 = np.float32


class _QDQ:
    """Helper emitting QDQ patterns into a Graph."""

    def __init__(self, g: Graph, rng):
        self.g = g
        self.rng = rng
        self.n = 0

    def uid(self, p):
        self.n += 1
        return f"{p}{self.n}"

    def scale(self):
        return F32(self.rng.uniform(0.01, 0.05))

    def qparams(self, s, zp, dt=np.uint8):
        n = self.uid("q")
        return (self.g.init(n + "_s", np.array(s, F32)),
                self.g.init(n + "_z", np.array(zp, dt)))

    def quant(self, x_f, s, zp, name=None):
        sn, zn = self.qparams(s, zp)
        return self.g.node("QuantizeLinear", [x_f, sn, zn], name=name or self.uid("Q")), (s, zp)

    def dequant(self, x_q, qp, name=None):
        s, zp = qp
        sn, zn = self.qparams(s, zp)
        return self.g.node("DequantizeLinear", [x_q, sn, zn], name=name or self.uid("DQ"))

    def conv(self, x_q, x_qp, cin, cout, k, stride=1, pad=0, relu=True, name=None, group=1,
             y_scale=None, y_zp=None):
        """DQ(x) -> Conv(DQ(w), DQ(b)) -> Q(y); returns (y_q, y_qp)."""
        g, rng = self.g, self.rng
        name = name or self.uid("conv")
        fan_in = cin // group * k * k
        w = rng.normal(0.0, np.sqrt(2.0 / fan_in), (cout, cin // group, k, k)).astype(F32)
        ws = (np.abs(w).reshape(cout, -1).max(1) / 127.0).astype(F32)
        ws = np.maximum(ws, F32(1e-8))
        wq = np.clip(np.rint(w / ws[:, None, None, None]), -127, 127).astype(np.int8)
        bias_f = rng.normal(0.0, 0.1, cout).astype(F32)
        bs = (F32(x_qp[0]) * ws).astype(F32)
        bq = np.rint(bias_f / bs).astype(np.int32)
        wn = g.init(name + "_w", wq)
        wsn = g.init(name + "_ws", ws)
        wzn = g.init(name + "_wz", np.zeros(cout, np.int8))
        bn = g.init(name + "_b", bq)
        bsn = g.init(name + "_bs", bs)
        bzn = g.init(name + "_bz", np.zeros(cout, np.int32))
        w_f = g.node("DequantizeLinear", [wn, wsn, wzn], name=name + "_wdq", axis=0)
        b_f = g.node("DequantizeLinear", [bn, bsn, bzn], name=name + "_bdq", axis=0)
        x_f = self.dequant(x_q, x_qp)
        y_f = g.node("Conv", [x_f, w_f, b_f], name=name, kernel_shape=[k, k],
                     strides=[stride, stride], pads=[pad, pad, pad, pad], group=group,
                     dilations=[1, 1])
        ys = self.scale() if y_scale is None else F32(y_scale)
        yz = (0 if relu else 128) if y_zp is None else y_zp
        return self.quant(y_f, ys, yz)


def resnet50(batch=256, hw=224, seed=3, num_classes=1000):
    """ResNet-50 v1.5 int8 QDQ: stem 7x7/2 + maxpool, bottleneck stages
    [3,4,6,3] widths 64/128/256/512 (x4 expansion, stride on the 3x3),
    fp32 GlobalAveragePool + Gemm head."""
    g = Graph()
    rng = np.random.default_rng(seed)
    q = _QDQ(g, rng)
    g.inputs["input"] = (np.float32, (batch, 3, hw, hw))
    x_q, x_qp = q.quant("input", F32(1.0 / 255.0), 0, name="input_Q")
    y_q, y_qp = q.conv(x_q, x_qp, 3, 64, 7, stride=2, pad=3, name="stem")
    # maxpool in the quantized domain: DQ -> MaxPool -> Q (same scale)
    mp_f = g.node("MaxPool", [q.dequant(y_q, y_qp)], name="maxpool", kernel_shape=[3, 3],
                  strides=[2, 2], pads=[1, 1, 1, 1])
    x_q, x_qp = q.quant(mp_f, *y_qp)
    cin = 64
    for si, (width, blocks) in enumerate(zip((64, 128, 256, 512), (3, 4, 6, 3))):
        for bi in range(blocks):
            stride = 2 if (bi == 0 and si > 0) else 1
            nm = f"s{si + 1}b{bi + 1}"
            a, a_qp = q.conv(x_q, x_qp, cin, width, 1, name=nm + "_c1")
            a, a_qp = q.conv(a, a_qp, width, width, 3, stride=stride, pad=1, name=nm + "_c2")
            a, a_qp = q.conv(a, a_qp, width, width * 4, 1, relu=False, name=nm + "_c3")
            if bi == 0:
                sc, sc_qp = q.conv(x_q, x_qp, cin, width * 4, 1, stride=stride, relu=False,
                                   name=nm + "_ds")
            else:
                sc, sc_qp = x_q, x_qp
            s = g.node("Add", [q.dequant(a, a_qp), q.dequant(sc, sc_qp)], name=nm + "_add")
            r = g.node("Relu", [s], name=nm + "_relu")
            x_q, x_qp = q.quant(r, q.scale(), 0)
            cin = width * 4
    # head: DQ -> GAP -> Flatten -> Gemm (fp32)
    f = q.dequant(x_q, x_qp, name="head_dq")
    p = g.node("GlobalAveragePool", [f], name="gap")
    fl = g.node("Flatten", [p], name="flatten", axis=1)
    fw = g.init("fc_w", rng.normal(0.0, np.sqrt(1.0 / cin), (num_classes, cin)).astype(F32))
    fb = g.init("fc_b", rng.normal(0.0, 0.01, num_classes).astype(F32))
    g.node("Gemm", [fl, fw, fb], outputs="logits", name="fc", transB=1)
    g.outputs.append("logits")
    return g


def resnet50_conv_ops(hw=224):
    """Algorithmic int8 ops per image of the ResNet-50 convolutions."""
    ops = 0.0
    s = hw // 2
    ops += 2 * 64 * s * s * 3 * 49
    s //= 2
    cin = 64
    for si, (w, blocks) in enumerate(zip((64, 128, 256, 512), (3, 4, 6, 3))):
        for bi in range(blocks):
            stride = 2 if (bi == 0 and si > 0) else 1
            so = s // stride
            ops += 2 * w * s * s * cin              # c1 at input resolution
            ops += 2 * w * so * so * w * 9          # c2
            ops += 2 * 4 * w * so * so * w          # c3
            if bi == 0:
                ops += 2 * 4 * w * so * so * cin    # downsample
            s = so
            cin = 4 * w
    return ops


def qconv_graph(batch=32, seed=2):
    """cfg2 as a graph: Q(input) -> DQ -> Conv 3x3 -> Q (Relu absorbed)."""
    g = Graph()
    rng = np.random.default_rng(seed)
    q = _QDQ(g, rng)
    g.inputs["input"] = (np.float32, (batch, 64, 56, 56))
    x_q, x_qp = q.quant("input", F32(0.02), 128, name="input_Q")
    y, _ = q.conv(x_q, x_qp, 64, 64, 3, pad=1, name="conv", y_scale=0.03, y_zp=0)
    g.outputs.append(y)
    return g


def qconv1d_graph(batch=4, C=16, W=50, OC=24, k=5, stride=1, pad=2, dil=1, group=1, seed=21):
    """A 1-D convolution in QDQ form on 3-D tensors: Q(input [N][C][W]) ->
    DQ -> Conv(kernel k) -> Q. NNR runs the fused QLinearConv through its
    exec_typed path (QLinearConv.cpp:286-334)."""
    g = Graph()
    rng = np.random.default_rng(seed)
    q = _QDQ(g, rng)
    g.inputs["input"] = (np.float32, (batch, C, W))
    x_q, x_qp = q.quant("input", F32(0.021), 120, name="input_Q")
    w = rng.normal(0.0, 0.3, (OC, C // group, k)).astype(F32)
    ws = np.maximum((np.abs(w).reshape(OC, -1).max(1) / 127.0).astype(F32), F32(1e-8))
    wq = np.clip(np.rint(w / ws[:, None, None]), -127, 127).astype(np.int8)
    bs = (F32(x_qp[0]) * ws).astype(F32)
    bq = rng.integers(-3000, 3000, OC).astype(np.int32)
    w_f = g.node("DequantizeLinear", [g.init("c1_w", wq), g.init("c1_ws", ws),
                                       g.init("c1_wz", np.zeros(OC, np.int8))], name="c1_wdq", axis=0)
    b_f = g.node("DequantizeLinear", [g.init("c1_b", bq), g.init("c1_bs", bs),
                                       g.init("c1_bz", np.zeros(OC, np.int32))], name="c1_bdq", axis=0)
    y_f = g.node("Conv", [q.dequant(x_q, x_qp), w_f, b_f], name="conv1d", kernel_shape=[k],
                 strides=[stride], pads=[pad, pad], dilations=[dil], group=group)
    y, _ = q.quant(y_f, F32(0.05), 7, name="out_Q")
    g.outputs.append(y)
    return g


def qoperator_net(batch=2, hw=20, seed=22, pool="avg"):
    """A QOperator-format graph (quantized operators, not QDQ pairs) using the
    rest of the QLinear family: Q(input) -> QLinearConv 3x3 (16) ->
    QLinearAveragePool -> two QLinearConv branches (1x1 -> 24, 3x3 -> 8) ->
    QLinearConcat along channels (the second branch already in the output's
    quantization, so it is copied) -> QLinearMul by a per-channel constant ->
    QLinearMul of the tensor with itself -> QLinearGlobalAveragePool ->
    DQ. The convolution outputs run NHWC; the pooled, concatenated and
    multiplied tensors follow them."""
    g = Graph()
    rng = np.random.default_rng(seed)
    u8, s8 = np.uint8, np.int8
    g.inputs["input"] = (np.float32, (batch, 3, hw, hw))

    def qp(name, s, z, dt=u8):
        return g.init(name + "_s", np.array(s, F32)), g.init(name + "_z", np.array(z, dt))

    def qconv(x, x_qp, cin, cout, k, pad, name, y_qp):
        w = rng.integers(-90, 91, (cout, cin, k, k), dtype=s8)
        ws = rng.uniform(0.002, 0.01, cout).astype(F32)
        b = rng.integers(-2000, 2000, cout).astype(np.int32)
        ins = [x, x_qp[0], x_qp[1], g.init(name + "_w", w), g.init(name + "_ws", ws),
               g.init(name + "_wz", np.zeros(cout, s8)), y_qp[0], y_qp[1], g.init(name + "_b", b)]
        return g.node("QLinearConv", ins, name=name, kernel_shape=[k, k], pads=[pad] * 4, strides=[1, 1])

    xq_qp = qp("xq", 0.02, 120)
    x = g.node("QuantizeLinear", ["input", *xq_qp], name="input_Q")
    c1_qp = qp("c1", 0.03, 5)
    c1 = qconv(x, xq_qp, 3, 16, 3, 1, "c1", c1_qp)
    p_qp = qp("pool", 0.027, 9)
    if pool == "avg":
        pl = g.node("QLinearAveragePool", [c1, *c1_qp, *p_qp], name="avgpool", kernel_shape=[3, 3],
                    strides=[2, 2], pads=[1, 1, 1, 1])
    else:
        pl = g.node("QLinearAveragePool", [c1, *c1_qp, *p_qp], name="avgpool", kernel_shape=[2, 2],
                    strides=[2, 2], ceil_mode=1)
    ba_qp = qp("ba", 0.041, 12)
    cat_qp = qp("cat", 0.036, 10)
    ba = qconv(pl, p_qp, 16, 24, 1, 0, "ba", ba_qp)
    bb = qconv(pl, p_qp, 16, 8, 3, 1, "bb", cat_qp)   # already in the concat's quantization
    cat = g.node("QLinearConcat", [*cat_qp, ba, *ba_qp, bb, *cat_qp], name="concat", axis=1)
    ch = g.init("mul_ch", rng.integers(100, 200, 32, dtype=u8))
    ch_qp = qp("mul_chq", 0.011, 128)
    m1_qp = qp("m1", 0.025, 3)
    m1 = g.node("QLinearMul", [cat, *cat_qp, ch, *ch_qp, *m1_qp], name="mul_channel")
    m2_qp = qp("m2", 0.02, 0)
    m2 = g.node("QLinearMul", [m1, *m1_qp, m1, *m1_qp, *m2_qp], name="mul_square")
    gp_qp = qp("gap", 0.01, 2)
    gp = g.node("QLinearGlobalAveragePool", [m2, *m2_qp, *gp_qp], name="gap")
    y = g.node("DequantizeLinear", [gp, *gp_qp], name="out_DQ")
    g.outputs.append(y)
    return g


def concat_net(batch=1, C=16, hw=8, seed=25):
    """Q(input) -> QLinearMul by a scalar (the input stays live) and
    QLinearAveragePool 3x3/1 pad 1, both already in the quantization of the
    QLinearConcat that joins them along channels -> QLinearAdd of the
    concatenation with itself -> QLinearGlobalAveragePool -> DQ. At batch 1
    the concatenation's parts can live inside its output (the memory
    planner's concat aliasing) and the add can write over its input."""
    g = Graph()
    rng = np.random.default_rng(seed)
    u8 = np.uint8
    g.inputs["input"] = (np.float32, (batch, C, hw, hw))

    def qp(name, s, z):
        return g.init(name + "_s", np.array(s, F32)), g.init(name + "_z", np.array(z, u8))

    x_qp = qp("x", 0.02, 100)
    x = g.node("QuantizeLinear", ["input", *x_qp], name="input_Q")
    cat_qp = qp("cat", 0.03, 20)
    k = g.init("k", np.array([int(rng.integers(150, 200))], u8))
    kq = qp("kq", 0.01, 128)
    b = g.node("QLinearMul", [x, *x_qp, k, *kq, *cat_qp], name="mul")
    a = g.node("QLinearAveragePool", [x, *x_qp, *cat_qp], name="avgpool", kernel_shape=[3, 3],
               strides=[1, 1], pads=[1, 1, 1, 1])
    cat = g.node("QLinearConcat", [*cat_qp, a, *cat_qp, b, *cat_qp], name="concat", axis=1)
    add_qp = qp("add", 0.05, 10)
    s2 = g.node("QLinearAdd", [cat, *cat_qp, cat, *cat_qp, *add_qp], name="add_self")
    gap_qp = qp("gap", 0.04, 3)
    gp = g.node("QLinearGlobalAveragePool", [s2, *add_qp, *gap_qp], name="gap")
    y = g.node("DequantizeLinear", [gp, *gap_qp], name="out_DQ")
    g.outputs.append(y)
    return g


def bn_net(batch=2, C=40, hw=13, seed=26):
    """BatchNormalization kept after quantization, both forms fold_bn_qdq
    folds: Q(input) -> QLinearConv 3x3 (NHWC uint8) -> DQ -> BN -> Q -> DQ
    (output "bn_a"), and the fp32 input -> BN -> Q -> DQ (output "bn_b",
    NCHW). C = 40 gives the NHWC kernel a 32-channel body and an 8-channel
    tail, hw = 13 a 160-element NCHW body and a 9-element tail; offsets and
    zero points put some results below zero."""
    g = Graph()
    rng = np.random.default_rng(seed)
    q = _QDQ(g, rng)
    g.inputs["input"] = (np.float32, (batch, C, hw, hw))

    def bn(x, name):
        p = [rng.uniform(0.5, 1.5, C), rng.normal(0.0, 0.6, C), rng.normal(0.0, 0.4, C), rng.uniform(0.3, 2.0, C)]
        ins = [x] + [g.init(f"{name}_{k}", v.astype(F32)) for k, v in zip(("scale", "bias", "mean", "var"), p)]
        return g.node("BatchNormalization", ins, name=name, epsilon=1e-3)

    x_q, x_qp = q.quant("input", F32(0.02), 128, name="input_Q")
    c, c_qp = q.conv(x_q, x_qp, C, C, 3, pad=1, name="conv", y_scale=0.05, y_zp=100)
    a = bn(q.dequant(c, c_qp, name="bn_a_dq"), "bn_a")
    a_q, a_qp = q.quant(a, F32(0.04), 6, name="bn_a_q")
    g.outputs.append(q.dequant(a_q, a_qp, name="out_a"))
    b = bn("input", "bn_b")
    b_q, b_qp = q.quant(b, F32(0.03), 4, name="bn_b_q")
    g.outputs.append(q.dequant(b_q, b_qp, name="out_b"))
    return g


def conv_integer_net(batch=2, C=16, hw=15, OC=24, k=3, seed=28, per_channel=True, auto_pad="NOTSET",
                     strides=(1, 1), pads=(1, 1, 1, 1), group=1, x_dtype=np.uint8):
    """Q(input) -> ConvInteger(x, w, x_zp, w_zp) -> int32 output (the form
    dynamically quantized convolutions take)."""
    g = Graph()
    rng = np.random.default_rng(seed)
    g.inputs["input"] = (np.float32, (batch, C, hw, hw))
    zdt = x_dtype
    x_zp = np.array(120 if x_dtype == np.uint8 else -5, zdt)
    xq = g.node("QuantizeLinear", ["input", g.init("xs", np.array(0.02, F32)), g.init("xz", x_zp)], name="input_Q")
    w = rng.integers(-128, 128, (OC, C // group, k, k), dtype=np.int8)
    wz = rng.integers(-20, 20, OC).astype(np.int8) if per_channel else np.array(3, np.int8)
    attrs = dict(auto_pad=auto_pad, strides=list(strides), group=group)
    if auto_pad == "NOTSET":
        attrs["pads"] = list(pads)
    y = g.node("ConvInteger", [xq, g.init("w", w), "xz", g.init("wz", wz)], name="convint", **attrs)
    g.outputs.append(y)
    return g


# MobileNetV2 (Sandler et al. 2018, width 1.0): (expansion t, channels c,
# repeats n, first stride s) of the 17 inverted-residual blocks
MBV2_BLOCKS = ((1, 16, 1, 1), (6, 24, 2, 2), (6, 32, 3, 2), (6, 64, 4, 2), (6, 96, 3, 1),
               (6, 160, 3, 2), (6, 320, 1, 1))


def hardswish_net(batch=2, hw=32, seed=29, num_classes=10, head="gemm"):
    """MobileNetV3-style QDQ graph around fp32 HardSwish. HardSwish is not
    quant-capable (fuse_qdq.cpp:96-100), so each DQ -> HardSwish -> Q between
    the QLinearConvs runs in fp32: stem 3x3/2 (3 -> 16) -> HardSwish -> 1x1
    (16 -> 20) -> HardSwish -> depthwise 3x3 (20) -> HardSwish -> fp32
    GlobalAveragePool -> Flatten -> Gemm -> HardSwish, the last one fused into
    the Gemm as a post-op (fuse_post_ops.cpp:25-68). head="matmul" ends in
    MatMul -> HardSwish instead, which stays unfused."""
    g = Graph()
    rng = np.random.default_rng(seed)
    q = _QDQ(g, rng)
    g.inputs["input"] = (np.float32, (batch, 3, hw, hw))
    x_q, x_qp = q.quant("input", F32(1.0 / 255.0), 0, name="input_Q")
    # 20 channels: element counts that are not multiples of 16, so the
    # HardSwish tail expression is exercised
    for i, (cin, cout, k, stride, group) in enumerate(((3, 16, 3, 2, 1), (16, 20, 1, 1, 1),
                                                       (20, 20, 3, 1, 20))):
        y, y_qp = q.conv(x_q, x_qp, cin, cout, k, stride=stride, pad=k // 2, relu=False,
                         name=f"conv{i + 1}", group=group, y_zp=128)
        h = g.node("HardSwish", [q.dequant(y, y_qp)], name=f"hswish{i + 1}")
        # HardSwish >= -0.375: a zero point low in the range
        x_q, x_qp = q.quant(h, q.scale(), 16)
    f = q.dequant(x_q, x_qp, name="head_dq")
    p = g.node("GlobalAveragePool", [f], name="gap")
    fl = g.node("Flatten", [p], name="flatten", axis=1)
    fw = g.init("fc_w", rng.normal(0.0, 1.0, (num_classes, 20)).astype(F32))
    fb = g.init("fc_b", rng.normal(0.0, 0.5, num_classes).astype(F32))
    if head == "gemm":
        fc = g.node("Gemm", [fl, fw, fb], name="fc", transB=1)
    else:
        fwt = g.init("fc_wt", np.ascontiguousarray(g.initializers.pop("fc_w").T))
        g.initializers.pop(fb)
        fc = g.node("MatMul", [fl, fwt], name="fc")
    g.node("HardSwish", [fc], outputs="logits", name="fc_hswish")
    g.outputs.append("logits")
    return g


def mobilenetv2(batch=256, hw=224, seed=4, num_classes=1000):
    """MobileNetV2 int8 QDQ: stem 3x3/2 (3->32), 17 inverted-residual blocks
    (1x1 expand, 3x3 depthwise, 1x1 linear project; residual add when the
    stride is 1 and the width is unchanged), 1x1 to 1280, fp32 GAP + Gemm.
    ReLU6 is absorbed into the output quantization (y_zp 0, y_scale 6/255),
    the form NNR fuses; the linear projections and the adds quantize with
    zero point 128."""
    g = Graph()
    rng = np.random.default_rng(seed)
    q = _QDQ(g, rng)
    relu6 = F32(6.0 / 255.0)
    g.inputs["input"] = (np.float32, (batch, 3, hw, hw))
    x_q, x_qp = q.quant("input", F32(1.0 / 255.0), 0, name="input_Q")
    x_q, x_qp = q.conv(x_q, x_qp, 3, 32, 3, stride=2, pad=1, name="stem", y_scale=relu6, y_zp=0)
    cin = 32
    bi = 0
    for t, c, n, s in MBV2_BLOCKS:
        for r in range(n):
            stride = s if r == 0 else 1
            bi += 1
            nm = f"b{bi}"
            hid = cin * t
            a, a_qp = x_q, x_qp
            if t != 1:
                a, a_qp = q.conv(a, a_qp, cin, hid, 1, name=nm + "_expand", y_scale=relu6, y_zp=0)
            a, a_qp = q.conv(a, a_qp, hid, hid, 3, stride=stride, pad=1, group=hid, name=nm + "_dw",
                             y_scale=relu6, y_zp=0)
            a, a_qp = q.conv(a, a_qp, hid, c, 1, relu=False, name=nm + "_project")
            if stride == 1 and cin == c:
                sm = g.node("Add", [q.dequant(a, a_qp), q.dequant(x_q, x_qp)], name=nm + "_add")
                x_q, x_qp = q.quant(sm, q.scale(), 128)
            else:
                x_q, x_qp = a, a_qp
            cin = c
    x_q, x_qp = q.conv(x_q, x_qp, cin, 1280, 1, name="last", y_scale=relu6, y_zp=0)
    f = q.dequant(x_q, x_qp, name="head_dq")
    p = g.node("GlobalAveragePool", [f], name="gap")
    fl = g.node("Flatten", [p], name="flatten", axis=1)
    fw = g.init("fc_w", rng.normal(0.0, np.sqrt(1.0 / 1280), (num_classes, 1280)).astype(F32))
    fb = g.init("fc_b", rng.normal(0.0, 0.01, num_classes).astype(F32))
    g.node("Gemm", [fl, fw, fb], outputs="logits", name="fc", transB=1)
    g.outputs.append("logits")
    return g


def bert(batch=64, seq=128, layers=12, hidden=768, heads=12, ffn=3072, seed=5, per_channel=False):
    """BERT-base-shaped int8 encoder (cfg5). Attention scores, Softmax,
    LayerNormalization and Gelu are fp32. Input: seeded uniform token
    embeddings [batch, seq, hidden]. The weights are N(0, 0.02) before
    quantization; each projection has one of two forms:
      per_channel=False: DynamicQuantizeLinear -> DQ -> MatMul(DQ(W int8)) ->
        Q -> DQ -> + bias, which the QDQ fusion turns into a QLinearMatMul
        reading the dynamic uint8 activation scale / zero point from device
        memory. W is quantized per tensor: NNR's QLinearMatMul reads
        b_scale[0] only (QLinearMatMul.cpp:118-119), so per-channel weight
        scales would not be applied in this form.
      per_channel=True: W quantized per output channel, as dynamic
        quantization emits it (and NNR runs it, MatMulInteger.cpp:11-150):
        DynamicQuantizeLinear -> MatMulInteger(x_q, W_q, x_zp) -> Cast(float)
        -> Mul(., Mul(x_scale, w_scale[N])) -> + bias."""
    g = Graph()
    rng = np.random.default_rng(seed)
    dh = hidden // heads
    g.inputs["input"] = (np.float32, (batch, seq, hidden))

    def dynq_raw(x_f, name):
        return g.node("DynamicQuantizeLinear", [x_f], outputs=[name + "_xq", name + "_xs", name + "_xz"],
                      name=name + "_dynq")

    def dynq(x_f, name):
        if per_channel:
            return dynq_raw(x_f, name)
        xq, xs, xz = dynq_raw(x_f, name)
        return g.node("DequantizeLinear", [xq, xs, xz], name=name + "_xdq")

    def qlinear_pc(x_f, din, dout, name, dyn=None):
        xq, xs, xz = dyn if dyn is not None else dynq_raw(x_f, name)
        w = rng.normal(0.0, 0.02, (din, dout)).astype(F32)
        ws = np.maximum(np.abs(w).max(0) / F32(127.0), F32(1e-8)).astype(F32)
        wq = np.clip(np.rint(w / ws[None, :]), -127, 127).astype(np.int8)
        sp = g.node("Mul", [xs, g.init(name + "_ws", ws)], name=name + "_scale")
        acc = g.node("MatMulInteger", [xq, g.init(name + "_w", wq), xz], name=name)
        af = g.node("Cast", [acc], name=name + "_cast", to=1)
        y = g.node("Mul", [af, sp], name=name + "_deq")
        b = g.init(name + "_b", rng.normal(0.0, 0.02, dout).astype(F32))
        return g.node("Add", [y, b], name=name + "_bias")

    def qlinear(x_f, din, dout, name, y_scale, xdq=None):
        if per_channel:
            return qlinear_pc(x_f, din, dout, name, xdq)
        if xdq is None:
            xdq = dynq(x_f, name)
        w = rng.normal(0.0, 0.02, (din, dout)).astype(F32)
        ws = F32(max(float(np.abs(w).max()) / 127.0, 1e-8))
        wq = np.clip(np.rint(w / ws), -127, 127).astype(np.int8)
        wdq = g.node("DequantizeLinear", [g.init(name + "_w", wq), g.init(name + "_ws", np.array(ws, F32)),
                                          g.init(name + "_wz", np.array(0, np.int8))], name=name + "_wdq")
        y = g.node("MatMul", [xdq, wdq], name=name)
        ys = g.init(name + "_ys", np.array(y_scale, F32))
        yz = g.init(name + "_yz", np.array(128, np.uint8))
        yq = g.node("QuantizeLinear", [y, ys, yz], name=name + "_q")
        ydq = g.node("DequantizeLinear", [yq, ys, yz], name=name + "_ydq")
        b = g.init(name + "_b", rng.normal(0.0, 0.02, dout).astype(F32))
        return g.node("Add", [ydq, b], name=name + "_bias")

    def shape(name, dims):
        return g.init(name, np.array(dims, np.int64))

    x = "input"
    for li in range(layers):
        p = f"l{li}"
        xdq = dynq(x, p + "_qkv")   # one dynamic quantization feeds Q, K and V
        q = qlinear(x, hidden, hidden, p + "_q", 0.03, xdq)
        k = qlinear(x, hidden, hidden, p + "_k", 0.03, xdq)
        v = qlinear(x, hidden, hidden, p + "_v", 0.03, xdq)
        heads4 = shape(p + "_heads", [batch, seq, heads, dh])
        q4 = g.node("Transpose", [g.node("Reshape", [q, heads4], name=p + "_qr")], name=p + "_qt",
                    perm=[0, 2, 1, 3])
        kt = g.node("Transpose", [g.node("Reshape", [k, heads4], name=p + "_kr")], name=p + "_kt",
                    perm=[0, 2, 3, 1])
        v4 = g.node("Transpose", [g.node("Reshape", [v, heads4], name=p + "_vr")], name=p + "_vt",
                    perm=[0, 2, 1, 3])
        s = g.node("MatMul", [q4, kt], name=p + "_scores")
        s = g.node("Mul", [s, g.init(p + "_scale", np.array(1.0 / np.sqrt(dh), F32))], name=p + "_scaled")
        pr = g.node("Softmax", [s], name=p + "_softmax", axis=-1)
        c = g.node("MatMul", [pr, v4], name=p + "_context")
        c = g.node("Transpose", [c], name=p + "_ct", perm=[0, 2, 1, 3])
        c = g.node("Reshape", [c, shape(p + "_merge", [batch, seq, hidden])], name=p + "_cr")
        o = qlinear(c, hidden, hidden, p + "_o", 0.03)
        h1 = g.node("LayerNormalization",
                    [g.node("Add", [x, o], name=p + "_res1"), g.init(p + "_ln1_g", np.ones(hidden, F32)),
                     g.init(p + "_ln1_b", np.zeros(hidden, F32))], name=p + "_ln1", axis=-1, epsilon=1e-12)
        f = qlinear(h1, hidden, ffn, p + "_ffn1", 0.04)
        f = g.node("Gelu", [f], name=p + "_gelu")
        f2 = qlinear(f, ffn, hidden, p + "_ffn2", 0.04)
        x = g.node("LayerNormalization",
                   [g.node("Add", [h1, f2], name=p + "_res2"), g.init(p + "_ln2_g", np.ones(hidden, F32)),
                    g.init(p + "_ln2_b", np.zeros(hidden, F32))], name=p + "_ln2", axis=-1, epsilon=1e-12)
    g.outputs.append(x)
    return g


def bert_int8_ops(batch=64, seq=128, layers=12, hidden=768, ffn=3072):
    """Algorithmic int8 ops of the projections of one forward pass."""
    return 2.0 * batch * seq * layers * (4 * hidden * hidden + 2 * hidden * ffn)
