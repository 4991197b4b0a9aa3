"""Graph-layer checks without a GPU: the host framework's passes turn the
synthetic QDQ graphs into the plan the reference's optimizer produces
(fuse_qdq_compute, fuse_qdq, assign_layouts) and each QLinearConv resolves to
the kernel branch QLinearConv::exec_simd_4d would take."""
import collections

import numpy as np
import pytest

from nnr_amd import graph as G
from nnr_amd import synth
from oracle import pyoracle as O


@pytest.fixture(scope="module")
def resnet_plan():
    g = synth.resnet50(batch=2, hw=224)
    s = G.Session(g, device=False)
    return g, s, s.plan()


def test_resnet50_fusion_counts(resnet_plan):
    g, s, plan = resnet_plan
    ops = collections.Counter(p["op"] for p in plan)
    assert ops == {"QLinearConv": 53, "QLinearAdd": 16, "QuantizeLinear": 1, "MaxPool": 1,
                   "DequantizeLinear": 1, "GlobalAveragePool": 1, "Flatten": 1, "Gemm": 1}
    assert s.fusion_stat("qdq_compute") == 53
    assert s.fusion_stat("qdq_add") == 16
    assert s.fusion_stat("qdq_transparent") == 1


def test_resnet50_branches_and_layouts(resnet_plan):
    g, s, plan = resnet_plan
    br = collections.Counter(p["variant"] for p in plan if p["op"] == "QLinearConv")
    # stem -> first-layer (RQ-C); 3x3 s1 -> NR16; 1x1 and 3x3 s2 -> NR48 (RQ-B)
    assert br == {"FIRST": 1, "NR16": 13, "PACKED": 39}
    fmt = lambda n: s.tensor_info(n)[3]
    for p in plan:
        if p["op"] in ("QLinearConv", "QLinearAdd", "MaxPool"):
            assert fmt(p["outputs"][0]) == 1, p["name"]      # int8 chains are NHWC
    assert fmt(plan[0]["outputs"][0]) == 0                    # input Q stays NCHW


def test_resnet50_branch_matches_oracle_dispatch(resnet_plan):
    """Each QLinearConv's branch equals the oracle's dispatch restatement for
    the same shapes, layouts and post-op flag."""
    g, s, plan = resnet_plan
    fmt = lambda n: s.tensor_info(n)[3]
    for p in plan:
        if p["op"] != "QLinearConv":
            continue
        a = g.node_by_name(p["name"]).attrs
        ins = p["inputs"]
        w = g.initializers[ins[3]]
        _, _, xs, _ = s.tensor_info(ins[0])
        cv = O.Conv(xs[0], xs[1], xs[2], xs[3], w.shape[0], w.shape[2], w.shape[3],
                    group=a.get("group", 1), stride=tuple(a["strides"]), pads=tuple(a["pads"]),
                    x_nhwc=fmt(ins[0]), y_nhwc=fmt(p["outputs"][0]), post_fn=p["post_fn"])
        assert O.lib().orc_conv_dispatch(__import__("ctypes").byref(cv.p)) == \
            O.BR[p["variant"]], p["name"]


def test_unfusable_graph_fails_loudly():
    """A float Conv without QDQ around it has no HIP implementation: prepare
    fails with a message instead of silently running something else."""
    g = G.Graph()
    g.inputs["x"] = (np.float32, (1, 4, 8, 8))
    w = g.init("w", np.zeros((4, 4, 3, 3), np.float32))
    g.node("Conv", ["x", w], outputs="y", name="plain_conv", kernel_shape=[3, 3], pads=[1, 1, 1, 1])
    g.outputs.append("y")
    with pytest.raises(G.NnrError, match="without a HIP implementation"):
        G.Session(g, device=False)


def test_post_op_fusion_sets_qmin():
    """QLinearConv followed by a Relu: fuse_post_ops marks post_fn and the
    Relu step is skipped (fuse_post_ops.cpp:24-71)."""
    g = G.Graph()
    g.inputs["x"] = (np.uint8, (1, 8, 6, 6))
    rng = np.random.default_rng(0)
    ins = ["x", g.init("xs", np.array(0.02, np.float32)), g.init("xz", np.array(128, np.uint8)),
           g.init("w", rng.integers(-5, 5, (8, 8, 3, 3)).astype(np.int8)),
           g.init("ws", np.full(8, 0.01, np.float32)), g.init("wz", np.zeros(8, np.int8)),
           g.init("ys", np.array(0.05, np.float32)), g.init("yz", np.array(10, np.uint8))]
    g.node("QLinearConv", ins, outputs="c", name="qc", kernel_shape=[3, 3], pads=[1, 1, 1, 1])
    g.node("Relu", ["c"], outputs="r", name="relu")
    g.outputs.append("r")
    s = G.Session(g, device=False)
    plan = s.plan()
    assert [p["op"] for p in plan] == ["QLinearConv"] and plan[0]["post_fn"] == 1
    assert s.fusion_stat("post_ops") == 1


def test_mobilenetv2_fusion_and_branches():
    """cfg4: 52 QLinearConv (stem first-layer, 17 depthwise, 34 pointwise
    NR48), 10 QLinearAdd, every int8 activation NHWC."""
    g = synth.mobilenetv2(batch=2, hw=224)
    s = G.Session(g, device=False)
    plan = s.plan()
    ops = collections.Counter(p["op"] for p in plan)
    assert ops == {"QLinearConv": 52, "QLinearAdd": 10, "QuantizeLinear": 1,
                   "DequantizeLinear": 1, "GlobalAveragePool": 1, "Flatten": 1, "Gemm": 1}
    br = collections.Counter(p["variant"] for p in plan if p["op"] == "QLinearConv")
    assert br == {"FIRST": 1, "DW": 17, "PACKED": 34}
    fmt = lambda n: s.tensor_info(n)[3]
    for p in plan:
        if p["op"] in ("QLinearConv", "QLinearAdd"):
            assert fmt(p["outputs"][0]) == 1, p["name"]


def test_bert_fusion():
    """cfg5: each projection's DynQ -> DQ -> MatMul -> Q becomes a
    QLinearMatMul (6 per layer, the Q/K/V ones sharing one
    DynamicQuantizeLinear); the fp32 attention (head split, scaled softmax,
    head merge) becomes one MultiHeadAttention per layer, or stays ten
    nodes with the fusions off."""
    g = synth.bert(batch=2, seq=16, layers=2)
    s = G.Session(g, device=False)
    ops = collections.Counter(p["op"] for p in s.plan())
    assert ops["QLinearMatMul"] == 12 and ops["DynamicQuantizeLinear"] == 8
    assert ops["MultiHeadAttention"] == 2 and ops["LayerNormalization"] == 4
    assert "MatMul" not in ops and "Softmax" not in ops and "Transpose" not in ops
    assert ops["Gelu"] == 2 and "QuantizeLinear" not in ops
    assert s.fusion_stat("qdq_compute") == 12 and s.fusion_stat("attention") == 2
    u = G.Session(g, device=False, conv_add=False)
    uops = collections.Counter(p["op"] for p in u.plan())
    assert uops["MatMul"] == 4 and uops["Softmax"] == 2 and uops["Transpose"] == 8
    assert "MultiHeadAttention" not in uops


def test_qoperator_graph_layouts():
    """A QOperator-format graph (QLinearConv, QLinearAveragePool,
    QLinearConcat, QLinearMul, QLinearGlobalAveragePool) resolves on the HIP
    registry; the activations after the convolutions stay NHWC (the concat is
    along channels, the per-channel Mul and the pools read NHWC)."""
    g = synth.qoperator_net(batch=2, hw=20)
    s = G.Session(g, device=False)
    plan = s.plan()
    ops = collections.Counter(p["op"] for p in plan)
    assert ops["QLinearConv"] == 3 and ops["QLinearAveragePool"] == 1 and ops["QLinearConcat"] == 1
    assert ops["QLinearMul"] == 2 and ops["QLinearGlobalAveragePool"] == 1
    fmt = {p["name"]: s.tensor_info(p["outputs"][0])[3] for p in plan}
    assert fmt["concat"] == 1 and fmt["mul_channel"] == 1 and fmt["mul_square"] == 1


def test_fold_bn_qdq_patterns():
    """DQ -> BN -> Q (after a QLinearConv, NHWC) and fp32 BN -> Q both fold
    (fold_bn_qdq.cpp:23-259): one BatchNormalization each, reading uint8 or
    fp32 and writing the Q's uint8 tensor; the DQ / Q are skipped."""
    from nnr_amd import graph as G, synth
    g = synth.bn_net()
    s = G.Session(g, device=False)
    plan = s.plan()
    bns = {p["name"]: p for p in plan if p["op"] == "BatchNormalization"}
    assert bns["bn_a"]["variant"] == "DQ-BN-Q" and bns["bn_b"]["variant"] == "BN-Q"
    assert bns["bn_a"]["fused_pre"] == ["bn_a_dq"] and bns["bn_a"]["fused_chain"] == ["bn_a_q"]
    assert bns["bn_a"]["outputs"] == ["bn_a_q_out"] and bns["bn_b"]["inputs"][0] == "input"
    assert "QuantizeLinear" not in [p["op"] for p in plan if p["name"] != "input_Q"]
    assert s.fusion_stat("bn_qdq") == 1 and s.fusion_stat("bn_q") == 1
    assert s.tensor_info("bn_a_q_out")[3] == 1      # NHWC after the convolution


def test_hardswish_graph_plan():
    """DQ -> HardSwish -> Q stays in fp32 between the QLinearConvs (HardSwish
    is not quant-capable, fuse_qdq.cpp:96-100), and the classifier's
    HardSwish is fused into the fp32 Gemm as a post-op
    (fuse_post_ops.cpp:25-68), recorded as the Gemm's fused chain."""
    g = synth.hardswish_net(batch=2, hw=32)
    s = G.Session(g, device=False)
    plan = s.plan()
    ops = collections.Counter(p["op"] for p in plan)
    assert ops["QLinearConv"] == 3 and ops["HardSwish"] == 3 and ops["Gemm"] == 1
    assert s.fusion_stat("qdq_compute") == 3
    assert [p["variant"] for p in plan if p["op"] == "QLinearConv"] == ["FIRST", "PACKED", "DW"]
    gemm = next(p for p in plan if p["op"] == "Gemm")
    assert gemm["post_fn"] == 1 and gemm["fused_chain"] == ["fc_hswish"]
    for p in plan:
        if p["op"] == "HardSwish":
            prev = next(q for q in plan if p["inputs"][0] in q["outputs"])
            assert prev["op"] == "DequantizeLinear"
