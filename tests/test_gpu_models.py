"""End-to-end parity of the configuration graphs through the host framework
(C++ context_t, HIP backend): every int8 tensor of the executed plan is
compared bit for bit with the oracle replaying the same plan; fp32 outputs
within the reference's float tolerance (tensor_equal: |a-b| <= 1e-3)."""
import numpy as np
import pytest

from nnr_amd import graph as G
from nnr_amd import synth
from oracle import graph_oracle

pytestmark = pytest.mark.gpu


def check_graph(g, feeds, out_name, atol=1e-3, conv_add=True):
    s = G.Session(g, conv_add=conv_add)
    for k, v in feeds.items():
        s.set_input(k, v)
    s.run()
    plan = s.plan()
    fmt = lambda n: s.tensor_info(n)[3]
    env = graph_oracle.run_plan(plan, g, feeds, fmt)
    n_int = 0
    for p in plan:
        o = p["outputs"][0]
        dev, _ = s.output(o)
        ref = env[o]
        assert dev.shape == ref.shape, (p["name"], dev.shape, ref.shape)
        if np.issubdtype(dev.dtype, np.integer):
            mism = np.count_nonzero(dev != ref)
            assert mism == 0, f"{p['name']} ({p['op']} {p['variant']}): {mism} of {dev.size} differ"
            if p["op"] == "QLinearConv":
                assert p.get("oracle_branch") is not None
            n_int += 1
        else:
            np.testing.assert_allclose(dev, ref, atol=atol, rtol=1e-4, err_msg=p["name"])
    out, _ = s.output(out_name)
    return plan, out, n_int


def test_resnet50_b2_bitexact(dev):
    g = synth.resnet50(batch=2, hw=224)
    rng = np.random.default_rng(10)
    x = rng.random((2, 3, 224, 224), dtype=np.float32)
    plan, logits, n_int = check_graph(g, {"input": x}, "logits")
    # every residual add runs in the epilogue of the conv that produces it
    fused = sum(1 for p in plan if p["fused_add"])
    assert fused == 16
    # the input QuantizeLinear runs in the stem's layout kernel, the head's
    # DequantizeLinear inside GlobalAveragePool
    pre = {p["op"]: p["fused_pre"] for p in plan if p["fused_pre"]}
    assert sorted(pre) == ["GlobalAveragePool", "QLinearConv"]
    # the MaxPool after the stem runs in the stem's kernel
    pooled = [p for p in plan if p["op"] == "QLinearConv" and p.get("fused_chain")]
    assert len(pooled) == 1 and pooled[0]["variant"] == "FIRST+MaxPool"
    assert "MaxPool" not in [p["op"] for p in plan]
    assert n_int == 53 + (16 - fused)  # convs (+adds)
    assert logits.shape == (2, 1000) and np.isfinite(logits).all()


# instantiations of the GEMM kernel (template arguments BM, BN, stages,
# A producer, epilogue, fusion, K bytes per stage, register-weight K steps,
# K split) that only the batch-256 plans take
B256_VARIANTS = {
    "resnet50": ("variant:dma<256,128,3,",        # 8-wave 256x128 tiles
                 "variant:dma<256,64,2,3,",       # 2-stage 256x64 uniform-tap conv tiles
                 ",128,0,2>",                     # K split over two waves a sub-tile
                 ",64,1,1>",                      # weights in registers (fused add, K = 64)
                 ",2,5,64,0,1>",                  # one residual buffer a block (fused add, K >= 128)
                 "variant:direct"),               # the short-K direct kernel (K = 64, no add)
    "mobilenetv2": ("variant:dma<256,64,", "variant:direct"),
}


@pytest.mark.parametrize("model", ["resnet50", "mobilenetv2"])
def test_model_b256_bitexact(dev, model):
    """cfg3 / cfg4 at the config's own batch (256 at 224x224), where the
    tile rules take instantiations batch 2 does not (8-wave 256x128 tiles,
    2-stage 256x64 tiles, K split on persistent grids, register weights for
    fused adds) and every persistent block walks many tiles: every int8
    tensor of the plan on images 0, 1, 254 and 255 (tiles from the start
    and the end of the blocks' walks) bit-exact with the oracle's replay of
    the plan on those images; fp32 within 1e-3."""
    from nnr_amd import _lib
    B = 256
    g = getattr(synth, model)(batch=B, hw=224)
    rng = np.random.default_rng(10 if model == "resnet50" else 16)
    x = rng.random((B, 3, 224, 224), dtype=np.float32)
    s = G.Session(g)
    s.set_input("input", x)
    _lib.profile_reset()
    _lib.profile_enable(True)
    s.run()
    _lib.profile_enable(False)
    variants = _lib.profile_read(variants=True)
    _lib.profile_reset()
    for v in B256_VARIANTS[model]:
        assert any(v in k for k in variants), (v, sorted(variants))
    plan = s.plan()
    idx = [0, 1, B - 2, B - 1]
    env = graph_oracle.run_plan(plan, g, {"input": x[idx]}, lambda n: s.tensor_info(n)[3])
    n_int = 0
    for p in plan:
        o = p["outputs"][0]
        d = s.output(o)[0][idx]
        if np.issubdtype(d.dtype, np.integer):
            mism = np.count_nonzero(d != env[o])
            assert mism == 0, f"{p['name']} ({p['op']} {p['variant']}): {mism} of {d.size} differ"
            n_int += 1
        else:
            np.testing.assert_allclose(d, env[o], atol=1e-3, rtol=1e-4, err_msg=p["name"])
    assert n_int >= (53 if model == "resnet50" else 52)


def test_resnet50_small_input(dev):
    """Same network at 96x96 (ragged spatial sizes 48/24/12/6/3)."""
    g = synth.resnet50(batch=3, hw=96, seed=11)
    rng = np.random.default_rng(12)
    x = rng.random((3, 3, 96, 96), dtype=np.float32)
    check_graph(g, {"input": x}, "logits")


def test_resnet50_unfused_adds(dev):
    """Without the conv+add epilogue fusion every conv and add output is a
    tensor of its own; all of them are bit-exact too."""
    g = synth.resnet50(batch=2, hw=64, seed=14)
    rng = np.random.default_rng(15)
    x = rng.random((2, 3, 64, 64), dtype=np.float32)
    plan, _, n_int = check_graph(g, {"input": x}, "logits", conv_add=False)
    assert not any(p["fused_add"] or p["fused_pre"] for p in plan)
    assert n_int == 53 + 16 + 1 + 1


def test_qconv_graph_config2(dev):
    g = synth.qconv_graph(batch=4)
    rng = np.random.default_rng(13)
    x = (rng.random((4, 64, 56, 56), dtype=np.float32) * 5 - 2.5).astype(np.float32)
    plan, y, _ = check_graph(g, {"input": x}, g.outputs[0])
    assert [p["variant"] for p in plan if p["op"] == "QLinearConv"] == ["NR16"]


@pytest.mark.parametrize("pool", ["avg", "ceil"])
def test_qoperator_graph(dev, pool):
    """QOperator-format graph through the host framework: QLinearConv ->
    QLinearAveragePool (3x3/2 padded, or 2x2/2 with ceil_mode) -> two conv
    branches -> QLinearConcat (one input copied) -> QLinearMul per channel and
    with itself -> QLinearGlobalAveragePool; every int8 tensor bit-exact with
    the oracle's replay of the plan, in the layouts the plan chose."""
    g = synth.qoperator_net(batch=3, hw=21, pool=pool)
    rng = np.random.default_rng(23)
    x = rng.uniform(-1.0, 1.5, (3, 3, 21, 21)).astype(np.float32)
    plan, y, n_int = check_graph(g, {"input": x}, g.outputs[0])
    ops = [p["op"] for p in plan]
    for op in ("QLinearAveragePool", "QLinearConcat", "QLinearMul", "QLinearGlobalAveragePool"):
        assert op in ops
    assert n_int >= 8 and y.size == 3 * 32   # [3, 32, 1, 1] (physically NHWC here)


def test_qconv1d_graph(dev):
    """A 1-D convolution in QDQ form (3-D tensors) through the host framework:
    fused to QLinearConv, run on its exec_typed path, bit-exact."""
    g = synth.qconv1d_graph(batch=3, C=16, W=57, OC=20, k=5, stride=2, pad=2, dil=1, group=4)
    rng = np.random.default_rng(22)
    x = rng.uniform(-2.0, 2.0, (3, 16, 57)).astype(np.float32)
    plan, y, _ = check_graph(g, {"input": x}, g.outputs[0])
    assert [p["variant"] for p in plan if p["op"] == "QLinearConv"] == ["TYPED"]
    assert y.shape == (3, 20, 29)


def test_mobilenetv2_b2_bitexact(dev):
    """cfg4 shape at batch 2: stem (first layer), 17 depthwise (RQ-A), 34
    pointwise (RQ-B), 10 residual adds; every int8 tensor bit-exact."""
    g = synth.mobilenetv2(batch=2, hw=224)
    rng = np.random.default_rng(16)
    x = rng.random((2, 3, 224, 224), dtype=np.float32)
    plan, logits, n_int = check_graph(g, {"input": x}, "logits")
    variants = [p["variant"].split("+")[0] for p in plan if p["op"] == "QLinearConv"]
    assert variants.count("DW") == 17 and variants.count("FIRST") == 1
    assert logits.shape == (2, 1000) and np.isfinite(logits).all()


def test_mobilenetv2_small_input(dev):
    """96x96 input: odd spatial sizes (48/24/12/6/3) through every stride."""
    g = synth.mobilenetv2(batch=3, hw=96, seed=17)
    rng = np.random.default_rng(18)
    x = rng.random((3, 3, 96, 96), dtype=np.float32)
    check_graph(g, {"input": x}, "logits")


def check_graph_per_node(g, feeds, atol=1e-3, rtol=1e-3, **session_kw):
    """Every node of the executed plan, recomputed by the oracle from the
    device's own input tensors: int8 outputs bit-exact, fp32 outputs within
    the reference's tolerance. Used where fp32 nodes feed dynamic
    quantization, so rounding noise must not propagate between nodes. The
    fp32 tensors a fused chain would store as uint8 bytes for its
    DynamicQuantizeLinear are materialized (codes off), so that the
    quantizer is checked on the device's own fp32 input; test_bert_codes
    checks the bytes path against this one."""
    session_kw.setdefault("codes", False)
    s = G.Session(g, **session_kw)
    for k, v in feeds.items():
        s.set_input(k, v)
    s.run()
    plan = s.plan()
    fmt = lambda n: s.tensor_info(n)[3]
    cache = {}

    def dev(name):
        if name not in cache:
            cache[name] = s.output(name)[0]
        return cache[name]

    env = graph_oracle.run_plan(plan, g, feeds, fmt, source=dev)
    n_int = n_f32 = 0
    exact_chains.clear()
    for p in plan:
        for o in p["outputs"]:
            if not o or o not in env:
                continue
            d, ref = dev(o), env[o]
            assert d.shape == np.shape(ref), (p["name"], o, d.shape, np.shape(ref))
            if d.dtype in (np.uint8, np.int8):
                mism = np.count_nonzero(d != ref)
                assert mism == 0, f"{p['name']} ({p['op']}) {o}: {mism} of {d.size} differ"
                n_int += 1
            else:
                np.testing.assert_allclose(d, ref, atol=atol, rtol=rtol, err_msg=f"{p['name']} {o}")
                n_f32 += 1
                # a projection's fused dequantize / scale / bias chain forms
                # the same binary32 operations in the same order as the
                # operators run apart: bit for bit (a Gelu's erf is the one
                # expression here whose float64 oracle differs by ulps)
                if (p["op"] in ("QLinearMatMul", "MatMulInteger") and p.get("fused_chain")
                        and "+Gelu" not in p["variant"]):
                    assert np.array_equal(d.view(np.uint32), np.asarray(ref, np.float32).view(np.uint32)), \
                        f"{p['name']} ({p['variant']}) {o}: fused chain not bit-exact"
                    exact_chains.append(p["name"])
    return plan, n_int, n_f32


exact_chains = []   # the fused projection chains the last per-node check compared bit for bit


@pytest.mark.parametrize("fused", [True, False])
def test_bert_per_node(dev, fused):
    """cfg5 structure (2 layers, batch 2, seq 64): DynamicQuantizeLinear ->
    QLinearMatMul with device-side activation scale / zero point, fp32
    attention (batched MatMul, Softmax), LayerNormalization, Gelu."""
    g = synth.bert(batch=2, seq=64, layers=2)
    rng = np.random.default_rng(19)
    x = rng.uniform(-1.0, 1.0, (2, 64, 768)).astype(np.float32)
    plan, n_int, n_f32 = check_graph_per_node(g, {"input": x}, conv_add=fused)
    ops = [p["op"] for p in plan]
    assert ops.count("QLinearMatMul") == 12 and ops.count("DynamicQuantizeLinear") == 8
    if not fused:
        assert not any(p.get("fused_chain") for p in plan)
        assert "MultiHeadAttention" not in ops
        assert n_int >= 12 + 8 * 2 and n_f32 > 0
        return
    # the head split / scaled-softmax attention / head merge of each layer is
    # one MultiHeadAttention
    assert ops.count("MultiHeadAttention") == 2 and "Softmax" not in ops and "Transpose" not in ops
    # every QLinearMatMul absorbs its DequantizeLinear and bias Add, so its
    # checked output is the fp32 end of the chain; the int8 outputs left are
    # those of DynamicQuantizeLinear (y and zero point)
    chains = [p for p in plan if p["op"] == "QLinearMatMul" and p.get("fused_chain")]
    assert len(chains) == 12
    # FF1 also absorbs its Gelu; each residual Add is formed inside its
    # LayerNormalization; the DynamicQuantizeLinear after a LayerNormalization,
    # a fused FF1 or the attention reads min / max pairs its producer wrote
    # (3 per layer, plus the next layer's input after LN2)
    assert sum(p["variant"].endswith("+Gelu") for p in chains) == 2 and "Gelu" not in ops
    assert [p["variant"] for p in plan if p["op"] == "LayerNormalization"] == ["+Add"] * 4
    assert "Add" not in ops
    assert sum(p["variant"] == "MinMaxIn" for p in plan if p["op"] == "DynamicQuantizeLinear") == 7
    # each layer's Q / K / V projections run as one grouped launch
    assert sum(p["variant"].endswith("+Group3") for p in chains) == 2
    assert sum(p["variant"].endswith("(grouped)") for p in chains) == 4
    assert n_int >= 8 * 2 and n_f32 >= 12
    # Q, K, V, O and FF2 of each layer: the per-tensor QLinearMatMul ->
    # DequantizeLinear -> bias Add chains bit-exact
    assert len(exact_chains) == 5 * 2


def test_operator_workspace(dev):
    """One scratch buffer per context, sized by the largest operator need
    (src/nnr.h:384,557-558, src/nnr.cpp:1067-1069): in BERT only the graph
    input's DynamicQuantizeLinear needs scratch once the other quantizers read
    their producers' pairs or bytes; with the fusions off all eight share the
    one buffer (test_bert_per_node checks those quantizers' bytes against
    the oracle, fused and unfused)."""
    from nnr_amd._lib import lib
    need = int(lib().nnrh_dynamic_quantize_workspace())
    g = synth.bert(batch=2, seq=64, layers=1)
    x = np.random.default_rng(23).uniform(-1.0, 1.0, (2, 64, 768)).astype(np.float32)
    for fused in (True, False):
        s = G.Session(g, conv_add=fused)
        s.set_input("input", x)
        s.run()
        assert s.workspace_bytes() == need, (fused, s.workspace_bytes(), need)
        for o in g.outputs:
            assert np.isfinite(s.output(o)[0]).all()
    # head size 32: the attention's general path, whose score matrix is the
    # largest need; every node of that plan checked against the oracle
    import ctypes as C
    g2 = synth.bert(batch=2, seq=64, layers=1, hidden=256, heads=8, ffn=1024)
    x2 = np.random.default_rng(29).uniform(-1.0, 1.0, (2, 64, 256)).astype(np.float32)
    att = C.c_size_t()
    assert lib().nnrh_multihead_attention_workspace(2, 64, 256, 8, C.byref(att)) == 0
    assert att.value > need
    s = G.Session(g2)
    s.set_input("input", x2)
    s.run()
    assert "MultiHeadAttention" in [p["op"] for p in s.plan()]
    assert s.workspace_bytes() == att.value
    check_graph_per_node(g2, {"input": x2})


def test_bert_full_depth_seq128(dev):
    """cfg5 at its real per-sequence shape: 12 layers, seq 128, hidden 768,
    12 heads, FFN 3072 (batch 2 of the config's 64: the batch only repeats
    the same per-sequence work). Every node recomputed by the oracle from the
    device's own inputs: int8 outputs (DynamicQuantizeLinear bytes and zero
    points) exact, fp32 outputs within 1e-3. Seq 128 takes the fused
    head-64 attention kernel."""
    g = synth.bert(batch=2, seq=128, layers=12)
    rng = np.random.default_rng(35)
    x = rng.uniform(-1.0, 1.0, (2, 128, 768)).astype(np.float32)
    plan, n_int, n_f32 = check_graph_per_node(g, {"input": x})
    ops = [p["op"] for p in plan]
    assert ops.count("QLinearMatMul") == 72 and ops.count("MultiHeadAttention") == 12
    assert ops.count("DynamicQuantizeLinear") == 48
    assert n_int >= 48 * 2 and n_f32 >= 72
    assert len(exact_chains) == 5 * 12   # every fused chain without Gelu, bit for bit


def test_bert_codes(dev):
    """fuse_dynq_codes and fuse_codes_readers: every projection chain stores
    its uint8 QLinearMatMul bytes -- FF1 (with Gelu) for its
    DynamicQuantizeLinear, Q / K / V (one grouped launch) for the fused
    attention, O and FF2 for the LayerNormalization with the residual Add --
    and each reader forms the values itself. Against a context that
    materializes the fp32 tensors: every tensor both plans hold in the same
    type (every DynamicQuantizeLinear, attention and LayerNormalization
    output, the graph output) bit-identical, on two inputs; every stored byte
    tensor equals the oracle's QLinearMatMul bytes from the device's own
    inputs; less device memory."""
    layers, B, S = 3, 2, 128
    g = synth.bert(batch=B, seq=S, layers=layers)
    rng = np.random.default_rng(37)
    on, off = G.Session(g), G.Session(g, codes=False)
    plan = on.plan()
    mm = [p for p in plan if p["op"] == "QLinearMatMul"]
    assert len(mm) == 6 * layers and all(p["variant"].endswith("+Codes") for p in mm)
    assert sorted({p["variant"] for p in mm}) == ["+DQ+Bias(grouped)+Codes", "+DQ+Bias+Codes", "+DQ+Bias+Gelu+Codes",
                                                  "+DQ+Bias+Group3+Codes"]
    assert sum(p["variant"] == "Codes" for p in plan if p["op"] == "DynamicQuantizeLinear") == layers
    assert [p["variant"] for p in plan if p["op"] == "MultiHeadAttention"] == ["Codes"] * layers
    assert [p["variant"] for p in plan if p["op"] == "LayerNormalization"] == ["+Add+Codes"] * (2 * layers)
    assert not any("Codes" in p["variant"] for p in off.plan())
    for p in mm:
        t = p["outputs"][0]
        assert on.tensor_info(t)[1] == np.uint8 and off.tensor_info(t)[1] == np.float32
    assert on.device_bytes() < off.device_bytes()
    for rep in range(2):
        x = rng.uniform(-1.0, 1.0, (B, S, 768)).astype(np.float32)
        for s in (on, off):
            s.set_input("input", x)
            s.run()
        same = 0
        for p in plan:
            for o in p["outputs"]:
                if not o or on.tensor_info(o)[1] != off.tensor_info(o)[1]:
                    continue
                a, b = np.atleast_1d(on.output(o)[0]), np.atleast_1d(off.output(o)[0])
                assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), (rep, p["name"], o)
                same += 1
        assert same >= layers * (4 * 3 + 3)   # 4 quantizers x 3 outputs, attention, 2 norms
    cache = {}

    def dev_t(name):
        if name not in cache:
            cache[name] = on.output(name)[0]
        return cache[name]

    skip = {p["op"] for p in plan} - {"QLinearMatMul"}
    env = graph_oracle.run_plan(plan, g, {"input": x}, lambda n: on.tensor_info(n)[3], source=dev_t,
                                skip_ops=skip, keep_chain=True)
    for p in mm:
        q = g.node_by_name(p["fused_chain"][0]).inputs[0]
        assert env[q].dtype == np.uint8
        assert np.array_equal(dev_t(p["outputs"][0]), env[q]), p["name"]


@pytest.mark.parametrize("layers,seq,fused", [(12, 128, True), (2, 64, False)])
def test_bert_per_channel(dev, layers, seq, fused):
    """cfg5 with per-channel weights in the dynamic-quantization form NNR runs
    (DynamicQuantizeLinear -> MatMulInteger -> Cast -> Mul(Mul(x_scale,
    w_scale[N])) -> Add): fused, every projection is one GEMM writing the fp32
    chain end (Q / K / V grouped, FF1 with its Gelu); unfused, each operator
    runs alone. Every node recomputed by the oracle from the device's own
    inputs: int8 exact; the fused projections without Gelu bit-exact, the
    rest of the fp32 values within 1e-3."""
    from oracle import graph_oracle as GO
    g = synth.bert(batch=2, seq=seq, layers=layers, per_channel=True)
    rng = np.random.default_rng(36)
    x = rng.uniform(-1.0, 1.0, (2, seq, 768)).astype(np.float32)
    plan, n_int, n_f32 = check_graph_per_node(g, {"input": x}, conv_add=fused)
    ops = [p["op"] for p in plan]
    assert ops.count("MatMulInteger") == 6 * layers
    if not fused:
        assert ops.count("Cast") == 6 * layers and not any(p.get("fused_chain") for p in plan)
        return
    assert "Cast" not in ops and "Gelu" not in ops
    mm = [p for p in plan if p["op"] == "MatMulInteger"]
    assert all(p["variant"].startswith("+Cast+Scale+Bias") for p in mm)
    assert sum(p["variant"].endswith("+Group3") for p in mm) == layers
    assert sum("+Gelu" in p["variant"] for p in mm) == layers
    # bit-exact fused chains (no Gelu): device vs the oracle on the device's inputs
    s = G.Session(g)
    s.set_input("input", x)
    s.run()
    plan = s.plan()
    cache = {}

    def dv(name):
        if name not in cache:
            cache[name] = s.output(name)[0]
        return cache[name]

    env = GO.run_plan(plan, g, {"input": x}, lambda n: s.tensor_info(n)[3], source=dv)
    exact = 0
    for p in mm:
        if "+Gelu" in p["variant"]:
            continue
        o = p["outputs"][0]
        assert np.array_equal(dv(o).view(np.uint32), env[o].view(np.uint32)), p["name"]
        exact += 1
    assert exact == 5 * layers


@pytest.mark.parametrize("name", ["resnet50", "mobilenetv2", "bert", "qoperator", "concat_b1", "concat_b2"])
def test_memory_planning(dev, name):
    """The device memory planner (shared arena slots, in-place outputs,
    concat parts inside their output) changes no result: with the fusions
    that need built operators in the plan, the graph outputs of two runs are
    bit-identical to those of a context with one allocation per tensor, and
    the applied plan keeps every pair of tensors live at once on disjoint
    bytes."""
    from test_memory_planner import check_plan
    rng = np.random.default_rng(30)
    if name == "resnet50":
        g, x = synth.resnet50(batch=2, hw=64, seed=14), rng.random((2, 3, 64, 64), dtype=np.float32)
    elif name == "mobilenetv2":
        g, x = synth.mobilenetv2(batch=2, hw=96, seed=17), rng.random((2, 3, 96, 96), dtype=np.float32)
    elif name == "bert":
        g, x = synth.bert(batch=2, seq=64, layers=2), rng.uniform(-1, 1, (2, 64, 768)).astype(np.float32)
    elif name == "qoperator":
        g, x = synth.qoperator_net(batch=3, hw=21), rng.uniform(-1, 1.5, (3, 3, 21, 21)).astype(np.float32)
    else:
        b = 1 if name == "concat_b1" else 2
        g, x = synth.concat_net(batch=b), rng.uniform(-1, 1.5, (b, 16, 8, 8)).astype(np.float32)
    outs = {}
    for planned in (False, True):
        s = G.Session(g, memory_planning=planned)
        s.set_input("input", x)
        runs = []
        for _ in range(2):
            s.run()
            runs.append({o: s.output(o)[0].copy() for o in g.outputs})
        for o in g.outputs:
            assert np.array_equal(runs[0][o], runs[1][o]), (name, planned, o)
        outs[planned] = (runs[0], s.device_bytes(), s)
    for o in g.outputs:
        assert np.array_equal(outs[False][0][o], outs[True][0][o]), (name, o)
    stats, entries = outs[True][2].memory_plan()
    check_plan(stats, entries)
    assert outs[True][1] < outs[False][1]
    if name == "concat_b1":
        assert stats["concat"] == 2


@pytest.mark.parametrize("name", ["resnet50", "bert", "qoperator"])
def test_onnx_model_bitexact(dev, name, tmp_path):
    """A model written as an ONNX file (initializers in an external-data
    file, symbolic batch) and loaded by the C++ loader runs to the same
    outputs, bit for bit, as the same graph built in process."""
    from nnr_amd import onnx_io
    rng = np.random.default_rng(31)
    if name == "resnet50":
        g, x = synth.resnet50(batch=2, hw=64, seed=14), rng.random((2, 3, 64, 64), dtype=np.float32)
    elif name == "bert":
        g, x = synth.bert(batch=2, seq=64, layers=2), rng.uniform(-1, 1, (2, 64, 768)).astype(np.float32)
    else:
        g, x = synth.qoperator_net(batch=3, hw=21), rng.uniform(-1, 1.5, (3, 3, 21, 21)).astype(np.float32)
    path = str(tmp_path / f"{name}.onnx")
    onnx_io.save(g, path, external_data=True, sym_dims=(0,))
    outs = []
    for s in (G.Session(g), G.Session(None, onnx=path, sym_dim=x.shape[0])):
        s.set_input("input", x)
        s.run()
        outs.append({o: s.output(o)[0] for o in g.outputs})
    for o in g.outputs:
        assert np.array_equal(outs[0][o], outs[1][o]), (name, o)


def test_bn_graph(dev):
    """fold_bn_qdq's two patterns through the host framework: DQ -> BN -> Q
    after a QLinearConv (NHWC) and fp32 BN -> Q (NCHW), every uint8 tensor
    bit-exact with the oracle's restatement of the fold and the kernel."""
    g = synth.bn_net(batch=2, C=40, hw=13)
    rng = np.random.default_rng(27)
    x = rng.uniform(-2.5, 2.5, (2, 40, 13, 13)).astype(np.float32)
    plan, _, n_int = check_graph(g, {"input": x}, g.outputs[0])
    assert sorted(p["variant"] for p in plan if p["op"] == "BatchNormalization") == ["BN-Q", "DQ-BN-Q"]
    assert n_int >= 4


@pytest.mark.parametrize("kw", [dict(), dict(per_channel=False, auto_pad="SAME_UPPER", strides=(2, 2)),
                                dict(auto_pad="VALID", group=2), dict(x_dtype=np.int8, auto_pad="SAME_LOWER",
                                                                      strides=(2, 1))])
def test_conv_integer_graph(dev, kw):
    """ConvInteger through the host framework (auto_pad forms, groups, scalar
    and per-channel weight zero points): int32 output exact."""
    g = synth.conv_integer_net(**kw)
    rng = np.random.default_rng(29)
    x = rng.uniform(-2.0, 2.0, (2, 16, 15, 15)).astype(np.float32)
    plan, y, _ = check_graph(g, {"input": x}, g.outputs[0], atol=0)
    assert [p["op"] for p in plan].count("ConvInteger") == 1 and y.dtype == np.int32


@pytest.mark.parametrize("shape", [(2, 24, 7, 9), (3, 5, 4)])
def test_bn_f32_unfolded(dev, shape):
    """BatchNormalization with no Q after it stays fp32 (BatchNormalization.cpp:
    126-160): within the reference's float tolerance of the float64 formula."""
    g = G.Graph()
    rng = np.random.default_rng(33)
    C = shape[1]
    g.inputs["input"] = (np.float32, shape)
    ins = ["input"] + [g.init(k, v.astype(np.float32)) for k, v in
                       (("sc", rng.uniform(0.5, 1.5, C)), ("bi", rng.normal(0, 1, C)),
                        ("me", rng.normal(0, 1, C)), ("va", rng.uniform(0.2, 2.0, C)))]
    y = g.node("BatchNormalization", ins, name="bn", epsilon=1e-4)
    g.outputs.append(y)
    x = rng.normal(0, 2, shape).astype(np.float32)
    plan, out, _ = check_graph(g, {"input": x}, y)
    assert [p["variant"] for p in plan] == [""] and out.dtype == np.float32


@pytest.mark.parametrize("hw,head", [(32, "gemm"), (29, "gemm"), (29, "matmul")])
def test_hardswish_graph(dev, hw, head):
    """MobileNetV3-style QDQ graph: each DQ -> HardSwish -> Q between the
    QLinearConvs runs the fp32 HardSwish operator, and the classifier's
    HardSwish runs fused into the fp32 Gemm. Every int8 tensor is bit-exact
    and fp32 values are within 1e-3 of the oracle's replay; each standalone
    HardSwish output also equals the oracle's HardSwish of the device's own
    input bit for bit (the same IEEE operations and body / tail split).
    With a MatMul classifier the HardSwish is not fused (its body / tail
    split would follow the reference's CPU tiles): it runs on its own."""
    from oracle import pyoracle as O
    g = synth.hardswish_net(batch=3, hw=hw, head=head)
    rng = np.random.default_rng(34)
    x = rng.random((3, 3, hw, hw), dtype=np.float32)
    plan, logits, n_int = check_graph(g, {"input": x}, "logits")
    assert [p["op"] for p in plan].count("HardSwish") == (3 if head == "gemm" else 4) and n_int >= 6
    assert logits.shape == (3, 10) and np.isfinite(logits).all()
    s = G.Session(g)
    s.set_input("input", x)
    s.run()
    tails = 0
    for p in plan:
        if p["op"] == "HardSwish":
            xin = s.output(p["inputs"][0])[0]
            assert np.array_equal(s.output(p["outputs"][0])[0], O.hardswish(xin)), p["name"]
            tails += xin.size % 16 != 0
    assert tails >= (1 if hw == 29 else 0)   # 15x15 maps of 20 channels: n % 16 != 0


@pytest.mark.parametrize("name", ["resnet50", "mobilenetv2", "bert", "bert_pc", "qoperator"])
def test_hip_graph_replay(dev, name):
    """From its second call on, run() replays the plan as one captured HIP
    graph (memory-planned context). Each replay, on a new input copied in
    between, with eager work and synchronizations between the replays,
    gives graph outputs bit-identical to a context that launches node by
    node."""
    import torch
    rng = np.random.default_rng(31)
    if name == "resnet50":
        g, shape = synth.resnet50(batch=2, hw=64, seed=14), (2, 3, 64, 64)
    elif name == "mobilenetv2":
        g, shape = synth.mobilenetv2(batch=2, hw=96, seed=17), (2, 3, 96, 96)
    elif name.startswith("bert"):
        g, shape = synth.bert(batch=2, seq=64, layers=2, per_channel=name == "bert_pc"), (2, 64, 768)
    else:
        g, shape = synth.qoperator_net(batch=3, hw=21), (3, 3, 21, 21)
    eager = G.Session(g, hip_graph=False)
    s = G.Session(g, memory_planning=True)
    for rep in range(4):
        print(f"{name} replay {rep}", flush=True)
        x = rng.uniform(-1.0, 1.5, shape).astype(np.float32)
        for sess in (eager, s):
            sess.set_input("input", x)
            sess.run()
        torch.cuda.synchronize()
        assert s.graph_active() == (rep >= 1), rep
        assert not eager.graph_active()
        for o in g.outputs:
            a, b = s.output(o)[0], eager.output(o)[0]
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), (rep, o)
        torch.zeros(1 << 20, device=dev).add_(1.0)   # eager work between the replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("name,parts", [("resnet50", 2), ("mobilenetv2", 4), ("qoperator", 3)])
def test_split_session(dev, name, parts):
    """The batch as `parts` slices run concurrently (SplitSession: one
    context and stream per slice, nnr_group_run) gives the whole-batch
    context's graph outputs bit for bit, on several steps with new inputs
    (the slices' graphs replay from the second step on), and the caller's
    stream waits for every slice."""
    import torch
    from nnr_amd import _lib
    rng = np.random.default_rng(41)
    if name == "resnet50":
        make, B, shape = (lambda b: synth.resnet50(batch=b, hw=64, seed=14)), 4, (3, 64, 64)
    elif name == "mobilenetv2":
        make, B, shape = (lambda b: synth.mobilenetv2(batch=b, hw=96, seed=17)), 4, (3, 96, 96)
    else:
        make, B, shape = (lambda b: synth.qoperator_net(batch=b, hw=21)), 6, (3, 21, 21)
    g = make(B)
    whole = G.Session(g, memory_planning=True)
    split = G.SplitSession(make, batch=B, parts=parts, memory_planning=True)
    try:
        for step in range(3):
            print(f"{name} split step {step}", flush=True)
            x = rng.uniform(-1.0, 1.5, (B,) + shape).astype(np.float32)
            whole.set_input("input", x)
            split.set_input("input", x)
            whole.run()
            torch.cuda.synchronize()
            split.run()
            # a copy enqueued on the caller's stream right after run() reads
            # the last slice's finished output (the join), with no other sync
            o0 = g.outputs[0]
            p, dt, oshape, _ = split.sessions[-1].tensor_info(o0)
            nbytes = int(np.prod(oshape)) * np.dtype(dt).itemsize
            buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
            _lib.check(_lib.lib().nnrh_memcpy(buf.data_ptr(), p, nbytes, 2, _lib.cur_stream()))
            torch.cuda.current_stream().synchronize()
            last = whole.output(o0)[0][split.slice(parts - 1)]
            assert np.array_equal(buf.cpu().numpy(), np.ascontiguousarray(last).view(np.uint8).reshape(-1)), step
            torch.cuda.synchronize()
            assert split.graph_active() == (step >= 1), step
            for o in g.outputs:
                a, b = split.output(o)[0], whole.output(o)[0]
                assert a.shape == b.shape
                assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), (step, o)
    finally:
        split.close()


def test_split_session_rejects_ragged_batch(dev):
    with pytest.raises(ValueError):
        G.SplitSession(lambda b: synth.resnet50(batch=b, hw=64), batch=5, parts=2)
