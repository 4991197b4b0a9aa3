"""ONNX loader (nnr_amd/host/onnx_loader.cpp, `nnr_ctx_load_onnx`; the
reference's src/format/onnx/onnx_loader.cpp:491-732) and the ONNX writer
(nnr_amd/onnx_io.py), on the CPU.

Pinned three ways: the writer's field numbers against the ONNX schema table
(tests/golden/onnx_fields.json, from the schema file); the writer's bytes
parsed by google.protobuf message classes built from that table, and a model
serialized by google.protobuf loaded by the C++ reader (an implementation of
the wire format that is not this project's); and every loaded model compared
with the same graph built in process -- the executed plan node by node and
every initializer byte for byte."""
import json
import os

import numpy as np
import pytest

from nnr_amd import graph as G
from nnr_amd import onnx_io, synth

HERE = os.path.dirname(os.path.abspath(__file__))
SCHEMA = json.load(open(os.path.join(HERE, "golden", "onnx_fields.json")))

GRAPHS = {
    "resnet50": lambda: synth.resnet50(batch=2, hw=64, seed=14),
    "mobilenetv2": lambda: synth.mobilenetv2(batch=2, hw=64, seed=17),
    "bert": lambda: synth.bert(batch=2, seq=32, layers=1),
    "qoperator": lambda: synth.qoperator_net(batch=2, hw=21),
    "qconv1d": lambda: synth.qconv1d_graph(batch=3, C=16, W=57, OC=20, k=5, stride=2, pad=2, group=4),
    "concat": lambda: synth.concat_net(batch=1),
}


def same_context(g, s_onnx, s_ref=None):
    """The loaded context equals the in-process one: plan and initializers."""
    s_ref = s_ref or G.Session(g, device=False)
    assert s_onnx.plan() == s_ref.plan()
    for name in g.initializers:
        assert s_onnx.initializer_bytes(name) == s_ref.initializer_bytes(name), name
    assert s_onnx.graph_io(True) == list(g.outputs)
    assert s_onnx.graph_io(False) == list(g.inputs)
    for name in g.inputs:
        assert s_onnx.tensor_info(name)[1:] == s_ref.tensor_info(name)[1:]


def test_writer_fields_match_schema():
    for msg, fields in onnx_io.FIELDS.items():
        for f, num in fields.items():
            assert SCHEMA[msg][f][0] == num, (msg, f)


SMALL = ["qoperator", "qconv1d", "concat"]    # typed payloads are written value by value


@pytest.mark.parametrize("name,mode,packed", [(n, "raw", True) for n in sorted(GRAPHS)]
                         + [(n, m, p) for n in SMALL for m, p in (("typed", True), ("typed", False))])
def test_roundtrip(name, mode, packed):
    g = GRAPHS[name]()
    model, ext = onnx_io.encode(g, mode=mode, packed=packed)
    assert ext == b""
    same_context(g, G.Session(None, device=False, onnx=model))


def test_external_data(tmp_path):
    g = GRAPHS["resnet50"]()
    path = str(tmp_path / "resnet50.onnx")
    onnx_io.save(g, path, external_data=True)
    assert os.path.getsize(path + ".data") > 1 << 20
    same_context(g, G.Session(None, device=False, onnx=path))
    os.remove(path + ".data")
    with pytest.raises(G.NnrError, match="external data file not found"):
        G.Session(None, device=False, onnx=path)


def test_symbolic_batch():
    g = GRAPHS["qoperator"]()
    model, _ = onnx_io.encode(g, sym_dims=(0,))
    same_context(g, G.Session(None, device=False, onnx=model, sym_dim=2))
    # unset: 1, as the reference's tensor_from_value_info
    s1 = G.Session(None, device=False, onnx=model)
    assert s1.tensor_info("input")[2] == (1, 3, 21, 21)


def test_constant_nodes():
    g = GRAPHS["qoperator"]()
    consts = [n for n in g.initializers if n.endswith(("_s", "_z"))] + ["mul_ch"]
    model, _ = onnx_io.encode(g, constants=consts)
    same_context(g, G.Session(None, device=False, onnx=model))


def test_malformed_models_fail_cleanly():
    g = GRAPHS["qoperator"]()
    model, _ = onnx_io.encode(g)
    for bad in (model[: len(model) // 2], b"\x0a\xff\xff\xff\xff\x0f", b"\xff" * 16, b""):
        with pytest.raises(G.NnrError, match="not a valid ONNX"):
            G.Session(None, device=False, onnx=bad)


def test_unknown_operator_named():
    g = synth.concat_net(batch=1)
    g.nodes[1].op = "FrobnicateLinear"
    model, _ = onnx_io.encode(g)
    with pytest.raises(G.NnrError, match="FrobnicateLinear"):
        G.Session(None, device=False, onnx=model)


# ---------------------------------------------------------------------------
# google.protobuf as the independent implementation of the wire format

def _protobuf_classes():
    from google.protobuf import descriptor_pb2, descriptor_pool, message_factory
    F = descriptor_pb2.FieldDescriptorProto
    scalar = {"int64": F.TYPE_INT64, "int32": F.TYPE_INT32, "uint64": F.TYPE_UINT64, "float": F.TYPE_FLOAT,
              "double": F.TYPE_DOUBLE, "string": F.TYPE_STRING, "bytes": F.TYPE_BYTES,
              "DataLocation": F.TYPE_INT32, "AttributeType": F.TYPE_INT32}
    fdp = descriptor_pb2.FileDescriptorProto(name="onnx_subset.proto", package="sub", syntax="proto3")
    protos = {}
    for msg in sorted(SCHEMA, key=lambda m: m.count(".")):
        parts = msg.split(".")
        if len(parts) == 1:
            protos[msg] = fdp.message_type.add(name=parts[0])
        else:
            protos[msg] = protos[parts[0]].nested_type.add(name=parts[1])
    for msg, fields in SCHEMA.items():
        for fname, (num, typ, label) in fields.items():
            lab = F.LABEL_REPEATED if label == "repeated" else F.LABEL_OPTIONAL
            if typ in scalar:
                protos[msg].field.add(name=fname, number=num, type=scalar[typ], label=lab)
                continue
            target = msg.split(".")[0] + "." + typ if msg.split(".")[0] + "." + typ in SCHEMA else typ
            if target not in SCHEMA:
                continue       # messages the loader does not read
            protos[msg].field.add(name=fname, number=num, type=F.TYPE_MESSAGE, label=lab,
                                  type_name=".sub." + target)
    pool = descriptor_pool.DescriptorPool()
    pool.Add(fdp)
    return {m: message_factory.GetMessageClass(pool.FindMessageTypeByName("sub." + m)) for m in SCHEMA}


@pytest.mark.parametrize("mode,packed", [("raw", True), ("typed", False)])
def test_writer_bytes_parse_with_protobuf(mode, packed):
    P = _protobuf_classes()
    g = GRAPHS["qoperator"]()
    model, _ = onnx_io.encode(g, mode=mode, packed=packed, sym_dims=(0,))
    m = P["ModelProto"].FromString(model)
    assert [(o.domain, o.version) for o in m.opset_import] == [("", 13), ("com.microsoft", 1)]
    assert [n.op_type for n in m.graph.node] == [n.op for n in g.nodes]
    for pn, n in zip(m.graph.node, g.nodes):
        assert pn.name == n.name and list(pn.input) == n.inputs and list(pn.output) == n.outputs
        for a in pn.attribute:
            v = n.attrs[a.name]
            got = {2: a.i, 1: a.f, 3: a.s.decode(), 7: list(a.ints), 6: list(a.floats)}[a.type]
            assert got == (list(v) if isinstance(v, (list, tuple)) else v), (n.name, a.name)
    inits = {t.name: t for t in m.graph.initializer}
    assert set(inits) == set(g.initializers)
    for name, arr in g.initializers.items():
        t = inits[name]
        assert list(t.dims) == list(arr.shape) and t.data_type == G.ONNX_DT[arr.dtype]
        if mode == "raw":
            got = np.frombuffer(t.raw_data, arr.dtype)
        elif arr.dtype == np.float32:
            got = np.array(t.float_data, np.float32)
        elif arr.dtype == np.int64:
            got = np.array(t.int64_data, np.int64)
        else:
            got = np.array(t.int32_data, np.int64).astype(arr.dtype)
        assert np.array_equal(got, arr.reshape(-1)), name
    (inp,) = m.graph.input
    dims = inp.type.tensor_type.shape.dim
    assert dims[0].dim_param == "d0" and [d.dim_value for d in dims[1:]] == [3, 21, 21]


@pytest.mark.parametrize("name", ["qoperator", "resnet50"])
def test_protobuf_serialized_model_loads(name):
    """A ModelProto built and serialized by google.protobuf (packed repeated
    fields, its own field order) loads into the same context."""
    P = _protobuf_classes()
    g = GRAPHS[name]()
    m = P["ModelProto"](ir_version=8)
    m.opset_import.add(domain="", version=13)
    for n in g.nodes:
        pn = m.graph.node.add(name=n.name, op_type=n.op, input=n.inputs, output=n.outputs)
        for k, v in n.attrs.items():
            a = pn.attribute.add(name=k)
            if isinstance(v, str):
                a.s, a.type = v.encode(), 3
            elif isinstance(v, (list, tuple)):
                if all(isinstance(x, (int, np.integer)) for x in v):
                    a.ints.extend(int(x) for x in v)
                    a.type = 7
                else:
                    a.floats.extend(float(x) for x in v)
                    a.type = 6
            elif isinstance(v, (int, np.integer)):
                a.i, a.type = int(v), 2
            else:
                a.f, a.type = float(v), 1
    for k, arr in g.initializers.items():
        m.graph.initializer.add(name=k, dims=arr.shape, data_type=G.ONNX_DT[arr.dtype], raw_data=arr.tobytes())
    for k, (dt, shape) in g.inputs.items():
        vi = m.graph.input.add(name=k)
        vi.type.tensor_type.elem_type = G.ONNX_DT[np.dtype(dt)]
        for d in shape:
            vi.type.tensor_type.shape.dim.add(dim_value=d)
    for k in g.outputs:
        m.graph.output.add(name=k)
    same_context(g, G.Session(None, device=False, onnx=m.SerializeToString()))


@pytest.mark.parametrize("dims", [[65536] * 4, [2**31 - 1] * 3, [2**31 - 1, 2**31 - 1]])
def test_oversized_initializer_dims_fail_cleanly(dims):
    """Dimensions whose element count wraps size_t ([65536]*4 is 2^64, which
    an unchecked product makes 0) or needs more host memory than any model
    holds are a load error with a message, never a crash or an exception
    escaping the C ABI."""
    P = _protobuf_classes()
    m = P["ModelProto"](ir_version=8)
    m.opset_import.add(domain="", version=13)
    m.graph.initializer.add(name="w", dims=dims, data_type=2, raw_data=b"\x01" * 16)
    m.graph.output.add(name="w")
    with pytest.raises(G.NnrError, match="too large"):
        G.Session(None, device=False, onnx=m.SerializeToString())


def test_element_types_use_reference_numbering():
    """The host C ABI takes and returns the reference's data_type_t codes
    (src/nnr.h:20-56: FLOAT32 1, INT8 5, INT32 7, INT64 8, UINT8 9); a model
    file's TensorProto codes (FLOAT 1, UINT8 2, INT8 3, INT32 6) are
    translated by the loader."""
    assert G.NNR_DT == {np.dtype(np.float32): 1, np.dtype(np.float16): 3, np.dtype(np.int8): 5,
                        np.dtype(np.int32): 7, np.dtype(np.int64): 8, np.dtype(np.uint8): 9}
    g = GRAPHS["qoperator"]()
    model, _ = onnx_io.encode(g)
    s = G.Session(None, device=False, onnx=model)
    for name, arr in g.initializers.items():
        assert s.tensor_info(name)[1] == arr.dtype, name
    for name, (dt, _) in g.inputs.items():
        assert s.tensor_info(name)[1] == np.dtype(dt), name


def test_bad_element_type_code_rejected():
    L = G.host_lib()
    import ctypes as C
    h = C.c_void_p()
    G._chk(L.nnr_ctx_create(C.byref(h), 4))
    try:
        dims = (C.c_int * 1)(4)
        data = (C.c_uint8 * 4)()
        for code in (0, 200, -1):
            assert L.nnr_ctx_add_initializer(h, b"t", code, dims, 1, data) != 0
            assert b"data_type_t" in L.nnr_last_error()
        assert L.nnr_ctx_add_initializer(h, b"t", 9, dims, 1, data) == 0
    finally:
        L.nnr_ctx_destroy(h)
