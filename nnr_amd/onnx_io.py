"""ONNX ModelProto writer for `Graph` (the in-process graph description).

Writes the subset of the ONNX protobuf schema that the loader
(nnr_amd/host/onnx_loader.cpp, include/nnr_host.h `nnr_ctx_load_onnx`) reads:
ModelProto (ir_version, opset_import, graph), GraphProto (node, initializer,
input, output), NodeProto, AttributeProto, TensorProto (raw_data or the typed
fields, external data), ValueInfoProto / TypeProto / TensorShapeProto. The
field numbers are the ONNX schema's (onnx.proto3); `FIELDS` lists them.

Use: `save(graph, path)` writes a .onnx file (optionally with initializers
in an external-data file beside it); `encode(graph)` returns the bytes.
"""
from __future__ import annotations

import os
import struct

import numpy as np

from .graph import ONNX_DT, Graph

# ONNX schema field numbers of the messages written here (onnx.proto3)
FIELDS = {
    "ModelProto": {"ir_version": 1, "producer_name": 2, "graph": 7, "opset_import": 8},
    "OperatorSetIdProto": {"domain": 1, "version": 2},
    "GraphProto": {"node": 1, "name": 2, "initializer": 5, "input": 11, "output": 12},
    "NodeProto": {"input": 1, "output": 2, "name": 3, "op_type": 4, "attribute": 5, "domain": 7},
    "AttributeProto": {"name": 1, "f": 2, "i": 3, "s": 4, "t": 5, "floats": 7, "ints": 8,
                       "strings": 9, "type": 20},
    "TensorProto": {"dims": 1, "data_type": 2, "float_data": 4, "int32_data": 5, "int64_data": 7,
                    "name": 8, "raw_data": 9, "external_data": 13, "data_location": 14},
    "StringStringEntryProto": {"key": 1, "value": 2},
    "ValueInfoProto": {"name": 1, "type": 2},
    "TypeProto": {"tensor_type": 1},
    "TypeProto.Tensor": {"elem_type": 1, "shape": 2},
    "TensorShapeProto": {"dim": 1},
    "TensorShapeProto.Dimension": {"dim_value": 1, "dim_param": 2},
}
# AttributeProto.AttributeType
ATTR_FLOAT, ATTR_INT, ATTR_STRING, ATTR_TENSOR, ATTR_FLOATS, ATTR_INTS = 1, 2, 3, 4, 6, 7
# operators of the com.microsoft domain (ONNX Runtime contrib ops)
MS_OPS = {"QLinearConcat", "QLinearGlobalAveragePool", "QLinearAveragePool", "QLinearMul",
          "QLinearAdd", "MultiHeadAttention"}


def _varint(v: int) -> bytes:
    v &= (1 << 64) - 1          # negative int64 as ten-byte two's complement
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def _key(field: int, wt: int) -> bytes:
    return _varint((field << 3) | wt)


def _ld(field: int, payload: bytes) -> bytes:
    return _key(field, 2) + _varint(len(payload)) + payload


def _str(field: int, s: str | bytes) -> bytes:
    return _ld(field, s.encode() if isinstance(s, str) else s)


def _int(field: int, v: int) -> bytes:
    return _key(field, 0) + _varint(int(v))


def _f32(field: int, v: float) -> bytes:
    return _key(field, 5) + struct.pack("<f", v)


def _rep_ints(field: int, vals, packed: bool) -> bytes:
    vals = [int(x) for x in vals]
    if not vals:
        return b""
    if packed:
        return _ld(field, b"".join(_varint(x) for x in vals))
    return b"".join(_int(field, x) for x in vals)


def _rep_f32(field: int, vals, packed: bool) -> bytes:
    vals = [float(x) for x in vals]
    if not vals:
        return b""
    if packed:
        return _ld(field, struct.pack(f"<{len(vals)}f", *vals))
    return b"".join(_f32(field, x) for x in vals)


def _tensor(name: str, arr: np.ndarray, mode: str, packed: bool, external=None) -> bytes:
    """mode 'raw': raw_data; 'typed': float_data / int32_data / int64_data.
    external: (location, offset) -> data_location EXTERNAL."""
    F = FIELDS["TensorProto"]
    a = np.ascontiguousarray(arr)
    out = _rep_ints(F["dims"], a.shape, packed) + _int(F["data_type"], ONNX_DT[a.dtype]) + _str(F["name"], name)
    if external is not None:
        loc, off = external
        kv = FIELDS["StringStringEntryProto"]
        for k, v in (("location", loc), ("offset", str(off)), ("length", str(a.nbytes))):
            out += _ld(F["external_data"], _str(kv["key"], k) + _str(kv["value"], v))
        return out + _int(F["data_location"], 1)
    if mode == "raw":
        return out + _ld(F["raw_data"], a.astype(a.dtype.newbyteorder("<"), copy=False).tobytes())
    flat = a.reshape(-1)
    if a.dtype == np.float32:
        return out + _rep_f32(F["float_data"], flat, packed)
    if a.dtype == np.int64:
        return out + _rep_ints(F["int64_data"], flat, packed)
    if a.dtype == np.float16:     # bit patterns, one per int32 element
        return out + _rep_ints(F["int32_data"], flat.view(np.uint16), packed)
    return out + _rep_ints(F["int32_data"], flat, packed)   # int32 / uint8 / int8


def _attr(name: str, v, packed: bool) -> bytes:
    """Python value -> AttributeProto, with the type inference Session uses."""
    F = FIELDS["AttributeProto"]
    out = _str(F["name"], name)
    if isinstance(v, str):
        return out + _str(F["s"], v) + _int(F["type"], ATTR_STRING)
    if isinstance(v, (list, tuple, np.ndarray)):
        vals = list(v)
        if all(isinstance(x, (int, np.integer)) for x in vals):
            return out + _rep_ints(F["ints"], vals, packed) + _int(F["type"], ATTR_INTS)
        return out + _rep_f32(F["floats"], vals, packed) + _int(F["type"], ATTR_FLOATS)
    if isinstance(v, (int, np.integer)):
        return out + _int(F["i"], v) + _int(F["type"], ATTR_INT)
    return out + _f32(F["f"], float(v)) + _int(F["type"], ATTR_FLOAT)


def _value_info(name: str, dtype, shape, sym_dims=()) -> bytes:
    D = FIELDS["TensorShapeProto.Dimension"]
    dims = b"".join(_ld(FIELDS["TensorShapeProto"]["dim"],
                        _str(D["dim_param"], f"d{i}") if i in sym_dims else _int(D["dim_value"], d))
                    for i, d in enumerate(shape))
    T = FIELDS["TypeProto.Tensor"]
    tt = _int(T["elem_type"], ONNX_DT[np.dtype(dtype)])
    if shape is not None:
        tt += _ld(T["shape"], dims)
    V = FIELDS["ValueInfoProto"]
    return _str(V["name"], name) + _ld(V["type"], _ld(FIELDS["TypeProto"]["tensor_type"], tt))


def encode(g: Graph, opset: int = 13, ir_version: int = 8, mode: str = "raw", packed: bool = True,
           sym_dims=(), external: str | None = None, external_min_bytes: int = 1024,
           constants=()) -> tuple[bytes, bytes]:
    """Graph -> (ModelProto bytes, external-data bytes).

    mode: 'raw' or 'typed' initializer payloads; packed: packed repeated
    scalars (proto3's default) or one record per value; sym_dims: input
    dimension indices written as symbolic (dim_param); external: the
    external-data file name (initializers of at least external_min_bytes go
    there, 64-byte aligned); constants: initializer names written as
    Constant nodes instead."""
    N = FIELDS["NodeProto"]
    G = FIELDS["GraphProto"]
    ext = bytearray()
    body = b""
    const_nodes = b""
    for name, arr in g.initializers.items():
        if name in constants:
            attr = (_str(FIELDS["AttributeProto"]["name"], "value")
                    + _ld(FIELDS["AttributeProto"]["t"], _tensor(name, arr, mode, packed))
                    + _int(FIELDS["AttributeProto"]["type"], ATTR_TENSOR))
            const_nodes += _ld(G["node"], _str(N["output"], name) + _str(N["name"], name + "_const")
                               + _str(N["op_type"], "Constant") + _ld(N["attribute"], attr))
            continue
        loc = None
        if external is not None and arr.nbytes >= external_min_bytes:
            off = (len(ext) + 63) & ~63
            ext.extend(b"\0" * (off - len(ext)))
            ext.extend(np.ascontiguousarray(arr).tobytes())
            loc = (external, off)
        body += _ld(G["initializer"], _tensor(name, arr, mode, packed, loc))
    nodes = const_nodes
    for nd in g.nodes:
        n = b"".join(_str(N["input"], s or "") for s in nd.inputs)
        n += b"".join(_str(N["output"], s) for s in nd.outputs)
        n += _str(N["name"], nd.name) + _str(N["op_type"], nd.op)
        n += b"".join(_ld(N["attribute"], _attr(k, v, packed)) for k, v in nd.attrs.items())
        if nd.op in MS_OPS:
            n += _str(N["domain"], "com.microsoft")
        nodes += _ld(G["node"], n)
    graph = nodes + _str(G["name"], "nnr_amd") + body
    for name, (dt, shape) in g.inputs.items():
        graph += _ld(G["input"], _value_info(name, dt, shape, sym_dims))
    for name in g.outputs:
        vi = _str(FIELDS["ValueInfoProto"]["name"], name)
        graph += _ld(G["output"], vi)
    M = FIELDS["ModelProto"]
    O = FIELDS["OperatorSetIdProto"]
    model = (_int(M["ir_version"], ir_version) + _str(M["producer_name"], "nnr_amd")
             + _ld(M["graph"], graph)
             + _ld(M["opset_import"], _str(O["domain"], "") + _int(O["version"], opset))
             + _ld(M["opset_import"], _str(O["domain"], "com.microsoft") + _int(O["version"], 1)))
    return model, bytes(ext)


def save(g: Graph, path: str, external_data: bool = False, **kw) -> None:
    """Write `g` as an ONNX file; with external_data the large initializers
    go to `<file name>.data` beside it."""
    ext_name = os.path.basename(path) + ".data" if external_data else None
    model, ext = encode(g, external=ext_name, **kw)
    with open(path, "wb") as f:
        f.write(model)
    if ext_name:
        with open(os.path.join(os.path.dirname(os.path.abspath(path)), ext_name), "wb") as f:
            f.write(ext)
