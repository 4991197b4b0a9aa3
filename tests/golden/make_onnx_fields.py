"""Writes onnx_fields.json: the field numbers, scalar types and labels of the
ONNX schema messages the loader reads and the writer emits, taken from the
reference's copy of the schema (src/format/onnx/onnx.proto3). The JSON is an
interface table (the public ONNX protobuf schema); tests compare
nnr_amd/onnx_io.FIELDS with it and build google.protobuf message classes
from it, so the writer and the C++ reader are checked against a protobuf
implementation that is not this project's.

Run from the repository root:  python tests/golden/make_onnx_fields.py
"""
import json
import os
import re
import sys

SRC = "/root/reference/src/format/onnx/onnx.proto3"
WANT = {"ModelProto", "OperatorSetIdProto", "GraphProto", "NodeProto", "AttributeProto", "TensorProto",
        "StringStringEntryProto", "ValueInfoProto", "TypeProto", "TypeProto.Tensor", "TensorShapeProto",
        "TensorShapeProto.Dimension"}


def parse(text):
    msgs, stack = {}, []
    depth_of = []          # brace depth at which each open message started
    depth = 0
    for raw in text.splitlines():
        line = raw.split("//")[0].strip()
        if not line:
            continue
        m = re.match(r"(message|enum|oneof)\s+(\w+)\s*\{", line)
        if m:
            depth += 1
            if m.group(1) == "message":
                stack.append(m.group(2))
                depth_of.append(depth)
                msgs.setdefault(".".join(stack), {})
            continue
        f = re.match(r"(repeated\s+)?([\w.]+)\s+(\w+)\s*=\s*(\d+)\s*(\[.*\])?\s*;", line)
        if f and stack and not line.startswith(("reserved", "option")):
            label = "repeated" if f.group(1) else "optional"
            msgs[".".join(stack)][f.group(3)] = [int(f.group(4)), f.group(2), label]
        depth += line.count("{") - line.count("}") if not m else 0
        while depth_of and depth < depth_of[-1]:
            depth_of.pop()
            stack.pop()
    return msgs


def main():
    msgs = parse(open(SRC).read())
    out = {k: msgs[k] for k in sorted(WANT)}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "onnx_fields.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
    print(path, sum(len(v) for v in out.values()), "fields", file=sys.stderr)


if __name__ == "__main__":
    main()
