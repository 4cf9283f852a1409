#!/usr/bin/env python3
"""Extract the reference's hot-path golden vectors into self-contained JSON.

Reads ``test/fixtures/<case>/{model.onnx,case.json}`` from the reference
source tree (default ``/root/reference``) for the eight fixtures that pin the
int4 ``MatMulNBits`` and int8 ``DynamicQuantizeLinear``/``MatMulInteger``
path, and the six that pin the decoder ops around it (RMSNorm chain,
``RotaryEmbedding``, ``GroupQueryAttention`` with and without KV cache,
rotary and bias), decodes the initializers and node attributes out of ``model.onnx`` with
a minimal protobuf wire-format reader (no ``onnx`` package needed), and writes
``tests/golden/<case>.json`` (and, for the loader tests, copies a few
``model.onnx`` files to ``tests/golden/onnx/<case>.onnx``).  The fixtures are data: the inputs the
reference's ORT-oracle fixture test feeds (``test/fixture_parity_test.dart``)
and the outputs native onnxruntime produced for them
(``tool/gen_fixtures.py:59-102``, ``:690-693``, ``:713-735``, ``:892-925``).

Run once in a tree that has the reference mounted:

    python tests/golden/extract_fixtures.py [--ref /root/reference]
"""
import argparse
import json
import struct
from pathlib import Path

CASES = [
    "matmulnbits_basic",
    "matmulnbits_zeropoints",
    "matmulnbits_partial_block",
    "dynamicquantizelinear",
    "matmulinteger_u8i8",
    "matmulinteger_nozp",
    "matmulinteger_batched",
    "matmulinteger_percol_bzp",
    # decoder ops (RMSNorm 7-node chain, rotary, grouped-query attention)
    "rmsnorm_pattern",
    "rotary_embedding",
    "gqa_causal",
    "gqa_kvcache",
    "gqa_kvcache_rotary",
    "gqa_kvcache_bias",
    # quantized ops adjacent to the path (QLinearMatMul, ConvInteger 2-D and
    # 1-D, QLinearConv per-tensor and per-channel with bias)
    "qlinearmatmul",
    "convinteger",
    "convinteger_1d",
    "qlinearconv_pertensor",
    "qlinearconv_perchannel_bias",
]

# Fixtures whose model.onnx is also kept (tests/golden/onnx/), as real
# exporter output for the weight-pack loader.
ONNX_FILES = {"matmulnbits_basic", "matmulnbits_zeropoints", "matmulnbits_partial_block",
              "matmulinteger_u8i8", "matmulinteger_percol_bzp", "qlinearmatmul",
              "convinteger", "convinteger_1d", "qlinearconv_perchannel_bias"}

# ONNX TensorProto.DataType codes used by these fixtures.
DTYPES = {1: ("float32", "<f", 4), 2: ("uint8", "<B", 1), 3: ("int8", "<b", 1),
          6: ("int32", "<i", 4), 7: ("int64", "<q", 8)}


def _varint(buf, pos):
    shift = result = 0
    while True:
        b = buf[pos]
        pos += 1
        result |= (b & 0x7F) << shift
        if not b & 0x80:
            return result, pos
        shift += 7


def fields(buf):
    """Yield (field_number, wire_type, value) for one protobuf message."""
    pos = 0
    while pos < len(buf):
        key, pos = _varint(buf, pos)
        fno, wt = key >> 3, key & 7
        if wt == 0:
            val, pos = _varint(buf, pos)
        elif wt == 1:
            val = buf[pos:pos + 8]
            pos += 8
        elif wt == 2:
            ln, pos = _varint(buf, pos)
            val = buf[pos:pos + ln]
            pos += ln
        elif wt == 5:
            val = buf[pos:pos + 4]
            pos += 4
        else:
            raise ValueError(f"unsupported wire type {wt}")
        yield fno, wt, val


def _packed_varints(val, wt):
    if wt == 0:
        return [val]
    out, pos = [], 0
    while pos < len(val):
        v, pos = _varint(val, pos)
        out.append(v)
    return out


def decode_tensor(buf):
    """TensorProto: dims=1, data_type=2, float_data=4, int32_data=5,
    int64_data=7, name=8, raw_data=9."""
    dims, dt, name, raw = [], None, "", None
    floats, ints32, ints64 = [], [], []
    for fno, wt, val in fields(buf):
        if fno == 1:
            dims += _packed_varints(val, wt)
        elif fno == 2:
            dt = val
        elif fno == 8:
            name = val.decode()
        elif fno == 9:
            raw = bytes(val)
        elif fno == 4:
            if wt == 5:
                floats.append(struct.unpack("<f", val)[0])
            else:
                floats += list(struct.unpack(f"<{len(val)//4}f", val))
        elif fno == 5:
            ints32 += _packed_varints(val, wt)
        elif fno == 7:
            ints64 += _packed_varints(val, wt)
    dname, fmt, size = DTYPES[dt]
    n = 1
    for d in dims:
        n *= d
    if raw is not None:
        data = list(struct.unpack("<" + fmt[1] * n, raw[:n * size]))
    elif dname == "float32":
        data = floats
    elif dname == "int64":
        data = [v - (1 << 64) if v >= (1 << 63) else v for v in ints64]
    else:
        # int32_data carries uint8/int8/int32 as varints (sign-extended int32)
        data = [v - (1 << 64) if v >= (1 << 63) else v for v in ints32]
    return name, {"dtype": dname, "shape": dims, "data": data}


def decode_attribute(buf):
    """AttributeProto: name=1, f=2, i=3, ints=8, type=20."""
    name, value, ints = "", None, None
    for fno, wt, val in fields(buf):
        if fno == 1:
            name = val.decode()
        elif fno == 3:
            value = val - (1 << 64) if val >= (1 << 63) else val
        elif fno == 2:
            value = struct.unpack("<f", val)[0]
        elif fno == 8:  # repeated int64, packed or not
            ints = (ints or []) + [v - (1 << 64) if v >= (1 << 63) else v
                                   for v in _packed_varints(val, wt)]
    return name, (ints if ints is not None else value)


def decode_node(buf):
    """NodeProto: input=1, output=2, name=3, op_type=4, attribute=5,
    domain=7."""
    node = {"inputs": [], "outputs": [], "op_type": "", "domain": "",
            "attrs": {}}
    for fno, _wt, val in fields(buf):
        if fno == 1:
            node["inputs"].append(val.decode())
        elif fno == 2:
            node["outputs"].append(val.decode())
        elif fno == 4:
            node["op_type"] = val.decode()
        elif fno == 7:
            node["domain"] = val.decode()
        elif fno == 5:
            k, v = decode_attribute(val)
            node["attrs"][k] = v
    return node


def decode_model(buf):
    """ModelProto.graph=7; GraphProto: node=1, initializer=5."""
    graph = None
    for fno, _wt, val in fields(buf):
        if fno == 7:
            graph = val
    nodes, inits = [], {}
    for fno, _wt, val in fields(graph):
        if fno == 1:
            nodes.append(decode_node(val))
        elif fno == 5:
            name, t = decode_tensor(val)
            inits[name] = t
    return nodes, inits


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    args = ap.parse_args()
    src = Path(args.ref) / "test" / "fixtures"
    dst = Path(__file__).resolve().parent
    for case in CASES:
        d = src / case
        nodes, inits = decode_model((d / "model.onnx").read_bytes())
        cj = json.loads((d / "case.json").read_text())
        out = {
            "provenance": f"onnx_runtime_dart test/fixtures/{case} "
                          "(ORT CPU outputs, tool/gen_fixtures.py seed 42)",
            "op_type": nodes[0]["op_type"],
            "domain": nodes[0]["domain"],
            "node_inputs": nodes[0]["inputs"],
            "attrs": nodes[0]["attrs"],
            "initializers": inits,
            "inputs": cj["inputs"],
            "expected": cj["expected"],
        }
        if len(nodes) > 1:  # a multi-node pattern (the RMSNorm chain)
            out["nodes"] = nodes
        (dst / f"{case}.json").write_text(json.dumps(out, indent=None) + "\n")
        if case in ONNX_FILES:  # the model file itself, for the weight loader
            (dst / "onnx").mkdir(exist_ok=True)
            (dst / "onnx" / f"{case}.onnx").write_bytes((d / "model.onnx").read_bytes())
        print(case, nodes[0]["op_type"], nodes[0]["attrs"],
              {k: v["shape"] for k, v in inits.items()})


if __name__ == "__main__":
    main()
