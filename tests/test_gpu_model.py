"""The weight-pack loader (mmnb_model_load) on the GPU.

Real exporter output: the reference's fixture model files (copied as data to
tests/golden/onnx/) load, and every packed node run with the fixture's
inputs reproduces the fixture's outputs (exact for integers, the reference's
rule for floats).  Written models: MatMulNBits with fp16 scales, per-column
uint8 zero points, bias and g_idx, all in an external data file (one entry
with no length field, so the size comes from the shape), and a
MatMulInteger with inline int32_data, against the oracles.  Unsafe or
out-of-range external references and malformed files are rejected.
"""
import numpy as np
import pytest

from oracle import nbits_ex as X
from oracle import refcpu
from onnx_runtime_dart_amd import _lib
from onnx_runtime_dart_amd.model import LoadedModel
from tests import onnx_writer as W
from tests.helpers import GOLDEN, fixture_float_ok, load_golden, node_arg, normwise_rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    return _lib.default_context()


def _range8(z):
    return (-128, 127) if z is not None and np.asarray(z).dtype == np.int8 else (0, 255)


@pytest.mark.parametrize("case", ["matmulnbits_basic", "matmulnbits_zeropoints",
                                  "matmulnbits_partial_block", "matmulinteger_u8i8",
                                  "matmulinteger_percol_bzp", "qlinearmatmul", "convinteger",
                                  "convinteger_1d", "qlinearconv_perchannel_bias"])
def test_reference_fixture_models(ctx, case):
    d, vals, exp = load_golden(case)
    mdl = LoadedModel(GOLDEN / "onnx" / f"{case}.onnx", ctx)
    try:
        assert len(mdl.nodes) == 1
        name = next(iter(mdl.nodes))
        ins = [node_arg(d, vals, i) for i in range(len(d["node_inputs"]))]
        at = d["attrs"]
        op = d["op_type"]
        assert mdl.op_type(name) == op
        if op == "MatMulNBits":
            y = mdl.matmul_nbits(name, ins[0])
            ok, max_abs, cos = fixture_float_ok(y, exp["out0"])
            assert ok, (max_abs, cos)
            return
        if op == "MatMulInteger":
            y = mdl.matmul_integer(name, ins[0], ins[2] if len(ins) > 2 else None)
        elif op == "QLinearMatMul":
            lo, hi = _range8(ins[7])
            y = mdl.qlinear_matmul(name, ins[0], ins[1], ins[2], ins[4], ins[6], ins[7],
                                   lo=lo, hi=hi)
        elif op == "ConvInteger":
            y = mdl.conv_integer(name, ins[0], ins[2], strides=at.get("strides"),
                                 pads=at.get("pads"), dilations=at.get("dilations"))
        else:
            lo, hi = _range8(ins[7])
            y = mdl.qlinear_conv(name, ins[0], ins[1], ins[2], ins[4], ins[6], ins[7],
                                 ins[8] if len(ins) > 8 else None, lo=lo, hi=hi,
                                 strides=at.get("strides"), pads=at.get("pads"),
                                 dilations=at.get("dilations"))
        np.testing.assert_array_equal(y, exp["out0"].astype(np.int64))
    finally:
        mdl.free()


def _nbits_model(tmp_path, rng, k, n, bs):
    nb = k // bs
    b = rng.integers(0, 256, (n, nb, bs // 2)).astype(np.uint8)
    s = rng.uniform(0.002, 0.02, (n, nb)).astype(np.float16)
    z = rng.integers(0, 256, (n, (nb + 1) // 2)).astype(np.uint8)
    g = rng.permutation(np.repeat(np.arange(nb), bs)).astype(np.int32)
    bias = rng.standard_normal(n).astype(np.float32)
    bi = rng.integers(-127, 128, (k, 48)).astype(np.int8)
    ext = W.ExternalFile("weights/w.bin")
    loc_b = ext.add(b)
    loc_s = ext.add(s)
    loc_z = ext.add(z)
    loc_g = ext.add(g)
    loc_bias = ext.add(bias)
    inits = [W.tensor("B", b, "external", loc_b),
             W.tensor("S", s, "external", (loc_s[0], loc_s[1], None)),   # length from shape
             W.tensor("Z", z, "external", loc_z),
             W.tensor("G", g, "external", loc_g),
             W.tensor("BIAS", bias, "external", loc_bias),
             W.tensor("Bi", bi, "inline"),
             W.tensor("Bz", np.int8(3), "inline")]
    nodes = [W.node("MatMulNBits", ["A", "B", "S", "Z", "G", "BIAS"], ["Y"], name="proj",
                    domain="com.microsoft", K=k, N=n, bits=4, block_size=bs),
             W.node("MatMulInteger", ["Aq", "Bi", "", "Bz"], ["Yi"])]
    (tmp_path / "weights").mkdir()
    (tmp_path / "weights" / "w.bin").write_bytes(bytes(ext.data))
    path = tmp_path / "model.onnx"
    path.write_bytes(W.model(nodes, inits))
    return path, (b, s, z, g, bias, bi)


def test_written_model_with_external_data(ctx, tmp_path):
    rng = np.random.default_rng(1)
    k, n, bs = 512, 96, 64
    path, (b, s, z, g, bias, bi) = _nbits_model(tmp_path, rng, k, n, bs)
    mdl = LoadedModel(path, ctx)
    try:
        assert set(mdl.nodes) == {"proj", "Yi"}
        a = rng.standard_normal((3, k)).astype(np.float32)
        y = mdl.matmul_nbits("proj", a)
        ref = X.matmul_nbits_ex(a, b, s, z, g, bias, k, n, 4, bs)
        assert normwise_rel_err(y, ref) <= 1e-5
        aq = rng.integers(0, 256, (5, k)).astype(np.uint8)
        yi = mdl.matmul_integer("Yi", aq, np.uint8(128))
        want = refcpu.matmul_integer(aq, bi, np.uint8(128), np.int8(3))
        np.testing.assert_array_equal(yi, want)
    finally:
        mdl.free()


@pytest.mark.parametrize("loc,off,ln", [("../w.bin", 0, 16), ("/etc/hostname", 0, 16),
                                        ("w.bin", 64, 1 << 20), ("w.bin", -1, 16)])
def test_unsafe_or_out_of_range_external_data_rejects(ctx, tmp_path, loc, off, ln):
    (tmp_path / "w.bin").write_bytes(b"\0" * 256)
    b = np.zeros((4, 1, 16), np.uint8)
    s = np.ones((4, 1), np.float32)
    inits = [W.tensor("B", b, "external", (loc, off, ln)), W.tensor("S", s)]
    nodes = [W.node("MatMulNBits", ["A", "B", "S"], ["Y"], K=32, N=4, bits=4, block_size=32)]
    path = tmp_path / "m.onnx"
    path.write_bytes(W.model(nodes, inits))
    with pytest.raises(ValueError):
        LoadedModel(path, ctx)


def test_malformed_file_rejects(ctx, tmp_path):
    path = tmp_path / "bad.onnx"
    path.write_bytes(b"\x3a\xff\xff\xff\xff\x0f garbage")
    with pytest.raises(ValueError):
        LoadedModel(path, ctx)


@pytest.mark.parametrize("which,arr", [
    ("scales", np.ones((4, 1), np.uint8)),            # 1 byte per value, read as floats
    ("scales", np.ones((4, 1), np.int32)),
    ("zero_points", np.full((4, 1), 8, np.int8)),
    ("bias", np.zeros(4, np.int32)),
])
def test_wrong_initializer_types_are_unsupported(ctx, tmp_path, which, arr):
    # Scales, bias and float zero points must be float / float16 and packed
    # zero points uint8: another type is rejected before anything reads its
    # bytes with the wrong element size.
    b = np.zeros((4, 1, 16), np.uint8)
    ins = {"scales": np.ones((4, 1), np.float32), "zero_points": None, "bias": None}
    ins[which] = arr
    inits = [W.tensor("B", b), W.tensor("S", ins["scales"])]
    names = ["A", "B", "S"]
    if ins["zero_points"] is not None or ins["bias"] is not None:
        names.append("Z" if ins["zero_points"] is not None else "")
        if ins["zero_points"] is not None:
            inits.append(W.tensor("Z", ins["zero_points"]))
    if ins["bias"] is not None:
        names += ["", "BIAS"]
        inits.append(W.tensor("BIAS", ins["bias"]))
    nodes = [W.node("MatMulNBits", names, ["Y"], K=32, N=4, bits=4, block_size=32)]
    path = tmp_path / "m.onnx"
    path.write_bytes(W.model(nodes, inits))
    with pytest.raises(NotImplementedError):
        LoadedModel(path, ctx)


@pytest.mark.parametrize("op", ["MatMulInteger", "ConvInteger"])
def test_integer_op_zero_point_must_be_8_bit(ctx, tmp_path, op):
    if op == "MatMulInteger":
        w = np.zeros((16, 8), np.int8)
        zp = np.zeros(8, np.int32)
    else:
        w = np.zeros((4, 2, 3, 3), np.int8)
        zp = np.zeros(4, np.int32)
    inits = [W.tensor("W", w), W.tensor("Z", zp)]
    nodes = [W.node(op, ["X", "W", "", "Z"], ["Y"])]
    path = tmp_path / "m.onnx"
    path.write_bytes(W.model(nodes, inits))
    with pytest.raises(NotImplementedError):
        LoadedModel(path, ctx)
