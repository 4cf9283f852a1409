"""Reader robustness of the host input code (CPU): the ONNX wire reader and
pack planner and the MatMulNBits host preparation
(onnx_runtime_dart_amd/csrc/mmnb_host.cpp) built with g++ under
AddressSanitizer + UBSan, driven by tests/fuzz/onnx_reader_fuzz.cpp.

The contract is the reference's (tool/fuzz/README.md:1-17,
test/parser_robustness_test.dart): any input parses or is rejected with a
documented status (MMNB_ERR_ARG / MMNB_ERR_UNSUPPORTED), with no read
outside the input, no allocation bomb (ASan's allocation cap) and no hang.
Seeds: the reference's fixture models (tests/golden/onnx) and written models
that reach every plan kind and every MatMulNBits extension, with external
data in companion files; each fuzz input is a seed after 1-4 mutations.
"""
import os
import re
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from tests import onnx_writer as W
from tests.helpers import GOLDEN

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "onnx_runtime_dart_amd" / "csrc"
HARNESS = ROOT / "tests" / "fuzz" / "onnx_reader_fuzz.cpp"
ENV = {"ASAN_OPTIONS": "max_allocation_size_mb=256:allocator_may_return_null=0:"
                       "detect_leaks=1:abort_on_error=0",
       "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}


@pytest.fixture(scope="module")
def fuzzer(tmp_path_factory):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ not available")
    out = tmp_path_factory.mktemp("fuzz") / "onnx_reader_fuzz"
    cmd = [cxx, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-I", str(CSRC),
           str(HARNESS), str(CSRC / "mmnb_host.cpp"), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return out


def _seed_models(d, rng):
    """Small written models covering every plan kind and extension."""
    (d / "w").mkdir()
    k, n, bs = 128, 24, 32
    nb = k // bs
    b4 = rng.integers(0, 256, (n, nb, bs // 2)).astype(np.uint8)
    s16 = rng.uniform(0.002, 0.02, (n, nb)).astype(np.float16)
    s32 = s16.astype(np.float32)
    zpc = rng.integers(0, 256, (n, (nb + 1) // 2)).astype(np.uint8)
    zfl = rng.integers(0, 256, ((n * nb + 1) // 2,)).astype(np.uint8)
    zf = rng.uniform(0, 15, (n, nb)).astype(np.float32)
    g = rng.permutation(np.repeat(np.arange(nb), bs)).astype(np.int32)
    bias = rng.standard_normal(n).astype(np.float32)
    b8 = rng.integers(0, 256, (n, nb, bs)).astype(np.uint8)
    z8 = rng.integers(0, 256, (n * nb,)).astype(np.uint8)
    bi = rng.integers(-127, 128, (2, k, 16)).astype(np.int8)
    wc = rng.integers(0, 256, (8, 4, 3, 3)).astype(np.uint8)
    ext = W.ExternalFile("w/w.bin")
    nbits = dict(domain="com.microsoft", K=k, N=n, block_size=bs)
    models = {
        # all extensions from external data (S with no length field)
        "nbits_ext.onnx": ([W.node("MatMulNBits", ["A", "B", "S", "Z", "G", "BIAS"], ["Y"],
                                   name="p", bits=4, **nbits)],
                           [W.tensor("B", b4, "external", ext.add(b4)),
                            W.tensor("S", s16, "external", ext.add(s16)[:2] + (None,)),
                            W.tensor("Z", zpc, "external", ext.add(zpc)),
                            W.tensor("G", g, "external", ext.add(g)),
                            W.tensor("BIAS", bias, "external", ext.add(bias))]),
        "nbits_flat_zp.onnx": ([W.node("MatMulNBits", ["A", "B", "S", "Z"], ["Y"], bits=4,
                                       **nbits)],
                               [W.tensor("B", b4), W.tensor("S", s32, "inline"),
                                W.tensor("Z", zfl)]),
        "nbits_float_zp.onnx": ([W.node("MatMulNBits", ["A", "B", "S", "Z", "", "BIAS"], ["Y"],
                                        bits=4, **nbits)],
                                [W.tensor("B", b4), W.tensor("S", s16, "inline"),
                                 W.tensor("Z", zf), W.tensor("BIAS", bias.astype(np.float16))]),
        "nbits_8bit.onnx": ([W.node("MatMulNBits", ["A", "B", "S", "Z"], ["Y"], bits=8,
                                    **nbits)],
                            [W.tensor("B", b8), W.tensor("S", s32), W.tensor("Z", z8)]),
        "integer.onnx": ([W.node("MatMulInteger", ["A", "Bi", "", "Bz"], ["Yi"]),
                          W.node("QLinearMatMul", ["a", "as", "az", "Bi", "bs", "Bz", "ys", "yz"],
                                 ["Yq"]),
                          W.node("ConvInteger", ["X", "Wc", "", "Wz"], ["Yc"], group=2),
                          W.node("QLinearConv", ["x", "xs", "xz", "Wc", "ws", "Wz", "ys", "yz"],
                                 ["Yqc"])],
                         [W.tensor("Bi", bi, "inline"), W.tensor("Bz", np.int8(3), "inline"),
                          W.tensor("Wc", wc, "external", ext.add(wc)),
                          W.tensor("Wz", np.full(8, 7, np.uint8))]),
    }
    for name, (nodes, inits) in models.items():
        (d / name).write_bytes(W.model(nodes, inits))
    (d / "w" / "w.bin").write_bytes(bytes(ext.data))
    for f in (GOLDEN / "onnx").glob("*.onnx"):
        shutil.copy(f, d / ("golden_" + f.name))


CODES = [1, 2, 3, 6, 7, 10, 0, 5, 11, 16, 1 << 40]   # TensorProto.DataType, valid and not
DIMS = [0, 1, 2, 3, 7, 16, 24, 32, 128, 4096, 1 << 31, 1 << 40, (1 << 64) - 1]


def _tensor_any(rng, name, ext):
    """A TensorProto with a random type, shape and payload that need not
    agree with each other (raw, inline, external or none)."""
    dims = [int(rng.choice(DIMS)) for _ in range(int(rng.integers(0, 5)))]
    out = W.f_packed(1, dims) + W.f_varint(2, int(rng.choice(CODES))) + W.f_bytes(8, name)
    mode = int(rng.integers(0, 5))
    nbytes = int(rng.choice([0, 1, 7, 64, 300, 4096]))
    if mode == 0:
        out += W.f_bytes(9, rng.integers(0, 256, nbytes).astype(np.uint8).tobytes())
    elif mode == 1:
        out += W.f_packed(5, rng.integers(-300, 300, nbytes // 8))
    elif mode == 2:
        out += W.f_bytes(4, rng.standard_normal(nbytes // 4).astype(np.float32).tobytes())
    elif mode == 3:
        loc = str(rng.choice(["w/w.bin", "w/none.bin", "../w.bin", "/etc/passwd", "", "w"]))
        off = str(rng.choice(["0", "64", "-1", "99999999999", "x", "18446744073709551616"]))
        ln = rng.choice([None, "0", "16", "4096", "-5", "1099511627776"])
        for key, val in (("location", loc), ("offset", off), ("length", ln)):
            if val is not None:
                out += W.f_bytes(13, W.f_bytes(1, key) + W.f_bytes(2, str(val)))
        out += W.f_varint(14, 1)
    return out


def _variants(d, rng, count):
    """Models whose nodes take initializers of random type, shape, payload
    and attributes: the planner's checks and the host preparation, beyond
    what byte mutations of consistent seeds reach."""
    ops = [("MatMulNBits", 6, 1), ("MatMulInteger", 4, 1), ("QLinearMatMul", 8, 3),
           ("ConvInteger", 4, 1), ("QLinearConv", 8, 3)]
    attr_vals = [0, 1, 2, 4, 8, 16, 32, 64, 128, 3, 24, 4096, 1 << 31, 1 << 40, -1]
    for i in range(count):
        op, nin, wi = ops[int(rng.integers(0, len(ops)))]
        names = [f"t{j}" if rng.random() < 0.8 else "" for j in range(nin)]
        names[wi] = "t%d" % wi
        attrs = {}
        for a in ("K", "N", "bits", "block_size", "group"):
            if rng.random() < 0.7:
                attrs[a] = int(rng.choice(attr_vals))
        nodes = [W.node(op, names, ["y"], **attrs)]
        inits = [_tensor_any(rng, nm, None) for nm in names if nm]
        (d / f"variant_{i:04d}.onnx.v").write_bytes(W.model(nodes, inits))


def _run(fuzzer, d, iters, seed):
    env = dict(os.environ, **ENV)
    r = subprocess.run([str(fuzzer), str(d), str(iters), str(seed)], capture_output=True,
                       text=True, env=env, timeout=600)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
    m = re.search(r"seeds (\d+) \(plans nbits (\d+) integer (\d+) conv (\d+)\) variants \d+ "
                  r"inputs (\d+): ok (\d+), ERR_ARG (\d+), ERR_UNSUPPORTED (\d+), plans (\d+), "
                  r"max ([\d.]+) ms, violations (\d+)", out)
    assert m, out[-2000:]
    return [float(x) for x in m.groups()]


def test_seeds_load_and_reach_every_plan_kind(fuzzer, tmp_path):
    _seed_models(tmp_path, np.random.default_rng(0))
    seeds, p_nbits, p_int, p_conv, inputs, ok, arg, uns, plans, max_ms, viol = \
        _run(fuzzer, tmp_path, 0, 1)
    assert seeds == 5 + len(list((GOLDEN / "onnx").glob("*.onnx")))
    assert p_nbits >= 7 and p_int >= 4 and p_conv >= 4
    assert viol == 0


@pytest.mark.parametrize("seed", [1, 2])
def test_mutated_models_parse_or_clean_reject(fuzzer, tmp_path, seed):
    rng = np.random.default_rng(seed)
    _seed_models(tmp_path, rng)
    _variants(tmp_path, rng, 400)
    seeds, _, _, _, inputs, ok, arg, uns, plans, max_ms, viol = _run(fuzzer, tmp_path, 200000,
                                                                       seed)
    assert viol == 0
    assert inputs >= 200000
    # the inputs reach every outcome and the planner's consumers
    assert ok > 1000 and arg > 10000 and uns > 100 and plans > 1000
    assert max_ms < 2000
