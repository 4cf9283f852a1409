"""The decoder-op oracle (oracle/decoder.py) against the reference's golden
vectors and against what the mathematics fixes.

Fixtures: the reference's ORT fixtures rmsnorm_pattern, rotary_embedding,
gqa_causal, gqa_kvcache, gqa_kvcache_rotary and gqa_kvcache_bias
(tool/gen_fixtures.py:636, :803-880, :882), accepted by the reference's own
rule (test/fixture_parity_test.dart:72-100).  Beyond them: attention against
a brute-force float64 softmax, incremental decoding (one token with the KV
cache) against the full-sequence result, rotary at position 0 as the
identity, and a planted mistake (rotary pairing x[i] with x[i+1]) that the
rotary fixture rejects.
"""
import numpy as np
import pytest

from oracle import decoder as D
from tests.helpers import fixture_float_ok, load_golden, node_arg


def test_rmsnorm_chain_golden():
    d, vals, exp = load_golden("rmsnorm_pattern")
    ops = [n["op_type"] for n in d["nodes"]]
    assert ops == ["Pow", "ReduceMean", "Add", "Sqrt", "Reciprocal", "Mul", "Mul"]
    assert int(vals["ax"][0]) == vals["x"].ndim - 1   # reduces the last axis
    y = D.rmsnorm(vals["x"], vals["gamma"], float(vals["eps"]))
    ok, max_abs, cos = fixture_float_ok(y, exp["out0"])
    assert ok, (max_abs, cos)


def _rotary_case():
    d, vals, exp = load_golden("rotary_embedding")
    return d, vals, exp


def test_rotary_golden():
    d, vals, exp = _rotary_case()
    y = D.rotary(vals["x"], vals["pos"], vals["cosc"], vals["sinc"],
                 interleaved=bool(d["attrs"].get("interleaved", 0)),
                 num_heads=d["attrs"].get("num_heads", 0))
    ok, max_abs, cos = fixture_float_ok(y, exp["out0"])
    assert ok, (max_abs, cos)


def test_rotary_fixture_rejects_wrong_pairing():
    d, vals, exp = _rotary_case()
    # planted mistake: the interleaved pairing for a non-interleaved node
    y = D.rotary(vals["x"], vals["pos"], vals["cosc"], vals["sinc"], interleaved=True)
    ok, _, _ = fixture_float_ok(y, exp["out0"])
    assert not ok


def test_rotary_position_zero_is_identity():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 3, 32)).astype(np.float32)
    cos, sin = D.rope_tables(8, 16, 10000.0)
    y = D.rotary(x, np.zeros((1, 3), np.int64), cos, sin, num_heads=2)
    np.testing.assert_array_equal(y, x)


@pytest.mark.parametrize("case", ["gqa_causal", "gqa_kvcache", "gqa_kvcache_rotary",
                                  "gqa_kvcache_bias"])
def test_gqa_golden(case):
    d, vals, exp = load_golden(case)
    at = d["attrs"]
    out, pk, pv = D.gqa(node_arg(d, vals, 0), node_arg(d, vals, 1), node_arg(d, vals, 2),
                        at["num_heads"], at["kv_num_heads"], at.get("scale"),
                        node_arg(d, vals, 3), node_arg(d, vals, 4),
                        node_arg(d, vals, 7), node_arg(d, vals, 8),
                        do_rotary=bool(at.get("do_rotary", 0)),
                        interleaved=bool(at.get("rotary_interleaved", 0)),
                        bias=node_arg(d, vals, 10))
    for name, have in (("out0", out), ("out1", pk), ("out2", pv)):
        if name in exp:
            assert have.shape == exp[name].shape, (case, name)
            ok, max_abs, cos = fixture_float_ok(have, exp[name])
            assert ok, (case, name, max_abs, cos)


def _brute_gqa(q, k, v, nh, kvh):
    b, s, _ = q.shape
    hd = q.shape[2] // nh
    out = np.zeros(q.shape, np.float64)
    for h in range(nh):
        kh = h // (nh // kvh)
        Q = q[0, :, h * hd:(h + 1) * hd].astype(np.float64)
        K = k[0, :, kh * hd:(kh + 1) * hd].astype(np.float64)
        V = v[0, :, kh * hd:(kh + 1) * hd].astype(np.float64)
        sc = Q @ K.T / np.sqrt(hd)
        sc[np.triu_indices(s, 1)] = -np.inf
        p = np.exp(sc - sc.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        out[0, :, h * hd:(h + 1) * hd] = p @ V
    return out


def test_gqa_matches_brute_force_softmax():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 7, 4 * 16)).astype(np.float32)
    k = rng.standard_normal((1, 7, 2 * 16)).astype(np.float32)
    v = rng.standard_normal((1, 7, 2 * 16)).astype(np.float32)
    out, _, _ = D.gqa(q, k, v, 4, 2)
    want = _brute_gqa(q, k, v, 4, 2)
    assert np.max(np.abs(out - want)) <= 1e-5 * np.max(np.abs(want))


def test_gqa_incremental_matches_full_sequence():
    rng = np.random.default_rng(2)
    s = 6
    q = rng.standard_normal((1, s, 4 * 16)).astype(np.float32)
    k = rng.standard_normal((1, s, 2 * 16)).astype(np.float32)
    v = rng.standard_normal((1, s, 2 * 16)).astype(np.float32)
    cos, sin = D.rope_tables(16, 16, 10000.0)
    full, fk, fv = D.gqa(q, k, v, 4, 2, None, None, None, cos, sin, do_rotary=True)
    part, pk, pv = D.gqa(q[:, :s - 1], k[:, :s - 1], v[:, :s - 1], 4, 2, None, None, None,
                         cos, sin, do_rotary=True)
    last, lk, lv = D.gqa(q[:, s - 1:], k[:, s - 1:], v[:, s - 1:], 4, 2, None, pk, pv,
                         cos, sin, do_rotary=True)
    np.testing.assert_array_equal(lk, fk)
    np.testing.assert_array_equal(lv, fv)
    np.testing.assert_allclose(last[0, 0], full[0, s - 1], rtol=0, atol=1e-6)


def test_silu_mul_closed_form():
    g = np.array([0.0, 1.0, -3.0, 20.0], np.float32)
    u = np.array([2.0, 1.0, 1.0, 0.5], np.float32)
    y = D.silu_mul(g, u)
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    np.testing.assert_allclose(y, want, rtol=2e-7)
    assert y[0] == 0.0


def test_gqa_rotary_batch_above_one_raises_like_the_reference():
    q = np.zeros((2, 1, 8), np.float32)
    k = np.zeros((2, 1, 8), np.float32)
    cos, sin = D.rope_tables(4, 8, 10000.0)
    with pytest.raises(ValueError):
        D.gqa(q, k, k, 1, 1, None, None, None, cos, sin, do_rotary=True)
