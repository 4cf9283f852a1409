"""Shared test helpers: golden-fixture loading and the reference's own
acceptance rules (test/fixture_parity_test.dart:66-70, :85, :99)."""
import json
import math
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"

_NP = {"float32": np.float32, "int64": np.int64, "uint8": np.uint8,
       "int8": np.int8, "int32": np.int32}


def tensor(t):
    return np.array(t["data"], dtype=_NP[t["dtype"]]).reshape(t["shape"])


def load_golden(case):
    """Returns (fixture dict, {name: ndarray} for initializers+inputs,
    {name: ndarray} expected)."""
    d = json.loads((GOLDEN / f"{case}.json").read_text())
    vals = {k: tensor(v) for k, v in d["initializers"].items()}
    vals.update({k: tensor(v) for k, v in d["inputs"].items()})
    exp = {k: tensor(v) for k, v in d["expected"].items()}
    return d, vals, exp


def node_arg(d, vals, i):
    """Positional node input i (None when absent), like _dispatch's ins[i]."""
    names = d["node_inputs"]
    if i >= len(names) or names[i] == "":
        return None
    return vals[names[i]]


def fixture_float_ok(have, want, tol=2e-5):
    """fixture_parity_test.dart:72-100: max|d| <= max(2e-5, 2e-5*max|want|)
    and cosine > 0.999999.  Returns (ok, max_abs, cosine)."""
    w = np.asarray(want, dtype=np.float64).ravel()
    h = np.asarray(have, dtype=np.float64).ravel()
    max_abs = float(np.max(np.abs(w - h))) if w.size else 0.0
    mag = float(np.max(np.abs(w))) if w.size else 0.0
    ok = max_abs <= max(tol, 2e-5 * mag)
    nw, nh = float(np.dot(w, w)), float(np.dot(h, h))
    cos = 1.0
    if nw > 0 and nh > 0:
        cos = float(np.dot(w, h)) / (math.sqrt(nw) * math.sqrt(nh))
        ok = ok and cos > 0.999999
    return ok, max_abs, cos


def normwise_rel_err(have, want):
    """max|have - want| / max|want| (the float parity metric of the path)."""
    w = np.asarray(want, dtype=np.float64)
    h = np.asarray(have, dtype=np.float64)
    den = float(np.max(np.abs(w))) if w.size else 0.0
    num = float(np.max(np.abs(h - w))) if w.size else 0.0
    return num / den if den > 0 else num
