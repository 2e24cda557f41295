"""Loading of the re-encoded reference fixtures and the reference's own
comparison rule (test/fixture_parity_test.dart:21, :63-108)."""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden" / "fixtures"

_NP = {"float32": np.float32, "float16": np.float16, "float64": np.float64,
       "int64": np.int64, "int32": np.int32, "uint8": np.uint8, "int8": np.int8}


def to_array(t: dict | None):
    if t is None:
        return None
    data = [float(v) if isinstance(v, str) else v for v in t["data"]]
    return np.array(data, dtype=_NP[t["dtype"]]).reshape(t["shape"])


def load(name: str) -> dict:
    d = json.loads((GOLDEN / f"{name}.json").read_text())
    d["arrays"] = [to_array(x) for x in d["inputs"]]
    d["want"] = {k: to_array(v) for k, v in d["expected"].items()}
    return d


def names(prefix: str = "") -> list[str]:
    return sorted(p.stem for p in GOLDEN.glob(f"{prefix}*.json"))


def assert_reference_parity(have, want, what: str, tolerance: float = 2e-5):
    """The reference's fixture rule: ints exact; floats max|d| <= max(tol,
    tol*max|ref|) and cosine > 0.999999."""
    have = np.asarray(have)
    want = np.asarray(want)
    assert tuple(have.shape) == tuple(want.shape), (what, have.shape, want.shape)
    if want.dtype.kind in "iu":
        np.testing.assert_array_equal(have.astype(np.int64), want.astype(np.int64),
                                      err_msg=what)
        return
    w = want.astype(np.float64).ravel()
    h = have.astype(np.float64).ravel()
    fin = np.isfinite(w)
    assert np.all(np.isfinite(h[fin])), what
    d = np.abs(w[fin] - h[fin])
    max_abs = float(d.max()) if d.size else 0.0
    mag = float(np.abs(w[fin]).max()) if d.size else 0.0
    tol = max(tolerance, tolerance * mag)
    assert max_abs <= tol, f"{what}: max|d|={max_abs} > {tol}"
    nw, nh = float(np.dot(w, w)), float(np.dot(h, h))
    if nw > 0 and nh > 0:
        cos = float(np.dot(w, h)) / math.sqrt(nw * nh)
        assert cos > 0.999999, f"{what}: cosine={cos}"


def rms_error(have, want) -> float:
    """max|have-want| / rms(want): the float/int4 acceptance measure."""
    want = np.asarray(want, dtype=np.float64)
    have = np.asarray(have, dtype=np.float64)
    rms = math.sqrt(float(np.mean(want * want))) if want.size else 0.0
    if rms == 0:
        return float(np.abs(have - want).max()) if want.size else 0.0
    return float(np.abs(have - want).max()) / rms
