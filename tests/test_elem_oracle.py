"""The oracle's elementwise restatements (oracle/fgm_oracle.c, ops.c:15-147,
316-350) pinned three ways:

* byte-for-byte against the reference's own ops.c outputs recorded in
  tests/golden/ref_outputs.json (tests/golden/make_golden.py ran the C built
  from the reference's sources), and live against oracle/_ref where present;
* against the mathematics the code approximates (tanh-GELU, exp, rotations,
  tanh soft-capping, the root mean square), with tolerances, so that a wrong
  constant or a dropped term fails even where the golden digests would
  still be regenerated from a wrong build;
* invariants: rmsnorm's scale invariance, rope at position 0 is the identity
  and preserves each pair's norm, softcap is odd and bounded.
"""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np
import pytest

import oracle
from tests.golden import cases

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "ref_outputs.json")))


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def oracle_elem(n: int) -> dict:
    e = cases.elem_inputs(n)
    return {
        "rmsnorm": oracle.rmsnorm(e["x"], e["w"], 1e-6),
        "rmsnorm_noscale": oracle.rmsnorm(e["x"], None, 1e-6),
        "gelu_mul": oracle.gelu_mul(e["gate"], e["up"]),
        "gelu": oracle.gelu_mul(e["gate"], None),
        "softcap": oracle.softcap(e["sc"], 30.0),
        "add": oracle.add(e["x"], e["w"]),
        "mul": oracle.mul(e["x"], e["w"]),
        "scale": oracle.scale(e["x"], 0.7071067811865476),
    }


@pytest.mark.parametrize("n", cases.ELEM_NS)
def test_elementwise_matches_reference_golden(n):
    got = oracle_elem(n)
    for name, want in GOLD["elem"][str(n)].items():
        assert sha(got[name]) == want, (name, n)


@pytest.mark.parametrize("nh,hd,pos", cases.ROPE_CASES)
def test_rope_matches_reference_golden(nh, hd, pos):
    x, inv = cases.rope_inputs(nh, hd)
    assert sha(oracle.rope(x, nh, hd, inv, pos)) == GOLD["rope"][f"{nh}x{hd}@{pos}"]


def test_elementwise_live_vs_reference():
    """Fresh inputs (other seeds, ragged lengths) against the compiled ops.c."""
    R = oracle.ref()
    if R is None:
        pytest.skip("oracle/_ref not built or host lacks AVX-512")
    P = oracle._ptr
    for n in (3, 17, 100, 1000, 4099):
        x = oracle.gen_student_t(77 + n, n, 3) * np.float32(5.0)
        w = oracle.gen_normal(78 + n, n)
        o = np.empty(n, np.float32)
        R.fgm_rmsnorm(P(o), P(x), P(w), n, 1e-5)
        assert sha(o) == sha(oracle.rmsnorm(x, w, 1e-5))
        g = x.copy()
        R.fgm_gelu(P(g), n)
        assert sha(g) == sha(oracle.gelu_mul(x, None))
        c = (x * np.float32(8.0)).astype(np.float32)
        c2 = c.copy()
        R.fgm_softcap(P(c2), n, 15.0)
        assert sha(c2) == sha(oracle.softcap(c, 15.0))


def test_exp16_against_exp():
    """Cephes exp: within 2 ulp of the correctly rounded exp on [-87, 87];
    clamped to +-88 outside."""
    for v in np.linspace(-87.0, 87.0, 4001, dtype=np.float32):
        got = np.float32(oracle.exp16(float(v)))
        want = np.float32(np.exp(np.float64(v)))
        assert abs(got - want) <= 2 * np.spacing(want), (v, got, want)
    assert oracle.exp16(1000.0) == oracle.exp16(88.0)
    assert oracle.exp16(-1000.0) == oracle.exp16(-88.0)
    assert oracle.exp16(0.0) == 1.0


def test_gelu_against_tanh_formula():
    x = np.linspace(-9.0, 9.0, 10001, dtype=np.float32)
    want = 0.5 * x.astype(np.float64) * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x.astype(np.float64) ** 3)))
    got = oracle.gelu_mul(x, None).astype(np.float64)
    assert np.max(np.abs(got - want)) < 2e-6 * 9.0
    # the product form multiplies by up exactly once
    up = np.linspace(-2, 2, x.size, dtype=np.float32)
    assert np.array_equal(oracle.gelu_mul(x, up), (oracle.gelu_mul(x, None) * up).astype(np.float32))


def test_rmsnorm_closed_forms_and_invariance():
    n = 2048
    w = oracle.gen_normal(5, n)
    c = np.full(n, 3.0, np.float32)          # sum of squares exact: 9 n
    got = oracle.rmsnorm(c, w, 0.0)
    inv = np.float32(1.0) / np.sqrt(np.float32(9.0))
    assert np.array_equal(got, (c * inv) * w)
    x = oracle.gen_normal(6, n)
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    assert np.max(np.abs(oracle.rmsnorm(x, w, 1e-6) - ref)) < 1e-5 * np.max(np.abs(ref))
    # scale invariance (powers of two keep every rounding)
    assert np.array_equal(oracle.rmsnorm(x * np.float32(4.0), w, 0.0), oracle.rmsnorm(x, w, 0.0))
    assert np.array_equal(oracle.rmsnorm(x, None, 1e-6), oracle.rmsnorm(x, np.ones(n, np.float32), 1e-6))


def test_rope_identity_and_norm():
    x, inv = cases.rope_inputs(8, 256)
    assert np.array_equal(oracle.rope(x, 8, 256, inv, 0), x)
    y = oracle.rope(x, 8, 256, inv, 1234).reshape(8, 2, 128)
    x3 = x.reshape(8, 2, 128).astype(np.float64)
    n0 = x3[:, 0] ** 2 + x3[:, 1] ** 2
    n1 = y[:, 0].astype(np.float64) ** 2 + y[:, 1].astype(np.float64) ** 2
    assert np.max(np.abs(n1 - n0) / np.maximum(n0, 1e-3)) < 1e-5
    # zero frequencies ("nope" dims) pass through untouched
    assert np.array_equal(y[:, :, 96:], x.reshape(8, 2, 128)[:, :, 96:])


def test_softcap_properties():
    x = np.linspace(-300, 300, 20001, dtype=np.float32)
    y = oracle.softcap(x, 30.0)
    assert np.all(np.abs(y) <= 30.0)
    assert np.max(np.abs(y.astype(np.float64) - 30 * np.tanh(x.astype(np.float64) / 30))) < 1e-5 * 30
    assert np.array_equal(oracle.softcap(-x[:16], 30.0), -oracle.softcap(x[:16], 30.0))


def test_add_mul_scale_exact():
    a = oracle.gen_normal(9, 1000)
    b = oracle.gen_normal(10, 1000)
    assert np.array_equal(oracle.add(a, b), a + b)
    assert np.array_equal(oracle.mul(a, b), a * b)
    assert np.array_equal(oracle.scale(a, 0.5), a * np.float32(0.5))
