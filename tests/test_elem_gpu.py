"""GPU parity of the elementwise primitives (fgm_elem.hip) against the oracle
restatement of ops.c (itself pinned to the reference's bytes by
tests/test_elem_oracle.py) and the reference's recorded digests.

Bar: bit-exact everywhere the reference uses IEEE operations -- rmsnorm (both
forms), the vector part of gelu / gelu_mul / softcap, rope (angles from the
host's libm), add / mul / scale.  The scalar tails of gelu and softcap
(n % 16 != 0 only) call glibc's tanhf in the reference (not correctly
rounded) and a double-evaluated tanh here; gelu's 1 + tanh cancels, so the
tail bound is stated on the term before cancellation: |got - want| <= 4 ulp of
0.5 |v| (times |up| for gelu_mul), and 4 ulp of the result for softcap.
"""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np
import pytest

import oracle
from fastgemma_amd import kernels as K
from tests.golden import cases
from tests import hip_util as H

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "ref_outputs.json")))
TAIL_ULP = 4


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def ulp_diff(a: np.ndarray, b: np.ndarray) -> int:
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return int(np.max(np.abs(ia - ib))) if a.size else 0


def assert_vec_exact_tail_close(got, want, n, scale=None):
    """Bit-exact on the 16-wide vector part; the tail within TAIL_ULP ulp of
    `scale` (the magnitude before 1 + tanh cancels) or of the result."""
    nv = n & ~15
    assert np.array_equal(got[:nv].view(np.uint32), want[:nv].view(np.uint32))
    if scale is None:
        assert ulp_diff(got[nv:], want[nv:]) <= TAIL_ULP
    else:
        tol = TAIL_ULP * np.spacing(np.abs(scale[nv:]).astype(np.float32))
        assert np.all(np.abs(got[nv:] - want[nv:]) <= tol)


def gpu(fn, *arrays):
    """Run fn on device copies of the arrays; return the device copies."""
    ds = [H.dev(a) for a in arrays]
    fn(*ds)
    return [H.host(d) for d in ds]


@pytest.mark.parametrize("n", cases.ELEM_NS)
def test_elementwise_device_matches_oracle_and_reference(n):
    e = cases.elem_inputs(n)
    gold = GOLD["elem"][str(n)]
    out = np.zeros(n, np.float32)
    o, _, _ = gpu(lambda o, x, w: K.rmsnorm(o, x, w, 1e-6), out, e["x"], e["w"])
    assert sha(o) == gold["rmsnorm"]
    o, _ = gpu(lambda o, x: K.rmsnorm_noscale(o, x, n, 1e-6), out, e["x"])
    assert sha(o) == gold["rmsnorm_noscale"]
    o, _, _ = gpu(lambda o, g, u: K.gelu_mul(o, g, u, n), out, e["gate"], e["up"])
    assert_vec_exact_tail_close(o, oracle.gelu_mul(e["gate"], e["up"]), n,
                                np.float32(0.5) * e["gate"] * e["up"])
    if n % 16 == 0:
        assert sha(o) == gold["gelu_mul"]
    (g,) = gpu(K.gelu, e["gate"])
    assert_vec_exact_tail_close(g, oracle.gelu_mul(e["gate"], None), n,
                                np.float32(0.5) * e["gate"])
    (c,) = gpu(lambda x: K.softcap(x, 30.0), e["sc"])
    assert_vec_exact_tail_close(c, oracle.softcap(e["sc"], 30.0), n)
    if n % 16 == 0:
        assert sha(c) == gold["softcap"]
    a, _ = gpu(K.add, e["x"], e["w"])
    assert sha(a) == gold["add"]
    a, _ = gpu(K.mul, e["x"], e["w"])
    assert sha(a) == gold["mul"]
    (a,) = gpu(lambda x: K.scale(x, 0.7071067811865476), e["x"])
    assert sha(a) == gold["scale"]


@pytest.mark.parametrize("nh,hd,pos", cases.ROPE_CASES)
def test_rope_device_matches_reference(nh, hd, pos):
    x, inv = cases.rope_inputs(nh, hd)
    (y,) = gpu(lambda t: K.rope(t, nh, hd, inv, pos), x)
    assert sha(y) == GOLD["rope"][f"{nh}x{hd}@{pos}"]


def test_rmsnorm_rows_equal_per_row_calls():
    """The batched device call (the forward pass's per-row / per-head loops,
    forward.rs:480-511) equals one reference call per row, byte for byte."""
    rows, n = 24, 256
    x = oracle.gen_student_t(31, rows * n, 3).reshape(rows, n) * np.float32(4.0)
    w = oracle.gen_normal(32, n)
    t = H.torch()
    dx, dw = H.dev(x), H.dev(w)
    out = t.empty((rows, n), dtype=t.float32, device="cuda")
    K.rmsnorm_rows(out, dx, dw, rows, n, 1e-6)
    got = H.host(out)
    want = np.stack([oracle.rmsnorm(x[r], w, 1e-6) for r in range(rows)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    K.rmsnorm_rows(out, dx, None, rows, n, 1e-6)
    want = np.stack([oracle.rmsnorm(x[r], None, 1e-6) for r in range(rows)])
    assert np.array_equal(H.host(out).view(np.uint32), want.view(np.uint32))


def test_rope_multi_position_rows():
    """Prefill: one (cos, sin) table per token row; equals per-token calls."""
    nh, hd = 4, 128
    rows = 5
    _, inv = cases.rope_inputs(nh, hd)
    x = oracle.gen_normal(44, rows * nh * hd).reshape(rows, nh * hd)
    pos = [0, 3, 17, 4096, 12345]
    cs = np.stack([K.rope_table(inv, hd, p) for p in pos])
    import fastgemma_amd as F
    dx, dcs = H.dev(x), H.dev(cs)
    F.check(F.lib().fgm_hip_rope_dev(dx.data_ptr(), rows, nh, hd, dcs.data_ptr(), None))
    got = H.host(dx)
    want = np.stack([oracle.rope(x[r], nh, hd, inv, pos[r]) for r in range(rows)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_elementwise_dropins_host_pointers():
    """The host-pointer drop-ins (the reference's signatures, lib.rs:47-59)."""
    n = 2048
    e = cases.elem_inputs(n)
    gold = GOLD["elem"][str(n)]
    out = np.empty(n, np.float32)
    K.rmsnorm(out, e["x"], e["w"], 1e-6)
    assert sha(out) == gold["rmsnorm"]
    K.gelu_mul(out, e["gate"], e["up"], n)
    assert sha(out) == gold["gelu_mul"]
    y = e["sc"].copy()
    K.softcap(y, 30.0)
    assert sha(y) == gold["softcap"]
    x, inv = cases.rope_inputs(8, 256)
    K.rope(x, 8, 256, inv, 997)
    assert sha(x) == GOLD["rope"]["8x256@997"]
