"""GPU parity of the fused producer + prep entry points
(fgm_hip_prep_rmsnorm_dev, fgm_hip_prep_gelu_mul_dev).

Each must equal, byte for byte, the reference's two calls: rmsnorm (or
gelu_mul) into the xn (act) buffer (forward.rs:477-481, 614-622), then
prep_rows over all rows (ops.c:293-314).  The checker is the oracle's
restatement of both (pinned against the reference in test_elem_oracle.py and
test_oracle.py), and the library's own separate device calls.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from fastgemma_amd import kernels as K
from tests import hip_util as H

pytestmark = pytest.mark.gpu

EPS = 1e-6

# (m, k, hsz, lda): decode and prefill rows of the model's widths, a rotation
# per case, a padded row stride, the largest k a row of LDS holds
# per-row float4s per thread (the row body is compiled once per count, 1 ..
# 8): 512 threads per row up to k = 2048 * 8 for rmsnorm, 1024 for gelu_mul;
# the cases below reach every count for both producers
RMS_CASES = [(1, 2560, 0, 2560), (8, 2560, 256, 2560), (13, 1536, 512, 1600),
             (37, 5376, 0, 5376), (3, 32768, 1024, 32768), (16, 64, 64, 64), (100, 3840, 128, 3840),
             (3, 8192, 128, 8192), (2, 10240, 0, 10240), (2, 12288, 512, 12352),
             (2, 14336, 128, 14336)]
GELU_CASES = [(8, 10240, 0, 10240), (5, 16384, 1024, 16384), (20, 6144, 512, 6400),
              (2, 32768, 0, 32768), (33, 2048, 2048, 2048), (2, 20480, 128, 20480),
              (2, 24576, 0, 24576), (2, 28672, 512, 28736)]


def bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


def oracle_prep(src, m, k, hsz):
    """prep_rows over rows [0, m) of a contiguous [m, k] f32 buffer."""
    rot = np.zeros((m, k), np.float32)
    qa = np.zeros((m, k), np.int8)
    qs = np.zeros(m, np.float32)
    pa = np.zeros(oracle.packed_a_len(m, k), np.int8)
    oracle.prep_rows(np.ascontiguousarray(src, np.float32), k, rot, qa, qs, pa, m, k, hsz, 0, m)
    return rot, qa, qs, pa


def dev_outputs(m, k):
    t = H.torch()
    return (t.full((m, k), 7.0, dtype=t.float32, device="cuda"),
            t.full((m, k), 7.0, dtype=t.float32, device="cuda"),
            t.full((m, k), 5, dtype=t.int8, device="cuda"),
            t.full((m,), 7.0, dtype=t.float32, device="cuda"),
            t.full((oracle.packed_a_len(m, k),), 5, dtype=t.int8, device="cuda"))


def rms_inputs(m, k, lda, seed):
    x = (oracle.gen_normal(seed, m * lda) * 3.0).reshape(m, lda)
    x[m // 2, :k] *= 1e-3                               # a small-norm row
    if m > 2:
        x[1, :k] = 0.0                                  # a zero row: xn 0, scale 1
    w = oracle.gen_uniform(seed + 1, k, -2.0, 2.0)
    return x, w


@pytest.mark.parametrize("scale", [True, False], ids=["w", "noscale"])
@pytest.mark.parametrize("case", RMS_CASES, ids=[f"m{c[0]}_k{c[1]}_h{c[2]}" for c in RMS_CASES])
def test_prep_rmsnorm_matches_rmsnorm_then_prep(case, scale):
    m, k, hsz, lda = case
    print(f"prep_rmsnorm m={m} k={k} hsz={hsz} lda={lda} scale={scale}", flush=True)
    x, w = rms_inputs(m, k, lda, 100 + m + k)
    wv = w if scale else None
    xn = np.stack([oracle.rmsnorm(x[r, :k], wv, EPS) for r in range(m)])
    want = (xn,) + oracle_prep(xn, m, k, hsz)
    dxn, drot, dqa, dqs, dpa = dev_outputs(m, k)
    dx, dw = H.dev(x), H.dev(w) if scale else None
    K.prep_rmsnorm(dx, lda, dw, EPS, dqs, dpa, m, k, hsz, xn=dxn, rot=drot, qa=dqa)
    got = [H.host(t) for t in (dxn, drot, dqa, dqs, dpa)]
    for g, w_, name in zip(got, want, ("xn", "rot", "qa", "qs", "pa")):
        assert np.array_equal(bits(g), bits(w_)), name


@pytest.mark.parametrize("case", GELU_CASES, ids=[f"m{c[0]}_k{c[1]}_h{c[2]}" for c in GELU_CASES])
def test_prep_gelu_mul_matches_gelu_mul_then_prep(case):
    m, k, hsz, lda = case
    print(f"prep_gelu_mul m={m} k={k} hsz={hsz} lda={lda}", flush=True)
    g = oracle.gen_uniform(7 + k, m * lda, -12.0, 12.0).reshape(m, lda)  # past exp's clamp too
    u = oracle.gen_normal(8 + k, m * lda).reshape(m, lda)
    act = np.stack([oracle.gelu_mul(g[r, :k], u[r, :k]) for r in range(m)])
    want = (act,) + oracle_prep(act, m, k, hsz)
    dact, drot, dqa, dqs, dpa = dev_outputs(m, k)
    K.prep_gelu_mul(H.dev(g), H.dev(u), lda, dqs, dpa, m, k, hsz, act=dact, rot=drot, qa=dqa)
    got = [H.host(t) for t in (dact, drot, dqa, dqs, dpa)]
    for gt, w_, name in zip(got, want, ("act", "rot", "qa", "qs", "pa")):
        assert np.array_equal(bits(gt), bits(w_)), name


def test_fused_equals_separate_device_calls_and_optional_outputs():
    """Only qs and pa requested; an unaligned weight and an odd row stride take
    the scalar load paths.  Equal to the library's separate rmsnorm and
    prep_rows launches."""
    t = H.torch()
    m, k, hsz, lda = 24, 2560, 256, 2563
    x, w = rms_inputs(m, k, lda, 5)
    dx = H.dev(x)
    wpad = t.zeros(k + 1, dtype=t.float32, device="cuda")
    wpad[1:] = H.dev(w)
    dw = wpad[1:]                                       # 4 bytes past a 16-byte boundary
    # separate: rmsnorm row by row into xn, then prep_rows
    xn = t.empty((m, k), dtype=t.float32, device="cuda")
    for r in range(m):
        K.rmsnorm(xn[r], dx[r, :k], dw, EPS)
    rot, qa, qs1, pa1 = (t.empty((m, k), dtype=t.float32, device="cuda"),
                         t.empty((m, k), dtype=t.int8, device="cuda"),
                         t.empty(m, dtype=t.float32, device="cuda"),
                         t.empty(oracle.packed_a_len(m, k), dtype=t.int8, device="cuda"))
    K.prep_rows(xn, k, rot, qa, qs1, pa1, m, k, hsz, 0, m)
    qs2 = t.full((m,), 7.0, dtype=t.float32, device="cuda")
    pa2 = t.full((oracle.packed_a_len(m, k),), 5, dtype=t.int8, device="cuda")
    K.prep_rmsnorm(dx, lda, dw, EPS, qs2, pa2, m, k, hsz)
    assert np.array_equal(bits(H.host(qs1)), bits(H.host(qs2)))
    assert np.array_equal(H.host(pa1), H.host(pa2))
    # and against the oracle
    xo = np.stack([oracle.rmsnorm(x[r, :k], w, EPS) for r in range(m)])
    _, _, qso, pao = oracle_prep(xo, m, k, hsz)
    assert np.array_equal(bits(H.host(qs2)), bits(qso))
    assert np.array_equal(H.host(pa2), pao)


def test_fused_rejects_bad_shapes():
    t = H.torch()
    x = t.zeros((4, 96), dtype=t.float32, device="cuda")
    qs = t.zeros(4, dtype=t.float32, device="cuda")
    pa = t.zeros(16 * 128, dtype=t.int8, device="cuda")
    with pytest.raises(Exception, match="multiple of 64"):
        K.prep_rmsnorm(x, 96, None, EPS, qs, pa, 4, 96, 0)
    with pytest.raises(Exception, match="hsz"):
        K.prep_gelu_mul(x, x, 96, qs, pa, 4, 64, 48)


ROT_CASES = [(5, 8192, h) for h in (1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024, 2048, 4096, 8192)] + \
            [(3, 2560, h) for h in (4, 32, 256, 512)] + [(17, 192, 64), (2, 32768, 32768)] + \
            [(3, 6144, 128), (2, 10240, 256), (2, 12288, 64), (2, 14336, 128), (2, 16384, 1024)]


@pytest.mark.parametrize("case", ROT_CASES, ids=[f"m{c[0]}_k{c[1]}_h{c[2]}" for c in ROT_CASES])
def test_prep_rows_every_rotation_size(case):
    """The rotation's stages run in three places (inside a thread, across the
    lanes of a wave, through LDS); every block size from 1 to a whole row,
    plain and fused, equals the oracle's prep_rows."""
    m, k, hsz = case
    print(f"prep_rows rotation m={m} k={k} hsz={hsz}", flush=True)
    x = (oracle.gen_student_t(31 + hsz, m * k, 3) * 2.0).reshape(m, k)
    want = oracle_prep(x, m, k, hsz)
    _, drot, dqa, dqs, dpa = dev_outputs(m, k)
    K.prep_rows(H.dev(x), k, drot, dqa, dqs, dpa, m, k, hsz, 0, m)
    for g, w_, name in zip([H.host(t) for t in (drot, dqa, dqs, dpa)], want, ("rot", "qa", "qs", "pa")):
        assert np.array_equal(bits(g), bits(w_)), name
    if m > 1 and k <= 8192:
        w = oracle.gen_uniform(3, k, 0.5, 1.5)
        xn = np.stack([oracle.rmsnorm(x[r], w, EPS) for r in range(m)])
        want = oracle_prep(xn, m, k, hsz)
        _, drot, dqa, dqs, dpa = dev_outputs(m, k)
        K.prep_rmsnorm(H.dev(x), k, H.dev(w), EPS, dqs, dpa, m, k, hsz, rot=drot, qa=dqa)
        for g, w_, name in zip([H.host(t) for t in (drot, dqa, dqs, dpa)], want,
                               ("rot", "qa", "qs", "pa")):
            assert np.array_equal(bits(g), bits(w_)), "fused " + name
