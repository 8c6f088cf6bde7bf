"""GPU parity of the HIP path against the reference.

Bar: int32 accumulators and all integer / byte outputs bit-exact; fp32
outputs bit-exact too, because the kernels reproduce the reference's epilogue
operation order (tolerance 0 ulp -- stricter than the north star's 1e-6
relative).  Checked against, in order of strength:

* the reference's own bytes for its own test cases (tests/golden, recorded
  from the reference C compiled from its sources);
* the oracle (oracle/fgm_oracle.c, itself pinned by tests/test_oracle.py);
* exact float64-BLAS products through an independent numpy layout decode.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

import oracle
from tests.golden import cases
from tests import hip_util as H

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "ref_outputs.json")))


def _inputs(kind, M, N, Kd, group, seed, dist="uniform"):
    A = oracle.gen_i8(seed, M * Kd, -127, 127).reshape(M, Kd)
    a_s = oracle.gen_uniform(seed + 1, max(M, 1), 1e-3, 1e-2)[:M].copy()
    if kind == "q8c":
        B = oracle.gen_i8(seed + 2, N * Kd, -127, 127)
        bs = oracle.gen_uniform(seed + 3, N, 1e-3, 1e-2)
    else:
        B = oracle.gen_u8(seed + 2, N * Kd // 2)
        bs = oracle.gen_uniform(seed + 3, (Kd // group) * N, 5e-3, 5e-2).astype(
            np.float16).view(np.uint16).reshape(Kd // group, N)
    return A, oracle.pack_a(M, Kd, A), a_s, B, bs


def _oracle(kind, M, N, Kd, Ap, a_s, B, bs, group, n0, n1, ldc=None, fill=0.0):
    ldc = N if ldc is None else ldc
    C = np.full((max(M, 1), ldc), fill, np.float32)
    if kind == "q8c":
        oracle.gemm_q8c(M, N, Kd, Ap, a_s, B, bs, C, ldc, n0, n1)
    else:
        oracle.gemm_q4g(M, N, Kd, Ap, a_s, B, bs, group, C, ldc, n0, n1)
    return C[:M]


def _bits_equal(x, y):
    return np.array_equal(np.ascontiguousarray(x).view(np.uint32),
                          np.ascontiguousarray(y).view(np.uint32))


# ----------------------------------------------- the reference's own cases
def test_reference_vnni_cases_bytes():
    """vnni_test.c:271-284 replayed: GPU bytes == the reference's bytes."""
    for (case, inp), rec in zip(cases.vnni_inputs(), GOLD["vnni"]):
        kind, M, N, Kd, group, n0, n1 = case
        print("case", case, flush=True)
        C = H.gpu_gemm(kind, M, N, Kd, inp["Ap"], inp["a_s"], inp["B"], inp["bs"], group, n0, n1)
        assert H.sha(C) == rec["sha256"], case


def test_reference_gemm_test_and_dbg_cases_bytes():
    a = cases.amx_inputs()
    for m in (a["M"], 8):
        Ap = oracle.pack_a(m, a["K"], a["A"][:m])
        for kind in ("q8c", "q4g"):
            B, bs = (a["B8"], a["bs8"]) if kind == "q8c" else (a["Bq"], a["bs4"])
            C = H.gpu_gemm(kind, m, a["N"], a["K"], Ap, a["a_s"][:m].copy(), B, bs, a["group"])
            assert H.sha(C) == GOLD["amx"][f"{kind}_M{m}"]["sha256"], (kind, m)
    d = cases.dbg_inputs()
    C = H.gpu_gemm("q4g", d["M"], d["N"], d["K"], oracle.pack_a(d["M"], d["K"], d["A"]),
                   d["a_s"], d["Bq"], d["bs"], d["group"])
    assert H.sha(C) == GOLD["dbg"]["sha256"]


# ------------------------------------------------ both kernel families
SHAPES = [1, 2, 7, 8, 15, 16, 17, 31, 33, 48, 64, 65, 100, 128, 129, 256]


@pytest.mark.parametrize("M", SHAPES)
@pytest.mark.parametrize("kind,group", [("q8c", 0), ("q4g", 64), ("q4g", 128)])
def test_gemm_matches_oracle(kind, group, M):
    N, Kd = 256, 1024
    print(kind, group, M, F_path(kind, M, Kd, group), flush=True)
    A, Ap, a_s, B, bs = _inputs(kind, M, N, Kd, group or 64, seed=1000 + M)
    C = H.gpu_gemm(kind, M, N, Kd, Ap, a_s, B, bs, group or 64)
    R = _oracle(kind, M, N, Kd, Ap, a_s, B, bs, group or 64, 0, N // 16)
    assert _bits_equal(C, R)


def F_path(kind, M, Kd, group):
    from fastgemma_amd import kernels
    return kernels.gemm_path(8 if kind == "q8c" else 4, M, Kd, group or 64)


@pytest.mark.parametrize("M", [8, 40, 200])
@pytest.mark.parametrize("kind", ["q8c", "q4g"])
def test_n_range_ldc_and_untouched_columns(kind, M):
    """Only rows < M and columns [16 n0, 16 n1) are written (vnni_gemm.c:232-243)."""
    N, Kd, ldc = 512, 512, 600
    A, Ap, a_s, B, bs = _inputs(kind, M, N, Kd, 128, seed=77 + M)
    for n0, n1 in ((4, 12), (0, 4), (20, 32)):
        C = H.gpu_gemm(kind, M, N, Kd, Ap, a_s, B, bs, 128, n0, n1, ldc=ldc, fill=7.0)
        R = _oracle(kind, M, N, Kd, Ap, a_s, B, bs, 128, n0, n1, ldc=ldc, fill=7.0)
        assert _bits_equal(C, R), (n0, n1)
        assert np.all(C[:, :16 * n0] == 7.0) and np.all(C[:, 16 * n1:] == 7.0)


@pytest.mark.parametrize("M", [1, 8, 16, 64, 65, 256])
@pytest.mark.parametrize("kind,group", [("q8c", 0), ("q4g", 64), ("q4g", 256)])
def test_raw_accumulators_exact(kind, group, M):
    N, Kd = 128, 2048
    A, Ap, a_s, B, bs = _inputs(kind, M, N, Kd, group or 64, seed=500 + M)
    acc = H.gpu_acc(kind, M, N, Kd, Ap, B, group or 64)
    if kind == "q8c":
        assert np.array_equal(acc, H.exact_acc(A, H.decode_b8(B, N, Kd)))
    else:
        assert np.array_equal(acc, H.exact_group_acc(A, H.decode_b4(B, N, Kd), group))


def test_closed_form_extremes():
    """A = 127, B = -127: every accumulator is -127^2 K (> 2^24, so the float
    conversion rounds); int4 B = -8: -8 sum(A)."""
    M, N, Kd = 8, 64, 8192
    Ap = oracle.pack_a(M, Kd, np.full((M, Kd), 127, np.int8))
    B = oracle.pack_b_tiles(np.full((N, Kd), -127, np.int8))
    acc = H.gpu_acc("q8c", M, N, Kd, Ap, B)
    assert np.all(acc == -127 * 127 * Kd)
    C = H.gpu_gemm("q8c", M, N, Kd, Ap, np.ones(M, np.float32), B, np.ones(N, np.float32))
    assert np.all(C == np.float32(-127 * 127 * Kd))
    a = oracle.gen_i8(9, M * Kd, -127, 127).reshape(M, Kd)
    Bq = oracle.pack_nibbles(oracle.pack_b_tiles(np.full((N, Kd), -8, np.int8)))
    acc = H.gpu_acc("q4g", M, N, Kd, oracle.pack_a(M, Kd, a), Bq, 8192)
    assert np.all(acc[0] == (-8 * a.astype(np.int64).sum(axis=1))[:, None])


# --------------------------------------------------------------- preamble
def test_quant_act_matches_reference_golden():
    x, tail = cases.quant_rows()
    t = H.torch()
    for arr, qk, sk in ((x, "q_sha256", "s_bits"), (tail, "tail_q_sha256", "tail_s_bits")):
        rows, k = arr.shape
        q = t.empty((rows, k), dtype=t.int8, device="cuda")
        s = t.empty(rows, dtype=t.float32, device="cuda")
        from fastgemma_amd import kernels
        kernels.quant_act(H.dev(arr), rows, k, q, s)
        assert [int(v) for v in H.host(s).view(np.uint32)] == GOLD["quant_act"][sk]
        assert H.sha(H.host(q)) == GOLD["quant_act"][qk]


@pytest.mark.parametrize("hsz", [0, 128])
@pytest.mark.parametrize("nsplit", [1, 3])
def test_prep_rows_matches_reference_golden(hsz, nsplit):
    from fastgemma_amd import kernels
    t = H.torch()
    m, k, lda, src = cases.prep_input()
    split = (0, m) if nsplit == 1 else (0, 16, 32, m)
    rot = t.zeros((m, k), dtype=t.float32, device="cuda")
    qa = t.zeros((m, k), dtype=t.int8, device="cuda")
    qs = t.zeros(m, dtype=t.float32, device="cuda")
    pa = t.zeros(oracle.packed_a_len(m, k), dtype=t.int8, device="cuda")
    dsrc = H.dev(src)
    for r0, r1 in zip(split[:-1], split[1:]):
        kernels.prep_rows(dsrc, lda, rot, qa, qs, pa, m, k, hsz, r0, r1)
    got = H.sha(H.host(rot), H.host(qa), H.host(qs), H.host(pa))
    assert got == GOLD["prep_rows"][f"hsz{hsz}_split{nsplit}"]["sha256"]


@pytest.mark.parametrize("hsz", [8, 16, 128, 256])
def test_fwht_matches_reference_golden(hsz):
    from fastgemma_amd import kernels
    x = H.dev(cases.fwht_input(hsz))
    kernels.fwht(x, hsz)
    assert H.sha(H.host(x)) == GOLD["fwht"][str(hsz)]["sha256"]


def test_pack_a_matches_oracle():
    from fastgemma_amd import kernels
    t = H.torch()
    for m, k in ((1, 64), (37, 192), (256, 2048)):
        a = oracle.gen_i8(m + k, m * k, -127, 127).reshape(m, k)
        ap = t.full((oracle.packed_a_len(m, k),), 5, dtype=t.int8, device="cuda")
        kernels.pack_a(m, k, H.dev(a), ap)
        assert np.array_equal(H.host(ap), oracle.pack_a(m, k, a))


def test_quant_heavy_tails_and_odd_lengths_vs_oracle():
    from fastgemma_amd import kernels
    t = H.torch()
    for rows, k in ((64, 2048), (9, 8192), (3, 100), (5, 16), (2, 1), (3, 6150), (2, 16376)):
        x = oracle.gen_student_t(rows * 7 + k, rows * k, 3).reshape(rows, k)
        x[:, :: max(1, k // 3)] *= 20.0
        q = t.empty((rows, k), dtype=t.int8, device="cuda")
        s = t.empty(rows, dtype=t.float32, device="cuda")
        kernels.quant_act(H.dev(x), rows, k, q, s)
        rq, rs = oracle.quant_act(x, rows, k)
        assert np.array_equal(H.host(q), rq) and _bits_equal(H.host(s), rs), (rows, k)


# ----------------------------------------------------------- drop-in ABI
def test_dropin_host_pointer_api():
    """The host-pointer drop-ins: weights cached by address, A / C per call;
    a different weight buffer at a reused address is detected."""
    from fastgemma_amd import kernels
    M, N, Kd = 8, 256, 1024
    for kind in ("q8c", "q4g"):
        A, Ap, a_s, B, bs = _inputs(kind, M, N, Kd, 64, seed=31)
        for rep in range(2):
            C = np.full((M, N + 16), 3.0, np.float32)
            if kind == "q8c":
                kernels.gemm_q8c(M, N, Kd, Ap, a_s, B, bs, C, N + 16, 4, 12)
            else:
                kernels.gemm_q4g(M, N, Kd, Ap, a_s, B, bs, 64, C, N + 16, 4, 12)
            R = _oracle(kind, M, N, Kd, Ap, a_s, B, bs, 64, 4, 12, ldc=N + 16, fill=3.0)
            assert _bits_equal(C, R), (kind, rep)
            B[:] = np.roll(B, 1)  # same address, new contents
    m, k, lda, src = cases.prep_input()
    rot = np.zeros((m, k), np.float32)
    qa = np.zeros((m, k), np.int8)
    qs = np.zeros(m, np.float32)
    pa = np.zeros(oracle.packed_a_len(m, k), np.int8)
    for r0, r1 in ((0, 16), (16, 32), (32, m)):
        kernels.prep_rows(src, lda, rot, qa, qs, pa, m, k, 128, r0, r1)
    assert H.sha(rot, qa, qs, pa) == GOLD["prep_rows"]["hsz128_split3"]["sha256"]
    x = cases.fwht_input(128).copy()
    kernels.fwht(x, 128)
    assert H.sha(x) == GOLD["fwht"]["128"]["sha256"]
    xr, _ = cases.quant_rows()
    q = np.zeros(xr.shape, np.int8)
    s = np.zeros(xr.shape[0], np.float32)
    kernels.quant_act(xr, xr.shape[0], xr.shape[1], q, s)
    assert H.sha(q) == GOLD["quant_act"]["q_sha256"]
    a = oracle.gen_i8(3, 37 * 192, -127, 127)
    ap = np.zeros(oracle.packed_a_len(37, 192), np.int8)
    kernels.pack_a(37, 192, a, ap)
    assert np.array_equal(ap, oracle.pack_a(37, 192, a.reshape(37, 192)))


def test_dropin_replaced_weights_are_reclaimed():
    """A weight buffer rewritten again and again at one address: every call
    sees the current contents, and each copy the cache replaces is freed at
    the next upload once no call holds it, so the cache keeps one copy of
    the buffer, not one per rewrite."""
    import fastgemma_amd as F
    from fastgemma_amd import kernels
    L = F.lib()
    M, N, Kd = 1, 4096, 4096                       # 16 MiB of int8 weights
    A, Ap, a_s, B, bs = _inputs("q8c", M, N, Kd, 64, seed=47)
    live = []
    for rep in range(6):
        B[:] = oracle.gen_i8(500 + rep, N * Kd, -127, 127)   # same address, new contents
        C = np.zeros((M, N), np.float32)
        kernels.gemm_q8c(M, N, Kd, Ap, a_s, B, bs, C, N, 0, N // 16)
        assert _bits_equal(C, _oracle("q8c", M, N, Kd, Ap, a_s, B, bs, 64, 0, N // 16)), rep
        assert L.fgm_hip_weight_cache_bytes(1) == 0, rep   # the replaced copy is gone
        live.append(L.fgm_hip_weight_cache_bytes(0))
    assert len(set(live)) == 1 and live[0] >= N * Kd, live


# --------------------------------------------- live reference (if present)
needs_ref = pytest.mark.skipif(oracle.ref() is None,
                               reason="oracle/_ref not present or host lacks AVX-512 VNNI")


@needs_ref
@pytest.mark.parametrize("kind,M", [("q8c", 8), ("q8c", 256), ("q4g", 8), ("q4g", 256)])
def test_gpu_vs_reference_live(kind, M):
    R = oracle.ref()
    N, Kd = 512, 2048
    A, Ap, a_s, B, bs = _inputs(kind, M, N, Kd, 64, seed=900 + M)
    C = H.gpu_gemm(kind, M, N, Kd, Ap, a_s, B, bs, 64)
    RC = np.zeros((M, N), np.float32)
    P = oracle._ptr
    if kind == "q8c":
        R.fgm_gemm_q8c_vnni(M, N, Kd, P(Ap), P(a_s), P(B), P(bs), P(RC), N, 0, N // 16)
    else:
        R.fgm_gemm_q4g_vnni(M, N, Kd, P(Ap), P(a_s), P(B), P(bs), 64, P(RC), N, 0, N // 16)
    assert _bits_equal(C, RC)


@pytest.mark.parametrize("M,N,Kd", [(256, 512, 8192), (256, 2560, 512), (200, 2048, 2048), (96, 1024, 4096)])
def test_dense_k_groups_exact(M, N, Kd):
    """Prefill-sized int8 GEMMs take the variants that split K over groups of
    waves and add the groups' int32 tiles: the accumulators equal the exact
    integer products and the scaled outputs the oracle's bytes."""
    print("q8c", M, N, Kd, F_path("q8c", M, Kd, 0), flush=True)
    A, Ap, a_s, B, bs = _inputs("q8c", M, N, Kd, 64, seed=4242 + M + N)
    acc = H.gpu_acc("q8c", M, N, Kd, Ap, B)
    assert np.array_equal(acc, H.exact_acc(A, H.decode_b8(B, N, Kd)))
    C = H.gpu_gemm("q8c", M, N, Kd, Ap, a_s, B, bs)
    R = _oracle("q8c", M, N, Kd, Ap, a_s, B, bs, 64, 0, N // 16)
    assert _bits_equal(C, R)


def test_dense_k_groups_large():
    """M=2048, K=8192 int8 (the long-prefill down projection) takes 128x128
    tiles with two K groups: exact accumulators, and the epilogue's bytes
    recomputed from them as (float)acc * (b_scale * a_scale)."""
    M, N, Kd = 2048, 2048, 8192
    print("q8c", M, N, Kd, flush=True)
    A, Ap, a_s, B, bs = _inputs("q8c", M, N, Kd, 64, seed=99)
    acc = H.gpu_acc("q8c", M, N, Kd, Ap, B)
    want = H.exact_acc(A, H.decode_b8(B, N, Kd))
    assert np.array_equal(acc, want)
    C = H.gpu_gemm("q8c", M, N, Kd, Ap, a_s, B, bs)
    R = want.astype(np.float32) * (bs[None, :].astype(np.float32) * a_s[:, None].astype(np.float32))
    assert _bits_equal(C, R.astype(np.float32))


def test_group64_chain_ignores_stale_lds():
    """int4 group 64 with K of one or two k-tiles: the fold reads its parked
    sums four k-tiles at a time, past what the stream parks.  Run right after
    a GEMM whose workgroups leave int32 partial sums in LDS (negative sums
    read as float are NaN bit patterns): the outputs still equal the oracle."""
    A, Ap, a_s, B, bs = _inputs("q8c", 256, 512, 2048, 64, seed=5)
    H.gpu_gemm("q8c", 256, 512, 2048, Ap, a_s, B, bs)       # K-group reduction through LDS
    for M in (1, 2, 8, 40, 64):
        for Kd in (64, 128):
            N = 64
            A, Ap, a_s, B, bs = _inputs("q4g", M, N, Kd, 64, seed=300 + M + Kd)
            C = H.gpu_gemm("q4g", M, N, Kd, Ap, a_s, B, bs, 64)
            R = _oracle("q4g", M, N, Kd, Ap, a_s, B, bs, 64, 0, N // 16)
            assert _bits_equal(C, R), (M, Kd)


# ----------------------------------------------------------- batched calls
@pytest.mark.parametrize("M", [8, 256])
def test_batched_gemms_equal_single_calls(M):
    """One batched call (several GEMMs per launch, both weight types, mixed
    shapes) writes the same bytes as the single calls."""
    from fastgemma_amd import kernels
    t = H.torch()
    specs = [("q4g", 8192 // 4, 2048), ("q4g", 2048 // 4, 8192 // 2), ("q8c", 512, 2048),
             ("q4g", 512, 2048), ("q8c", 1024, 1024), ("q4g", 256, 1024)]
    probs, refs = [], []
    for i, (kind, N, Kd) in enumerate(specs):
        A, Ap, a_s, B, bs = _inputs(kind, M, N, Kd, 64, seed=7000 + i)
        C = t.full((M, N), 9.0, device="cuda")
        probs.append(dict(bits=8 if kind == "q8c" else 4, m=M, n=N, k=Kd, group=64,
                          a=H.dev(Ap), a_scale=H.dev(a_s), b=H.dev(B), b_scale=H.dev(bs), c=C,
                          ldc=N, n0=0, n1=N // 16))
        refs.append(H.gpu_gemm(kind, M, N, Kd, Ap, a_s, B, bs, 64, fill=9.0))
    kernels.gemm_batch(probs)
    for p, r in zip(probs, refs):
        assert _bits_equal(H.host(p["c"]), r)


def test_batched_prep_equals_single_calls():
    from fastgemma_amd import kernels
    t = H.torch()
    probs, refs = [], []
    for i, (m, k, hsz) in enumerate([(8, 2048, 0), (8, 8192, 0), (37, 256, 128), (256, 2048, 0),
                                     (1, 1024, 64)]):
        x = oracle.gen_normal(60 + i, m * k).reshape(m, k)
        qs = t.zeros(m, device="cuda")
        pa = t.zeros(oracle.packed_a_len(m, k), dtype=t.int8, device="cuda")
        qa = t.zeros((m, k), dtype=t.int8, device="cuda")
        probs.append(dict(src=H.dev(x), lda=k, rot=None, qa=qa, qs=qs, pa=pa, m=m, k=k, hsz=hsz,
                          r0=0, r1=m))
        xr = oracle.fwht(x, hsz) if hsz else x
        rq, rs = oracle.quant_act(xr, m, k)
        refs.append((rq, rs, oracle.pack_a(m, k, rq)))
    kernels.prep_batch(probs)
    for p, (rq, rs, rap) in zip(probs, refs):
        assert np.array_equal(H.host(p["qa"]), rq)
        assert _bits_equal(H.host(p["qs"]), rs)
        assert np.array_equal(H.host(p["pa"]), rap)


def test_batched_prep_wide_and_narrow_rows():
    """One launch sizes its workgroups for the widest row (32768 columns:
    1024 threads), so a 64-column row leaves whole waves past its end and a
    6144-column one runs with two float4s per thread; rotations through
    lanes and through LDS, every output requested, against the oracle."""
    from fastgemma_amd import kernels
    t = H.torch()
    probs, refs = [], []
    for i, (m, k, hsz) in enumerate([(3, 32768, 1024), (5, 64, 64), (2, 6144, 512)]):
        x = (oracle.gen_student_t(90 + i, m * k, 3) * 2.0).reshape(m, k)
        rot = t.full((m, k), 7.0, device="cuda")
        qa = t.full((m, k), 5, dtype=t.int8, device="cuda")
        qs = t.full((m,), 7.0, device="cuda")
        pa = t.full((oracle.packed_a_len(m, k),), 5, dtype=t.int8, device="cuda")
        probs.append(dict(src=H.dev(x), lda=k, rot=rot, qa=qa, qs=qs, pa=pa, m=m, k=k, hsz=hsz,
                          r0=0, r1=m))
        want = (np.zeros((m, k), np.float32), np.zeros((m, k), np.int8), np.zeros(m, np.float32),
                np.zeros(oracle.packed_a_len(m, k), np.int8))
        oracle.prep_rows(np.ascontiguousarray(x, np.float32), k, *want, m, k, hsz, 0, m)
        refs.append(want)
    kernels.prep_batch(probs)
    for p, want in zip(probs, refs):
        for name, w in zip(("rot", "qa", "qs", "pa"), want):
            assert np.array_equal(H.host(p[name]).view(np.uint8), np.ascontiguousarray(w).view(np.uint8)), \
                (p["k"], name)
