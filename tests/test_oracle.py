"""Pin the CPU oracle (oracle/fgm_oracle.c) before trusting it.

Each oracle function is checked by something other than a retyped copy of its
own formula:

* the reference's own outputs, produced by the reference's C compiled from its
  sources (oracle/_ref) and recorded in tests/golden/ref_outputs.json -- the
  reference's test case lists (vnni_test.c:271-284, gemm_test.c:84-130,
  dbg.c:21-57) replayed with their own generators;
* the reference's known-answer nibble table (vnni_test.c:62-69);
* brute-force int64 products through an independent numpy decode of the
  weight layout (quant.py:85-107 restated with reshapes, not index formulas);
* closed forms and invariants: constant operands, one-hot activations,
  M-invariance, n-range invariance, untouched columns, the Hadamard matrix
  (quant.py:58-64), FWHT involution, half-to-even ties (numpy.rint);
* when oracle/_ref is built on this host, live byte-for-byte comparison with
  the reference on further random shapes.
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
P = oracle._ptr


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


# ---------------------------------------------------- independent decoders
def decode_b8(blob: np.ndarray, n: int, k: int) -> np.ndarray:
    """VNNI tile stream -> q [N, K]: inverse of quant.py:105-107's transpose."""
    t = blob.astype(np.int8).reshape(n // 16, k // 64, 16, 16, 4)  # nb, kb, k/4, n, k%4
    return np.ascontiguousarray(t.transpose(0, 3, 1, 2, 4)).reshape(n, k)


def np_unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    """quant.py:85-92 in numpy."""
    p = packed.reshape(-1, 32)
    lo = (p & 0x0F).astype(np.int16)
    hi = ((p >> 4) & 0x0F).astype(np.int16)
    lo = (lo ^ 8) - 8
    hi = (hi ^ 8) - 8
    return np.concatenate([lo, hi], axis=1).reshape(-1).astype(np.int8)


def decode_b4(bq: np.ndarray, n: int, k: int) -> np.ndarray:
    return decode_b8(np_unpack_nibbles(bq), n, k)


def unpack_a(ap: np.ndarray, m: int, k: int) -> np.ndarray:
    t = ap.reshape(-1, k // 64, 16, 64)  # mb, kb, r, 64
    return np.ascontiguousarray(t.transpose(0, 2, 1, 3)).reshape(-1, k)[:m]


# ------------------------------------------------------------------ layout
def test_nibble_convention_known_answer():
    """vnni_test.c:62-69: nibble v decodes to {0..7, -8..-1}."""
    want = [0, 1, 2, 3, 4, 5, 6, 7, -8, -7, -6, -5, -4, -3, -2, -1]
    packed = np.zeros(32, np.uint8)
    packed[:16] = np.arange(16, dtype=np.uint8)          # low nibbles -> values 0..15
    packed[16:] = (np.arange(16, dtype=np.uint8) << 4)    # high nibbles -> values 48..63
    out = oracle.unpack_nibbles(packed)
    assert out[:16].tolist() == want
    assert out[32 + 16:64].tolist() == want


def test_nibble_roundtrip_all_values():
    flat = np.tile(np.arange(-8, 8, dtype=np.int8), 64 * 8)[: 64 * 16]
    flat = np.random.default_rng(0).permutation(flat).astype(np.int8)
    packed = oracle.pack_nibbles(flat)
    assert np.array_equal(oracle.unpack_nibbles(packed), flat)
    assert np.array_equal(np_unpack_nibbles(packed), flat)


def test_pack_b_tiles_matches_reshape_form():
    q = oracle.gen_i8(5, 64 * 256, -127, 127).reshape(64, 256)
    assert np.array_equal(decode_b8(oracle.pack_b_tiles(q), 64, 256), q)
    # quant.py:105-107's own reshape/transpose
    t = q.reshape(4, 16, 4, 16, 4).transpose(0, 2, 3, 1, 4)
    assert np.array_equal(oracle.pack_b_tiles(q), np.ascontiguousarray(t).reshape(-1))


def test_packers_match_reference_kernel_layout():
    """Unit scales make the reference kernel's output an exact integer product:
    oracle-packed weights must give numpy's A @ Q.T through the reference."""
    lay = cases.layout_inputs()
    exact8 = (lay["A"].astype(np.int64) @ lay["Q8"].astype(np.int64).T).astype(np.float32)
    exact4 = (lay["A"].astype(np.int64) @ lay["Q4"].astype(np.int64).T).astype(np.float32)
    assert sha(exact8) == GOLD["layout"]["q8c_sha256"]
    assert sha(exact4) == GOLD["layout"]["q4g_sha256"]


def test_pack_a_closed_form():
    m, k = 37, 192
    a = oracle.gen_i8(6, m * k, -127, 127).reshape(m, k)
    ap = oracle.pack_a(m, k, a)
    assert ap.size == oracle.packed_a_len(m, k) == 48 * k
    assert np.array_equal(unpack_a(ap, m, k), a)
    assert not unpack_a(ap, 48, k)[m:].any()  # padding rows are zero


# -------------------------------------------------------------------- f16
def test_f16_widening_all_halves():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))


def test_f16_narrowing_is_round_to_nearest_even():
    x = np.concatenate([oracle.gen_uniform(7, 4000, 5e-3, 5e-2),
                        oracle.gen_normal(8, 4000) * np.float32(1e3),
                        np.float32([6.1e-5, 3e-8, 65504.0, 65520.0, 1e9, 0.0, -0.0])])
    got = oracle.f32_to_f16(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# -------------------------------------------------------------- quantiser
def test_quant_act_matches_reference_golden():
    x, tail = cases.quant_rows()
    q, s = oracle.quant_act(x, x.shape[0], x.shape[1])
    g = GOLD["quant_act"]
    assert [int(v) for v in s.view(np.uint32)] == g["s_bits"]
    assert sha(q) == g["q_sha256"]
    qt, st = oracle.quant_act(tail, tail.shape[0], tail.shape[1])
    assert [int(v) for v in st.view(np.uint32)] == g["tail_s_bits"]
    assert sha(qt) == g["tail_q_sha256"]


def test_quant_act_closed_forms():
    k = 64
    x = np.zeros((4, k), np.float32)
    x[1, 7] = -2.5                     # single non-zero -> -127
    x[2] = np.linspace(-1, 1, k)       # extremes map to +-127
    x[3] = np.arange(k) - 31.5         # amax 32.5
    q, s = oracle.quant_act(x, 4, k)
    assert s[0] == 1.0 and not q[0].any()          # zero row: s = 1, q = 0
    assert q[1, 7] == -127 and np.count_nonzero(q[1]) == 1
    assert q[2, 0] == -127 and q[2, -1] == 127
    assert s[1] == np.float32(2.5) / np.float32(127.0)
    # ties go to even: amax 127 gives inv == 1 exactly
    r = np.array([[127.0] + [v + 0.5 for v in range(-20, 43)]], np.float32)
    q, s = oracle.quant_act(r, 1, 64)
    assert s[0] == 1.0
    assert np.array_equal(q[0, 1:], np.rint(r[0, 1:]).astype(np.int8))


# ------------------------------------------------------------------- FWHT
@pytest.mark.parametrize("hsz", [8, 16, 128, 256])
def test_fwht_matches_reference_golden(hsz):
    y = oracle.fwht(cases.fwht_input(hsz), hsz)
    assert sha(y) == GOLD["fwht"][str(hsz)]["sha256"]


def hadamard(n):
    """quant.py:58-64."""
    h = np.ones((1, 1))
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


@pytest.mark.parametrize("hsz", [16, 64, 128])
def test_fwht_equals_normalised_hadamard(hsz):
    x = oracle.gen_normal(40 + hsz, 3 * hsz).reshape(3, hsz)
    y = oracle.fwht(x, hsz)
    want = x.astype(np.float64) @ (hadamard(hsz) / np.sqrt(hsz)).T
    assert np.allclose(y, want, rtol=1e-5, atol=1e-5)
    back = oracle.fwht(y, hsz)                     # H is an involution
    assert np.allclose(back, x, rtol=1e-5, atol=1e-5)


def test_fwht_small_block_is_unscaled():
    """ops.c:172-173 scales 16 at a time, so hsz < 16 is left unnormalised."""
    x = oracle.gen_i8(9, 4 * 8, -20, 20).astype(np.float32).reshape(4, 8)
    y = oracle.fwht(x, 8)
    assert np.array_equal(y, (x.astype(np.float64) @ hadamard(8).T).astype(np.float32))


# --------------------------------------------------------------- prep_rows
@pytest.mark.parametrize("hsz", [0, 128])
@pytest.mark.parametrize("nsplit", [1, 3])
def test_prep_rows_matches_reference_golden(hsz, nsplit):
    m, k, lda, src = cases.prep_input()
    split = (0, m) if nsplit == 1 else (0, 16, 32, m)
    rot = np.zeros((m, k), np.float32)
    qa = np.zeros((m, k), np.int8)
    qs = np.zeros(m, np.float32)
    pa = np.zeros(oracle.packed_a_len(m, k), np.int8)
    for r0, r1 in zip(split[:-1], split[1:]):
        oracle.prep_rows(src, lda, rot, qa, qs, pa, m, k, hsz, r0, r1)
    assert sha(rot, qa, qs, pa) == GOLD["prep_rows"][f"hsz{hsz}_split{nsplit}"]["sha256"]
    # composition: copy -> fwht -> quant -> pack
    x = np.ascontiguousarray(src[:, :k])
    if hsz:
        x = oracle.fwht(x, hsz)
    q2, s2 = oracle.quant_act(x, m, k)
    assert np.array_equal(q2, qa) and np.array_equal(s2, qs)
    assert np.array_equal(oracle.pack_a(m, k, q2), pa)


# ------------------------------------------------------------------ GEMMs
def run_oracle(kind, M, N, K, group, n0, n1, inp):
    C = np.zeros((M, N), np.float32)
    if kind == "q8c":
        oracle.gemm_q8c(M, N, K, inp["Ap"], inp["a_s"], inp["B"], inp["bs"], C, N, n0, n1)
    else:
        oracle.gemm_q4g(M, N, K, inp["Ap"], inp["a_s"], inp["B"], inp["bs"], group, C, N,
                        n0, n1)
    return C


def test_gemm_matches_reference_vnni_and_amx_cases():
    """vnni_test.c:271-284 cases: oracle bytes == reference VNNI bytes (and the
    reference AMX bytes, which the golden shows are identical)."""
    for (case, inp), rec in zip(cases.vnni_inputs(), GOLD["vnni"]):
        assert list(case) == rec["case"]
        C = run_oracle(*case, inp)
        assert sha(C) == rec["sha256"], case
        if "amx_sha256" in rec:
            assert rec["amx_sha256"] == rec["sha256"]


def test_gemm_matches_reference_gemm_test_and_dbg_cases():
    a = cases.amx_inputs()
    for m in (a["M"], 8):
        Ap = oracle.pack_a(m, a["K"], a["A"][:m])
        for kind in ("q8c", "q4g"):
            inp = dict(Ap=Ap, a_s=a["a_s"][:m].copy(),
                       B=a["B8"] if kind == "q8c" else a["Bq"],
                       bs=a["bs8"] if kind == "q8c" else a["bs4"])
            C = run_oracle(kind, m, a["N"], a["K"], a["group"], 0, a["N"] // 16, inp)
            assert sha(C) == GOLD["amx"][f"{kind}_M{m}"]["sha256"], (kind, m)
    d = cases.dbg_inputs()
    inp = dict(Ap=oracle.pack_a(d["M"], d["K"], d["A"]), a_s=d["a_s"], B=d["Bq"], bs=d["bs"])
    C = run_oracle("q4g", d["M"], d["N"], d["K"], d["group"], 0, d["N"] // 16, inp)
    assert sha(C) == GOLD["dbg"]["sha256"]
    # dbg.c:39-57's independent scalar: every product and sum here is exact
    q = decode_b4(d["Bq"], d["N"], d["K"]).astype(np.float64)
    s = oracle.f16_to_f32(d["bs"]).astype(np.float64)           # [K/g, N]
    want = np.zeros((d["M"], d["N"]))
    for g in range(d["K"] // d["group"]):
        sl = slice(g * d["group"], (g + 1) * d["group"])
        want += (d["A"][:, sl].astype(np.float64) @ q[:, sl].T) * s[g]
    assert np.array_equal(C, want.astype(np.float32))


@pytest.mark.parametrize("case", [c for c in cases.VNNI_CASES])
def test_accumulators_equal_brute_force(case):
    kind, M, N, K, group, n0, n1 = case
    inp = dict(next(i for c, i in cases.vnni_inputs() if c == case))
    A = inp["A"].astype(np.int64)
    if kind == "q8c":
        Q = decode_b8(inp["B"], N, K).astype(np.int64)
        acc = oracle.acc_q8c(M, K, inp["Ap"], inp["B"], n0, n1, N)
        want = A @ Q.T
        assert np.array_equal(acc[:, n0 * 16:n1 * 16], want[:, n0 * 16:n1 * 16])
    else:
        Q = decode_b4(inp["B"], N, K).astype(np.int64)
        acc = oracle.acc_q4g(M, K, inp["Ap"], inp["B"], group, n0, n1, N)
        for g in range(K // group):
            sl = slice(g * group, (g + 1) * group)
            want = A[:, sl] @ Q[:, sl].T
            assert np.array_equal(acc[g][:, n0 * 16:n1 * 16], want[:, n0 * 16:n1 * 16])


def test_gemm_closed_forms():
    M, N, K = 3, 32, 2048
    Ap = oracle.pack_a(M, K, np.full((M, K), 127, np.int8))
    B = oracle.pack_b_tiles(np.full((N, K), -127, np.int8))
    C = np.zeros((M, N), np.float32)
    oracle.gemm_q8c(M, N, K, Ap, np.ones(M, np.float32), B, np.ones(N, np.float32), C, N, 0, 2)
    assert np.all(C == np.float32(-127 * 127 * K))  # rounds: |acc| > 2^24
    # int4, every weight -8: C = -8 * sum(A) * s
    a = oracle.gen_i8(50, M * K, -127, 127).reshape(M, K)
    Bq = oracle.pack_nibbles(oracle.pack_b_tiles(np.full((N, K), -8, np.int8)))
    s = np.full((K // 64, N), 0x3C00, np.uint16)
    C = np.zeros((M, N), np.float32)
    oracle.gemm_q4g(M, N, K, oracle.pack_a(M, K, a), np.ones(M, np.float32), Bq, s, 64, C, N,
                    0, 2)
    for m in range(M):
        assert np.all(C[m] == np.float32(-8 * int(a[m].astype(np.int64).sum())))
    # one-hot activation selects a weight row
    Q = oracle.gen_i8(51, N * K, -127, 127).reshape(N, K)
    e = np.zeros((1, K), np.int8)
    e[0, 777] = 1
    acc = oracle.acc_q8c(1, K, oracle.pack_a(1, K, e), oracle.pack_b_tiles(Q), 0, 2, N)
    assert np.array_equal(acc[0], Q[:, 777].astype(np.int32))


@pytest.mark.parametrize("kind", ["q8c", "q4g"])
def test_gemm_m_and_range_invariance(kind):
    """Row m depends only on row m of A; any [n0, n1) split writes the same
    bytes; columns outside [16 n0, 16 n1) stay untouched."""
    M, N, K, group = 21, 128, 512, 128
    A = oracle.gen_i8(60, M * K, -127, 127).reshape(M, K)
    a_s = oracle.gen_uniform(61, M, 1e-3, 1e-2)
    if kind == "q8c":
        B = oracle.gen_i8(62, N * K, -127, 127)
        bs = oracle.gen_uniform(63, N, 1e-3, 1e-2)
    else:
        B = oracle.gen_u8(62, N * K // 2)
        bs = oracle.gen_uniform(63, (K // group) * N, 5e-3, 5e-2).astype(np.float16).view(
            np.uint16).reshape(K // group, N)
    inp = dict(Ap=oracle.pack_a(M, K, A), a_s=a_s, B=B, bs=bs)
    full = run_oracle(kind, M, N, K, group, 0, N // 16, inp)
    part = np.full((M, N), 7.0, np.float32)
    for n0, n1 in ((0, 4), (4, 8)):
        if kind == "q8c":
            oracle.gemm_q8c(M, N, K, inp["Ap"], a_s, B, bs, part, N, n0, n1)
        else:
            oracle.gemm_q4g(M, N, K, inp["Ap"], a_s, B, bs, group, part, N, n0, n1)
    assert np.array_equal(part, full)
    one = dict(inp, Ap=oracle.pack_a(1, K, A[13:14].copy()), a_s=a_s[13:14].copy())
    row = run_oracle(kind, 1, N, K, group, 2, 6, one)
    assert np.array_equal(row[0, 32:96], full[13, 32:96])
    assert not row[0, :32].any() and not row[0, 96:].any()


# ------------------------------------------------- live reference (optional)
needs_ref = pytest.mark.skipif(oracle.ref() is None,
                               reason="oracle/_ref not built or host lacks AVX-512 VNNI")


@needs_ref
@pytest.mark.parametrize("kind,M,N,K,group,n0,n1", [
    ("q8c", 8, 512, 2048, 0, 0, 32), ("q8c", 40, 256, 8192, 0, 4, 16),
    ("q4g", 8, 512, 2048, 64, 0, 32), ("q4g", 24, 256, 8192, 64, 8, 16),
    ("q4g", 3, 256, 4096, 512, 0, 16)])
def test_gemm_live_vs_reference(kind, M, N, K, group, n0, n1):
    R = oracle.ref()
    seed = M * 1000 + K
    A = oracle.gen_i8(seed, M * K, -127, 127).reshape(M, K)
    a_s = oracle.gen_uniform(seed + 1, M, 1e-3, 1e-2)
    if kind == "q8c":
        B = oracle.gen_i8(seed + 2, N * K, -127, 127)
        bs = oracle.gen_uniform(seed + 3, N, 1e-3, 1e-2)
    else:
        B = oracle.gen_u8(seed + 2, N * K // 2)
        bs = oracle.gen_uniform(seed + 3, (K // group) * N, 5e-3, 5e-2).astype(
            np.float16).view(np.uint16)
    Ap = oracle.pack_a(M, K, A)
    inp = dict(Ap=Ap, a_s=a_s, B=B, bs=bs)
    C = run_oracle(kind, M, N, K, group, n0, n1, inp)
    R_C = np.zeros((M, N), np.float32)
    if kind == "q8c":
        R.fgm_gemm_q8c_vnni(M, N, K, P(Ap), P(a_s), P(B), P(bs), P(R_C), N, n0, n1)
    else:
        R.fgm_gemm_q4g_vnni(M, N, K, P(Ap), P(a_s), P(B), P(bs), group, P(R_C), N, n0, n1)
    assert np.array_equal(C.view(np.uint32), R_C.view(np.uint32))


@needs_ref
def test_quant_act_live_vs_reference_heavy_tails():
    R = oracle.ref()
    rows, k = 64, 2048
    x = oracle.gen_student_t(77, rows * k, 3).reshape(rows, k)
    x[:, [100, 1500]] *= 20.0
    q, s = oracle.quant_act(x, rows, k)
    rq = np.empty_like(q)
    rs = np.empty_like(s)
    R.fgm_quant_act(P(x), rows, k, P(rq), P(rs))
    assert np.array_equal(q, rq) and np.array_equal(s.view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("bits", [4, 8])
def test_pooled_gemm_equals_single_call(bits):
    """oracle.gemm_pooled (the N-split over host threads the GPU tests use as
    a full-range checker) gives the single-threaded oracle's bytes, with the
    oracle and, where oracle/_ref is built, with the reference's kernels."""
    M, N, K = 24, 1024, 1024
    A = oracle.gen_i8(71, M * K, -127, 127).reshape(M, K)
    Ap = oracle.pack_a(M, K, A)
    s = oracle.gen_uniform(72, M, 1e-3, 1e-2)
    if bits == 8:
        B = oracle.gen_i8(73, N * K, -127, 127)
        bs = oracle.gen_uniform(74, N, 1e-3, 1e-2)
    else:
        B = oracle.gen_u8(73, N * K // 2)
        bs = oracle.gen_uniform(74, (K // 64) * N, 5e-3, 5e-2).astype(np.float16).view(np.uint16)
    want = np.zeros((M, N), np.float32)
    if bits == 8:
        oracle.gemm_q8c(M, N, K, Ap, s, B, bs, want, N, 0, N // 16)
    else:
        oracle.gemm_q4g(M, N, K, Ap, s, B, bs, 64, want, N, 0, N // 16)
    for use_ref in (False, True):
        got = np.zeros((M, N), np.float32)
        oracle.gemm_pooled(bits, M, N, K, Ap, s, B, bs, 64, got, N, use_ref=use_ref)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), use_ref
