"""Negative controls: the parity checks reject plausible wrong variants.

The reference's journal records a case where a kernel and its scalar
reference agreed bit for bit while both decoded int4 nibbles the wrong way
(JOURNAL.md:1908-1937; vnni_test.c:62-69 was added because of it).  A byte
comparison is only evidence if it fails for the neighbouring conventions, so
each test here plants one mistake in the ORACLE (on the CPU, through
``oracle.fault``; see the orc_fault table in oracle/fgm_oracle.c) and checks
that the reference's recorded bytes reject it, while the unmodified oracle
matches them:

  1  q8c epilogue (float)acc * as * bs             vnni_test.c:72-85
  2  q8c per-64-k-tile float sums, then * (as*bs)  amx_gemm.c:500-522
  3  int4 nibbles as offset binary v - 8           JOURNAL.md:1908-1937
  4  q4g unfused (float)acc * s + C                amx_gemm.c:478-498
  5  q4g groups in descending order
  6  quant_act truncating instead of rounding half to even
  10 attention softmax sum as one serial chain     ops.c:493-505
  11 attention P.V counting a slot that two ring spans share once  ops.c:605-631

The cases are BASELINE.json-shaped (cfg1 M=1 N=8192 K=2048 int8; cfg2 M=8
int4 g64 up and down; a cfg5-style heavy-tailed int8 case) plus two whose
accumulators are large enough for rounding to matter: on ordinary N(0,1) rows
variant 2's per-tile float sums and variant 4's unfused products are exact
and so indistinguishable, which this file records too.
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


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def run_case(name):
    """The oracle's prep_rows + GEMM on one BASELINE case: (prep digest, C digest)."""
    kind, M, N, K, group, _ = cases.BASELINE_CASES[name]
    x, B, bs = cases.baseline_inputs(name)
    rot = np.zeros((M, K), np.float32)
    qa = np.zeros((M, K), np.int8)
    qs = np.zeros(M, np.float32)
    pa = np.zeros(oracle.packed_a_len(M, K), np.int8)
    oracle.prep_rows(x, K, rot, qa, qs, pa, M, K, 0, 0, M)
    C = np.zeros((M, N), np.float32)
    if kind == "q8c":
        oracle.gemm_q8c(M, N, K, pa, qs, B, bs, C, N, 0, N // 16)
    else:
        oracle.gemm_q4g(M, N, K, pa, qs, B, bs, group, C, N, 0, N // 16)
    return sha(qs, pa), sha(C)


@pytest.mark.parametrize("name", list(cases.BASELINE_CASES))
def test_oracle_matches_reference_on_baseline_shapes(name):
    p, c = run_case(name)
    g = GOLD["baseline"][name]
    assert p == g["prep_sha256"] and c == g["c_sha256"]


# fault -> the cases whose recorded bytes must reject it
REJECTS = {
    1: ["cfg1_q8c_m1", "cfg5_down_q8c_m64"],
    2: ["bigacc_q8c_m16"],
    3: ["cfg2_up_q4g_m8", "cfg2_down_q4g_m8"],
    4: ["bigacc_q4g_m16"],
    5: ["cfg2_up_q4g_m8", "cfg2_down_q4g_m8", "bigacc_q4g_m16"],
    6: ["cfg1_q8c_m1", "cfg2_up_q4g_m8", "cfg5_down_q8c_m64"],
}


@pytest.mark.parametrize("fault,names", list(REJECTS.items()), ids=[f"fault{k}" for k in REJECTS])
def test_planted_gemm_mistakes_fail_the_golden_bytes(fault, names):
    for name in names:
        with oracle.fault(fault):
            p, c = run_case(name)
        g = GOLD["baseline"][name]
        assert (p, c) != (g["prep_sha256"], g["c_sha256"]), (fault, name)
    # and the switch is off again
    p, c = run_case(names[0])
    assert c == GOLD["baseline"][names[0]]["c_sha256"]


def test_variants_invisible_on_small_accumulators():
    """Variant 2 on cfg1 (|acc| << 2^24) and variant 4 on cfg2 (per-group
    products of at most 24 bits): every partial result is exact, so the bytes
    agree -- the reason the bigacc cases exist."""
    with oracle.fault(2):
        _, c = run_case("cfg1_q8c_m1")
    assert c == GOLD["baseline"]["cfg1_q8c_m1"]["c_sha256"]
    with oracle.fault(4):
        _, c = run_case("cfg2_up_q4g_m8")
    assert c == GOLD["baseline"]["cfg2_up_q4g_m8"]["c_sha256"]


def test_planted_mistakes_fail_the_reference_vnni_cases():
    """The reference's own vnni_test.c cases reject the int4 variants too."""
    for fault in (3, 5):
        bad = 0
        for (case, inp), rec in zip(cases.vnni_inputs(), GOLD["vnni"]):
            kind, M, N, K, group, n0, n1 = case
            if kind != "q4g":
                continue
            C = np.zeros((M, N), np.float32)
            with oracle.fault(fault):
                oracle.gemm_q4g(M, N, K, inp["Ap"], inp["a_s"], inp["B"], inp["bs"], group, C, N, n0, n1)
            bad += sha(C) != rec["sha256"]
        assert bad >= 5, (fault, bad)


# ---------------------------------------------------------------- attention
def attn_digest(case):
    name, nh, kvh, hd, cap, ring, st, en, h0, h1, qmul, path = case
    q, kv = cases.attn_inputs(name, nh, kvh, hd, cap, qmul)
    o = np.full(nh * hd, 7.0, np.float32)
    if path == "row":
        oracle.attend_row(q, kv, nh, st, en, ring, out=o)
    elif path == "q8":
        oracle.attend_heads(q, kv, nh, st, en, 0, nh, 0, out=o)
    else:
        oracle.attend_heads(q, kv, nh, st, en, h0, h1, ring, out=o)
    return hashlib.sha256(o.tobytes()).hexdigest()


@pytest.mark.parametrize("fault", [10, 11])
def test_planted_attention_mistakes_fail_the_golden_bytes(fault):
    """A serial softmax sum (10) and a span double count dropped (11) each
    change at least one of the reference's recorded attention cases; the
    unmodified oracle matches all of them."""
    rejected = []
    for case in cases.ATTN_CASES:
        with oracle.fault(fault):
            d = attn_digest(case)
        if d != GOLD["attn"][case[0]]["sha256"]:
            rejected.append(case[0])
    assert rejected, fault
    if fault == 11:
        # only ring_gap1 (ring 100, positions [150, 249): runs [50, 100) and
        # [0, 49), whose four-slot spans share slots 48..51) has such a slot
        assert rejected == ["ring_gap1"], rejected
    for case in cases.ATTN_CASES[:4]:
        assert attn_digest(case) == GOLD["attn"][case[0]]["sha256"]
