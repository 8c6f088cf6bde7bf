"""GPU edge cases of the GEMM entry points:

* the reference's recorded bytes for the BASELINE.json-shaped golden cases
  (prep_rows, then the GEMM), the same cases the negative controls use;
* an empty contraction (k == 0) through the device API writes zeros to
  columns [16 n0, 16 n1) of rows < m and nothing else (vnni_gemm.c:232-243),
  with a fill kernel rather than a memset;
* dense int8 shapes whose K is 64 times an odd number, so a K group's last
  pipeline stage holds only zero-padded k-blocks;
* a weight of more than 2^30 bytes, which the library cuts into launches along
  N with rebased pointers: columns on both sides of each cut against the
  oracle.

Bar: bit-exact (int32 accumulators and fp32 outputs).
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

import oracle
from tests import hip_util as H
from tests.golden import cases

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "ref_outputs.json")))


def _bits_equal(x, y):
    return np.array_equal(np.ascontiguousarray(x).view(np.uint32), np.ascontiguousarray(y).view(np.uint32))


@pytest.mark.parametrize("name", list(cases.BASELINE_CASES))
def test_baseline_golden_cases(name):
    """GPU prep_rows + GEMM equal the reference's recorded bytes."""
    from fastgemma_amd import kernels as K
    kind, M, N, Kd, group, _ = cases.BASELINE_CASES[name]
    print(name, flush=True)
    x, B, bs = cases.baseline_inputs(name)
    t = H.torch()
    qs = t.zeros(M, device="cuda")
    pa = t.zeros(oracle.packed_a_len(M, Kd), dtype=t.int8, device="cuda")
    K.prep_rows(H.dev(x), Kd, None, None, qs, pa, M, Kd, 0, 0, M)
    C = t.zeros((M, N), device="cuda")
    if kind == "q8c":
        K.gemm_q8c(M, N, Kd, pa, qs, H.dev(B), H.dev(bs), C, N, 0, N // 16)
    else:
        K.gemm_q4g(M, N, Kd, pa, qs, H.dev(B), H.dev(bs), group, C, N, 0, N // 16)
    g = GOLD["baseline"][name]
    assert H.sha(H.host(qs), H.host(pa)) == g["prep_sha256"]
    assert H.sha(H.host(C)) == g["c_sha256"]


@pytest.mark.parametrize("kind", ["q8c", "q4g"])
@pytest.mark.parametrize("M", [8, 256])
def test_empty_contraction_writes_zeros_in_range_only(kind, M):
    from fastgemma_amd import kernels as K
    t = H.torch()
    N, ldc, n0, n1 = 256, 272, 4, 12
    C = t.full((M + 2, ldc), 7.0, device="cuda")
    one = t.ones(1, device="cuda")
    dummy = t.zeros(64, dtype=t.int8, device="cuda")
    if kind == "q8c":
        K.gemm_q8c(M, N, 0, dummy, one, dummy, one, C, ldc, n0, n1)
    else:
        K.gemm_q4g(M, N, 0, dummy, one, dummy.view(t.uint8), dummy.view(t.int16), 64, C, ldc, n0, n1)
    got = H.host(C)
    want = np.full((M + 2, ldc), 7.0, np.float32)
    want[:M, 16 * n0:16 * n1] = 0.0
    assert np.array_equal(got, want)


@pytest.mark.parametrize("M,N,Kd", [(2048, 2048, 4160), (256, 2048, 576), (256, 2048, 1088), (256, 512, 8256)])
def test_dense_odd_k_blocks(M, N, Kd):
    """K = 64 * odd: the K-group variants end on stages of zero-padded
    k-blocks (K = 4160 takes the kmin >= 4096 path)."""
    from fastgemma_amd import kernels as K
    print("q8c", M, N, Kd, K.gemm_path(8, M, Kd), flush=True)
    A = oracle.gen_i8(17 + Kd, M * Kd, -127, 127).reshape(M, Kd)
    Ap = oracle.pack_a(M, Kd, A)
    a_s = oracle.gen_uniform(18 + Kd, M, 1e-3, 1e-2)
    B = oracle.gen_i8(19 + Kd, N * Kd, -127, 127)
    bs = oracle.gen_uniform(20 + Kd, N, 1e-3, 1e-2)
    acc = H.gpu_acc("q8c", M, N, Kd, Ap, B)
    want = H.exact_acc(A, H.decode_b8(B, N, Kd))
    assert np.array_equal(acc, want)
    C = H.gpu_gemm("q8c", M, N, Kd, Ap, a_s, B, bs)
    R = want.astype(np.float32) * (bs[None, :] * a_s[:, None])
    assert _bits_equal(C, R.astype(np.float32))


@pytest.mark.parametrize("M", [8, 128])
def test_weight_past_1gib_is_cut_along_n(M):
    """int8 N=73728 K=16384 (1.21 GB of weights): launches of at most 2^30
    bytes of B, i.e. 4096 n-blocks each; n-blocks at the start, on both sides
    of the cut and at the end equal the oracle on the same bytes."""
    from fastgemma_amd import kernels as K
    t = H.torch()
    N, Kd = 73728, 16384
    print("q8c chunked", M, N, Kd, K.gemm_path(8, M, Kd), flush=True)
    g = t.Generator(device="cuda")
    g.manual_seed(1234 + M)
    B = t.randint(-127, 128, (N * Kd,), dtype=t.int8, device="cuda", generator=g)
    bs = t.rand(N, device="cuda", generator=g) * 0.009 + 0.001
    A = oracle.gen_i8(55 + M, M * Kd, -127, 127).reshape(M, Kd)
    Ap = oracle.pack_a(M, Kd, A)
    a_s = oracle.gen_uniform(56 + M, M, 1e-3, 1e-2)
    C = t.full((M, N), 3.0, device="cuda")
    K.gemm_q8c(M, N, Kd, H.dev(Ap), H.dev(a_s), B, bs, C, N, 0, N // 16)
    got = H.host(C)
    for nb0, nb1 in ((0, 4), (4092, 4100), (N // 16 - 4, N // 16)):
        sub = H.host(B[nb0 * Kd * 16:nb1 * Kd * 16])
        sbs = H.host(bs[16 * nb0:16 * nb1])
        n = 16 * (nb1 - nb0)
        R = np.zeros((M, n), np.float32)
        oracle.gemm_q8c(M, n, Kd, Ap, a_s, sub, sbs, R, n, 0, n // 16)
        assert _bits_equal(got[:, 16 * nb0:16 * nb1], R), (nb0, nb1)
    del B


@pytest.mark.parametrize("kind", ["q8c", "q4g"])
@pytest.mark.parametrize("M", [256, 96])
def test_dropin_dense_column_range(kind, M):
    """Host-pointer drop-ins on the dense kernel with a column range that does
    not start at 0 (the reference's pool hands each thread [n0, n1),
    pool.rs:119-145): every written value equals the oracle, the rest of C is
    untouched.  Regression: the drop-in passes a C base shifted by 16 n0
    columns, and the dense epilogue's store range once dropped the last row
    of every tile for such a base."""
    from fastgemma_amd import kernels as K
    N, Kd, n0, n1 = 1024, 2048, 12, 44
    A = oracle.gen_i8(81, M * Kd, -127, 127).reshape(M, Kd)
    Ap = oracle.pack_a(M, Kd, A)
    a_s = oracle.gen_uniform(82, M, 1e-3, 1e-2)
    if kind == "q8c":
        B = oracle.gen_i8(83, N * Kd, -127, 127)
        bs = oracle.gen_uniform(84, N, 1e-3, 1e-2)
    else:
        B = oracle.gen_u8(83, N * Kd // 2)
        bs = oracle.gen_uniform(84, (Kd // 64) * N, 5e-3, 5e-2).astype(np.float16).view(np.uint16)
    C = np.full((M, N), -5.0, np.float32)
    W = np.full((M, N), -5.0, np.float32)
    if kind == "q8c":
        K.gemm_q8c(M, N, Kd, Ap, a_s, B, bs, C, N, n0, n1)
        oracle.gemm_q8c(M, N, Kd, Ap, a_s, B, bs, W, N, n0, n1)
    else:
        K.gemm_q4g(M, N, Kd, Ap, a_s, B, bs, 64, C, N, n0, n1)
        oracle.gemm_q4g(M, N, Kd, Ap, a_s, B, bs, 64, W, N, n0, n1)
    assert K.gemm_path(8 if kind == "q8c" else 4, M, Kd) == "dense"
    assert _bits_equal(C, W)
    assert np.all(C[:, :16 * n0] == -5.0) and np.all(C[:, 16 * n1:] == -5.0)


@pytest.mark.parametrize("M", [8, 128])
def test_int4_weight_past_1gib_is_cut_along_n(M):
    """int4 group 64, N=163840 K=16384 (1.34 GB of weights): launches of at
    most 2^30 bytes of B (8192 n-blocks each), the f16 scale table rebased by
    16 columns per n-block with N kept as its row stride; n-blocks at the
    start, on both sides of the cut and at the end equal the oracle on the
    same bytes, on the skinny (M=8) and the dense (M=128) kernel."""
    from fastgemma_amd import kernels as K
    t = H.torch()
    N, Kd, G = 163840, 16384, 64
    print("q4g chunked", M, N, Kd, K.gemm_path(4, M, Kd, G), flush=True)
    g = t.Generator(device="cuda")
    g.manual_seed(4321 + M)
    B = t.randint(0, 256, (N * Kd // 2,), dtype=t.uint8, device="cuda", generator=g)
    bs = (t.rand((Kd // G) * N, device="cuda", generator=g) * 0.045 + 0.005).half().view(t.int16)
    A = oracle.gen_i8(65 + M, M * Kd, -127, 127).reshape(M, Kd)
    Ap = oracle.pack_a(M, Kd, A)
    a_s = oracle.gen_uniform(66 + M, M, 1e-3, 1e-2)
    C = t.full((M, N), 3.0, device="cuda")
    K.gemm_q4g(M, N, Kd, H.dev(Ap), H.dev(a_s), B, bs, G, C, N, 0, N // 16)
    got = H.host(C)
    bs_h = H.host(bs).view(np.uint16).reshape(Kd // G, N)
    for nb0, nb1 in ((0, 4), (8188, 8196), (N // 16 - 4, N // 16)):
        sub = H.host(B[nb0 * Kd * 8:nb1 * Kd * 8])
        sbs = np.ascontiguousarray(bs_h[:, 16 * nb0:16 * nb1])
        n = 16 * (nb1 - nb0)
        R = np.zeros((M, n), np.float32)
        oracle.gemm_q4g(M, n, Kd, Ap, a_s, sub, sbs, G, R, n, 0, n // 16)
        assert _bits_equal(got[:, 16 * nb0:16 * nb1], R), (nb0, nb1)
    del B


def test_single_n_block_past_1gib_launches_whole():
    """int8, M=8, K = 2^26 + 64: one n-block holds 16 K > 2^30 bytes of B, so
    every cut along N is a lone n-block, launched as it is (once the cause of
    an unbounded recursion on the host).  A is zero outside three k-blocks
    (the first, one in the middle, the last), so the result equals the
    oracle's on the problem reduced to those k-blocks, bit for bit."""
    from fastgemma_amd import kernels as K
    t = H.torch()
    M, N, Kd = 8, 64, (1 << 26) + 64
    KB = Kd // 64
    kbs = [0, KB // 2, KB - 1]
    print("q8c lone n-block", M, N, Kd, K.gemm_path(8, M, Kd), flush=True)
    g = t.Generator(device="cuda")
    g.manual_seed(99)
    B = t.randint(-127, 128, (N * Kd,), dtype=t.int8, device="cuda", generator=g)
    bs = oracle.gen_uniform(71, N, 1e-3, 1e-2)
    a_s = oracle.gen_uniform(72, M, 1e-3, 1e-2)
    Ar = oracle.gen_i8(73, M * 192, -127, 127).reshape(M, 192)
    Apr = oracle.pack_a(M, 192, Ar)             # [1][3][16][64]: one 1 KB chunk per k-block
    Ap = t.zeros(16 * Kd, dtype=t.int8, device="cuda")
    for i, kb in enumerate(kbs):
        Ap[kb * 1024:(kb + 1) * 1024] = H.dev(Apr[i * 1024:(i + 1) * 1024])
    C = t.full((M, N), 3.0, device="cuda")
    K.gemm_q8c(M, N, Kd, Ap, H.dev(a_s), B, H.dev(bs), C, N, 0, N // 16)
    got = H.host(C)
    Br = np.concatenate([H.host(B[(nb * KB + kb) * 1024:(nb * KB + kb + 1) * 1024])
                         for nb in range(N // 16) for kb in kbs])
    R = np.zeros((M, N), np.float32)
    oracle.gemm_q8c(M, N, 192, Apr, a_s, Br, bs, R, N, 0, N // 16)
    assert _bits_equal(got, R)
    del B, Ap
