"""The skinny kernel's park-in-ring variant (int4, M <= 8, group 64, grids of
more than 2048 workgroups): the tile sums go back into the ring slot their
weights came from and each wave streams a contiguous run of units.  Every
shape below yields 4096 or more workgroups, so the variant runs; the bytes
must equal the oracle's gemm_q4g (vnni_gemm.c:291-322 restated), tolerance 0,
and the untouched columns stay untouched."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests import hip_util as H

pytestmark = pytest.mark.gpu


def run(M, N, K, seed, n0=0, n1=None, group=64):
    n1 = N // 16 if n1 is None else n1
    A = oracle.gen_i8(seed, M * K, -127, 127).reshape(M, K)
    Ap = oracle.pack_a(M, K, A)
    a_s = oracle.gen_uniform(seed + 1, M, 1e-3, 1e-2)
    B = oracle.gen_u8(seed + 2, N * K // 2)
    bs = oracle.gen_uniform(seed + 3, (K // group) * N, 5e-3, 5e-2).astype(np.float16).view(
        np.uint16).reshape(K // group, N)
    got = H.gpu_gemm("q4g", M, N, K, Ap, a_s, B, bs, group, n0, n1, fill=-9.0)
    want = np.full((M, N), -9.0, np.float32)
    oracle.gemm_q4g(M, N, K, Ap, a_s, B, bs, group, want, N, n0, n1)
    return got, want


def same(a, b):
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


# (M, N, K): 4096 workgroups at K = 2048 (4 stream waves) and K = 8192 (16),
# an odd k-tile count (K = 576), two k-tiles (K = 128), one (K = 64),
# every row count
CASES = [(8, 65536, 2048), (8, 65536, 8192), (5, 131072, 576), (3, 131072, 1024), (1, 65536, 2048),
         (8, 262144, 128), (7, 262144, 64), (2, 65536, 4096)]


@pytest.mark.parametrize("case", CASES, ids=[f"m{c[0]}_n{c[1]}_k{c[2]}" for c in CASES])
def test_park_in_ring_matches_oracle(case):
    M, N, K = case
    got, want = run(M, N, K, seed=M + N + K)
    assert same(got, want), f"{int((got.view(np.uint32) != want.view(np.uint32)).sum())} words differ"


def test_park_in_ring_n_range():
    """A column range inside a large grid: only [16 n0, 16 n1) is written."""
    got, want = run(8, 131072, 2048, seed=5, n0=100, n1=7000)
    assert same(got, want)
    assert np.all(got[:, :1600] == -9.0) and np.all(got[:, 7000 * 16:] == -9.0)


def test_park_in_ring_batch_gate_up():
    """Two up-projection-like problems in one launch (4096 workgroups)."""
    from fastgemma_amd import kernels as K
    t = H.torch()
    outs, wants, probs = [], [], []
    A = oracle.gen_i8(31, 8 * 2048, -127, 127).reshape(8, 2048)
    Ap = oracle.pack_a(8, 2048, A)
    a_s = oracle.gen_uniform(32, 8, 1e-3, 1e-2)
    dA, das = H.dev(Ap), H.dev(a_s)
    N = 32768
    for i in range(2):
        B = oracle.gen_u8(40 + i, N * 1024)
        bs = oracle.gen_uniform(50 + i, 32 * N, 5e-3, 5e-2).astype(np.float16).view(np.uint16)
        c = t.full((8, N), -9.0, dtype=t.float32, device="cuda")
        outs.append(c)
        probs.append(dict(bits=4, m=8, n=N, k=2048, a=dA, a_scale=das, b=H.dev(B), b_scale=H.dev(bs),
                          c=c, ldc=N, n0=0, n1=N // 16, group=64))
        w = np.full((8, N), -9.0, np.float32)
        oracle.gemm_q4g(8, N, 2048, Ap, a_s, B, bs.reshape(32, N), 64, w, N, 0, N // 16)
        wants.append(w)
    K.gemm_batch(probs)
    for c, w in zip(outs, wants):
        assert same(H.host(c), w)
