"""The allocation-free Gemm::run (fgm_hip_linear_run_noalloc_dev): its scratch
is a file-scope device array, not a caller buffer.  Its output must equal,
byte for byte, fgm_hip_linear_run_dev with a caller scratch on the same
inputs -- on two calls in a row, the second with a smaller input, so that
whatever the first call left in the shared array cannot reach the second's
result.  Calls go through the C ABI (ctypes)."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import oracle
from fastgemma_amd import FgmHipError, LinearInfo, check, lib
from tests import hip_util as H

pytestmark = pytest.mark.gpu


def weight(bits, n, k, group, hadamard, seed):
    """A resident linear weight as the C struct fgm_hip_linear, plus the
    tensors that keep its device memory alive."""
    if bits == 8:
        b = H.dev(oracle.gen_i8(seed, n * k, -127, 127))
        s = H.dev(oracle.gen_uniform(seed + 1, n, 1e-3, 1e-2))
    else:
        b = H.dev(oracle.gen_u8(seed, n * k // 2))
        s = H.dev(oracle.gen_uniform(seed + 1, (k // group) * n, 5e-3, 5e-2).astype(
            np.float16).view(np.uint16))
    info = LinearInfo(bits, n, k, group if bits == 4 else 0, hadamard, b.data_ptr(), s.data_ptr(),
                      None, None)
    return info, (b, s)


def stream():
    return H.torch().cuda.current_stream().cuda_stream


def run_with_scratch(info, x, m, lda):
    t = H.torch()
    out = t.full((m, info.n), 7.0, dtype=t.float32, device="cuda")
    nb = lib().fgm_hip_linear_scratch_bytes(m, info.k)
    sc = t.empty(nb, dtype=t.uint8, device="cuda")
    check(lib().fgm_hip_linear_run_dev(C.byref(info), x.data_ptr(), m, lda, out.data_ptr(),
                                       sc.data_ptr(), nb, stream()))
    return H.host(out)


def run_noalloc(info, x, m, lda):
    t = H.torch()
    out = t.full((m, info.n), -7.0, dtype=t.float32, device="cuda")
    check(lib().fgm_hip_linear_run_noalloc_dev(C.byref(info), x.data_ptr(), m, lda,
                                               out.data_ptr(), stream()))
    return H.host(out)


def same_bits(a, b):
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


# (bits, n, k, group, hadamard, m first call, m second call): decode rows on the
# skinny kernel, prefill rows on the dense one, both weight types, rotations
CASES = [
    (4, 2048, 8192, 64, 128, 8, 3),
    (8, 1024, 2048, 0, 0, 256, 40),
    (4, 512, 2048, 128, 0, 200, 1),
    (8, 2048, 8192, 0, 128, 64, 17),
]


@pytest.mark.parametrize("case", CASES, ids=[f"q{c[0]}_n{c[1]}_k{c[2]}_h{c[4]}" for c in CASES])
def test_noalloc_equals_linear_run(case):
    bits, n, k, group, hadamard, m1, m2 = case
    info, keep = weight(bits, n, k, group, hadamard, seed=n + k + bits)
    for i, m in enumerate((m1, m2)):
        x = H.dev((oracle.gen_normal(100 * i + m, m * k) * 2.0).reshape(m, k))
        want = run_with_scratch(info, x, m, k)
        got = run_noalloc(info, x, m, k)
        assert same_bits(got, want), f"call {i + 1} (m={m}): no-alloc output differs"
    del keep


def test_noalloc_refuses_beyond_its_limit():
    limit = lib().fgm_hip_linear_noalloc_max_bytes()
    assert limit == 8 << 20
    info, keep = weight(8, 64, 8192, 0, 0, seed=5)
    m = 1024  # 1024 rows x 8192 bytes of packed A is past 8 MiB
    assert lib().fgm_hip_linear_scratch_bytes(m, 8192) > limit
    t = H.torch()
    x = t.zeros((m, 8192), dtype=t.float32, device="cuda")
    out = t.zeros((m, 64), dtype=t.float32, device="cuda")
    with pytest.raises(FgmHipError, match="no-alloc"):
        check(lib().fgm_hip_linear_run_noalloc_dev(C.byref(info), x.data_ptr(), m, 8192,
                                                   out.data_ptr(), stream()))
    del keep
