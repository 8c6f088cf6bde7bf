"""Helpers for the GPU tests: move numpy inputs to the device, call the HIP
path through the C ABI (fastgemma_amd's mirror of lib.rs), bring results back.
torch is used only for device memory and the stream."""
from __future__ import annotations

import hashlib

import numpy as np

import fastgemma_amd as F
from fastgemma_amd import kernels as K


def torch():
    import torch as _t
    return _t


def dev(x: np.ndarray):
    return torch().from_numpy(np.ascontiguousarray(x)).cuda()


def host(t) -> np.ndarray:
    torch().cuda.synchronize()
    return t.cpu().numpy()


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def gpu_gemm(kind, M, N, Kd, Ap, a_s, B, bs, group=64, n0=0, n1=None, ldc=None, fill=0.0):
    """Run the device GEMM; C starts filled with `fill` (untouched entries keep it)."""
    t = torch()
    n1 = N // 16 if n1 is None else n1
    ldc = N if ldc is None else ldc
    C = t.full((max(M, 1), ldc), fill, dtype=t.float32, device="cuda")
    dA, das, dB, dbs = dev(Ap), dev(a_s), dev(B), dev(bs)
    if kind == "q8c":
        K.gemm_q8c(M, N, Kd, dA, das, dB, dbs, C, ldc, n0, n1)
    else:
        K.gemm_q4g(M, N, Kd, dA, das, dB, dbs, group, C, ldc, n0, n1)
    return host(C)[:M]


def gpu_acc(kind, M, N, Kd, Ap, B, group=64, n0=0, n1=None):
    """Raw int32 accumulators: q8c [M, N]; q4g [K/group, M, N]."""
    t = torch()
    n1 = N // 16 if n1 is None else n1
    rows = M if kind == "q8c" else (Kd // group) * M
    acc = t.zeros((rows, N), dtype=t.int32, device="cuda")
    if kind == "q8c":
        K.acc_q8c(M, N, Kd, dev(Ap), dev(B), acc, N, n0, n1)
        return host(acc)
    K.acc_q4g(M, N, Kd, dev(Ap), dev(B), group, acc, N, n0, n1)
    return host(acc).reshape(Kd // group, M, N)


def decode_b8(blob: np.ndarray, n: int, k: int) -> np.ndarray:
    """VNNI tile stream -> q [N, K] (inverse of quant.py:105-107)."""
    t = blob.astype(np.int8).reshape(n // 16, k // 64, 16, 16, 4)
    return np.ascontiguousarray(t.transpose(0, 3, 1, 2, 4)).reshape(n, k)


def decode_b4(bq: np.ndarray, n: int, k: int) -> np.ndarray:
    p = bq.reshape(-1, 32)
    lo = ((p & 0x0F).astype(np.int16) ^ 8) - 8
    hi = (((p >> 4) & 0x0F).astype(np.int16) ^ 8) - 8
    flat = np.concatenate([lo, hi], axis=1).reshape(-1).astype(np.int8)
    return decode_b8(flat, n, k)


def exact_acc(A: np.ndarray, Q: np.ndarray) -> np.ndarray:
    """A[M,K] @ Q[N,K].T exactly: float64 BLAS is exact while |sum| < 2^53."""
    return (A.astype(np.float64) @ Q.astype(np.float64).T).astype(np.int64)


def exact_group_acc(A: np.ndarray, Q: np.ndarray, group: int) -> np.ndarray:
    M, Kd = A.shape
    out = np.empty((Kd // group, M, Q.shape[0]), np.int64)
    for g in range(Kd // group):
        sl = slice(g * group, (g + 1) * group)
        out[g] = exact_acc(A[:, sl], Q[:, sl])
    return out
