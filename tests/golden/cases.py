"""Input builders for the golden cases.

Shared by ``make_golden.py`` (which runs the reference's own C, compiled from
its sources into ``oracle/_ref``, on these inputs and records its outputs in
``ref_outputs.json``) and by the tests (which rebuild the same inputs and check
the oracle and the HIP path against the recorded outputs).

The GEMM case lists are the reference's own:

* ``VNNI_CASES`` -- bench/kernels/vnni_test.c:271-284, inputs from its
  xorshift64 (seed 0x243F6A8885A308D3, state carried across cases in the
  order main() runs them, vnni_test.c:39-43,133-176).
* ``AMX_CASE`` -- bench/kernels/gemm_test.c:84-130 (LCG seed 12345), the
  M=40/N=64/K=256/g=64 case and its M=8 decode variant.
* ``DBG_CASE`` -- bench/kernels/dbg.c:21-37 (LCG seed 7, a_scale = 1).
"""
from __future__ import annotations

import numpy as np

import oracle

# (kind, M, N, K, group, n0, n1) in vnni_test.c main() order.
VNNI_CASES = [
    ("q8c", 1, 256, 1536, 0, 0, 16),
    ("q8c", 8, 256, 1536, 0, 0, 16),
    ("q8c", 15, 256, 1536, 0, 0, 16),
    ("q8c", 16, 256, 1536, 0, 0, 16),
    ("q8c", 17, 256, 1536, 0, 0, 16),
    ("q8c", 33, 512, 1536, 0, 4, 12),
    ("q8c", 64, 256, 2048, 0, 0, 16),
    ("q4g", 1, 256, 1536, 128, 0, 16),
    ("q4g", 8, 256, 1536, 128, 0, 16),
    ("q4g", 15, 256, 1536, 64, 0, 16),
    ("q4g", 16, 256, 1536, 256, 0, 16),
    ("q4g", 17, 256, 1536, 128, 0, 16),
    ("q4g", 33, 512, 1536, 128, 4, 12),
    ("q4g", 64, 256, 2048, 128, 0, 16),
]


def _f32(x) -> np.float32:
    return np.float32(x)


def vnni_inputs():
    """Yield (case, inputs) for VNNI_CASES with vnni_test.c's exact inputs.

    inputs = dict(A int8 [M, K], Ap packed, as f32 [M], B (int8 tiles or
    packed int4 bytes), bs (f32 [N] or f16 bits [K/g, N])).
    """
    rs = oracle.XorShift()
    for case in VNNI_CASES:
        kind, M, N, K, group, n0, n1 = case
        KB, NB = K // 64, N // 16
        A = rs.ints(M * K, -127, 127).astype(np.int8).reshape(M, K)
        # as[i] = 0.01f + 0.001f * (i % 7)
        a_s = np.array([_f32(0.01) + _f32(0.001) * _f32(i % 7) for i in range(M)], np.float32)
        if kind == "q8c":
            B = rs.ints(NB * KB * 1024, -127, 127).astype(np.int8)
            bs = np.array([_f32(0.02) + _f32(0.0005) * _f32(i % 11) for i in range(N)],
                          np.float32)
        else:
            B = rs.ints(NB * KB * 512, 0, 255).astype(np.uint8)
            NG = K // group
            bsf = np.array([_f32(0.002) + _f32(0.0001) * _f32(i % 13) for i in range(NG * N)],
                           np.float32)
            bs = bsf.astype(np.float16).view(np.uint16).reshape(NG, N)
        yield case, dict(A=A, Ap=oracle.pack_a(M, K, A), a_s=a_s, B=B, bs=bs)


def amx_inputs():
    """gemm_test.c:84-107's inputs (LCG seed 12345)."""
    M, N, K, group = 40, 64, 256, 64
    KB, NB = K // 64, N // 16
    g = oracle.Lcg(12345)
    A = g.ints(M * K, -127, 127).astype(np.int8).reshape(M, K)
    a_s = np.array([_f32(0.002) + _f32(0.001) * _f32(i % 7) for i in range(M)], np.float32)
    Bq = np.empty(NB * KB * 512, np.uint8)
    for i in range(Bq.size):  # lo first, then hi (gemm_test.c:98-101)
        lo = int(g.ints(1, -8, 7)[0]) & 0xF
        hi = int(g.ints(1, -8, 7)[0]) & 0xF
        Bq[i] = lo | (hi << 4)
    B8 = g.ints(NB * KB * 1024, -127, 127).astype(np.int8)
    bs4f = np.array([_f32(0.01) + _f32(0.001) * _f32(i % 5) for i in range((K // group) * N)],
                    np.float32)
    bs4 = bs4f.astype(np.float16).view(np.uint16).reshape(K // group, N)
    bs8 = np.array([_f32(0.003) + _f32(0.0005) * _f32(i % 11) for i in range(N)], np.float32)
    return dict(M=M, N=N, K=K, group=group, A=A, a_s=a_s, Bq=Bq, B8=B8, bs4=bs4, bs8=bs8)


def dbg_inputs():
    """dbg.c:23-37's inputs (LCG seed 7; a_scale = 1)."""
    M, N, K, group = 2, 64, 128, 64
    KB, NB = K // 64, N // 16
    g = oracle.Lcg(7)
    A = (g.ints(M * K, 0, 8) - 4).astype(np.int8).reshape(M, K)
    Bq = g.ints(NB * KB * 512, 0, 255).astype(np.uint8)
    bsf = np.array([1.0 + 0.25 * (i % 3) for i in range((K // group) * N)], np.float32)
    bs = bsf.astype(np.float16).view(np.uint16).reshape(K // group, N)
    return dict(M=M, N=N, K=K, group=group, A=A, a_s=np.ones(M, np.float32), Bq=Bq, bs=bs)


def layout_inputs():
    """Small q [N, K] matrices packed by the oracle's pack_b_tiles/pack_nibbles;
    the reference kernel run on them with unit scales gives exact integer
    products, pinning the packers to the reference kernel's layout."""
    M, N, K = 5, 64, 192
    A = oracle.gen_i8(31, M * K, -127, 127).reshape(M, K)
    Q8 = oracle.gen_i8(32, N * K, -127, 127).reshape(N, K)
    Q4 = oracle.gen_i8(33, N * K, -8, 7).reshape(N, K)
    return dict(M=M, N=N, K=K, A=A, Q8=Q8, Q4=Q4)


def quant_rows():
    """Activation rows for quant_act / prep_rows goldens: normal, heavy-tailed,
    outlier channels, all-zero, one non-zero, exact .5 ties, +-inf, subnormal
    rows, and a row length that is not a multiple of 16 (the scalar tail)."""
    K = 256
    rows = []
    rows.append(oracle.gen_normal(11, K))
    rows.append(oracle.gen_student_t(12, K, 3))
    r = oracle.gen_normal(13, K)
    r[[5, 77]] *= 20.0
    rows.append(r)
    rows.append(np.zeros(K, np.float32))
    r = np.zeros(K, np.float32)
    r[42] = -3.5
    rows.append(r)
    # amax = 127 -> s = 1, inv = 1: x*inv = x, so k + 0.5 values are exact ties
    r = np.array([(i % 40) - 20 + 0.5 for i in range(K)], np.float32)
    r[0] = 127.0
    rows.append(r)
    r = oracle.gen_normal(14, K)
    r[9] = np.inf
    r[200] = -np.inf
    rows.append(r)
    rows.append((oracle.gen_normal(15, K) * np.float32(1e-39)).astype(np.float32))
    rows.append((oracle.gen_normal(16, K) * np.float32(1e-44)).astype(np.float32))
    rows.append((oracle.gen_normal(17, K) * np.float32(5e37)).astype(np.float32))
    x = np.stack(rows).astype(np.float32)
    tail = oracle.gen_normal(18, 3 * 100).reshape(3, 100)
    tail[1, 97] = 50.0
    tail[2, 99] = np.inf
    return x, tail.astype(np.float32)


def fwht_input(hsz: int) -> np.ndarray:
    return oracle.gen_normal(100 + hsz, 4 * 256).reshape(4, 256)


def prep_input():
    """m=37 rows of k=256 in an lda=300 buffer."""
    m, k, lda = 37, 256, 300
    src = oracle.gen_normal(21, m * lda).reshape(m, lda)
    src[3, 10] = 40.0
    return m, k, lda, src.astype(np.float32)


# ---------------------------------------------------------- elementwise ops
# Row lengths: model dimensions (hidden 2048 / 1536, intermediate 8192, head
# 256 / 512) and ragged ones with a scalar tail (n % 16 != 0), as ops.c's
# vector + tail structure has them.
ELEM_NS = [16, 256, 512, 1536, 2048, 8192, 7, 31, 2063]


def elem_inputs(n: int):
    """Seeded inputs for one row length: x ~ 3 N(0,1), w and up ~ N(0,1),
    gate ~ 2 N(0,1) (reaching exp's clamp region is the softcap input's job:
    20 N(0,1) with cap 30)."""
    x = oracle.gen_normal(0xE1E0 + n, n) * np.float32(3.0)
    w = oracle.gen_normal(0xE1E1 + n, n)
    up = oracle.gen_normal(0xE1E2 + n, n)
    gate = oracle.gen_normal(0xE1E3 + n, n) * np.float32(2.0)
    sc = oracle.gen_normal(0xE1E4 + n, n) * np.float32(20.0)
    return dict(x=x.astype(np.float32), w=w, up=up, gate=gate.astype(np.float32),
                sc=sc.astype(np.float32))


# RoPE: a Gemma-style proportional table (theta 1e6, the last quarter of the
# half-dimension zero: "nope" dims pass through, ops.c:133-134), 8 heads.
ROPE_CASES = [(8, 256, 0), (8, 256, 1), (8, 256, 997), (4, 512, 32767), (2, 64, 5)]


def rope_inputs(n_heads: int, head_dim: int):
    h = head_dim // 2
    j = np.arange(h, dtype=np.float64)
    inv = (1.0e6 ** (-2.0 * j / head_dim)).astype(np.float32)
    inv[3 * h // 4:] = 0.0
    x = oracle.gen_normal(0xA0BE + head_dim, n_heads * head_dim)
    return x, inv



# ------------------------------------------------------ int8-KV attention
# (name, n_heads, kv_heads, head_dim, cap, ring, start, end, h0, h1, qmul, path)
# path: "heads" = fgm_attend_q8_heads, "row" = fgm_attend_q8_row,
# "q8" = fgm_attend_q8.  Caches are filled at every slot.
ATTN_CASES = [
    ("dec256_n1000", 8, 1, 256, 1024, 0, 0, 1000, 0, 8, 1.0, "heads"),
    ("dec512_n4096", 8, 1, 512, 4096, 0, 0, 4096, 0, 8, 1.0, "heads"),
    ("dec512_n4096_row", 8, 1, 512, 4096, 0, 0, 4096, 0, 8, 1.0, "row"),
    ("q8_n777", 8, 1, 256, 800, 0, 0, 777, 0, 8, 1.0, "q8"),
    ("n1", 8, 1, 256, 64, 0, 0, 1, 0, 8, 1.0, "heads"),
    ("n15", 8, 1, 256, 64, 0, 0, 15, 0, 8, 1.0, "heads"),
    ("n16", 8, 1, 256, 64, 0, 0, 16, 0, 8, 1.0, "heads"),
    ("n17_off", 8, 1, 256, 64, 0, 5, 22, 0, 8, 1.0, "heads"),
    ("win_off", 8, 1, 512, 2048, 0, 1023, 1536, 0, 8, 1.0, "heads"),
    ("sharp", 8, 1, 256, 512, 0, 0, 512, 0, 8, 16.0, "heads"),
    ("flat", 8, 1, 256, 512, 0, 0, 512, 0, 8, 0.01, "heads"),
    ("heads_sub", 8, 1, 256, 512, 0, 0, 300, 2, 5, 1.0, "heads"),
    ("gqa_kv2", 8, 2, 256, 512, 0, 0, 333, 0, 8, 1.0, "heads"),
    ("gqa_kv2_row", 8, 2, 256, 512, 0, 0, 333, 0, 8, 1.0, "row"),
    ("row_nh4", 4, 1, 256, 512, 0, 0, 200, 0, 4, 1.0, "row"),
    ("row_nh12", 12, 1, 128, 256, 0, 0, 100, 0, 12, 1.0, "row"),
    ("ring_nowrap", 8, 1, 256, 520, 520, 100, 612, 0, 8, 1.0, "heads"),
    ("ring_wrap", 8, 1, 256, 520, 520, 1301, 1813, 0, 8, 1.0, "heads"),
    ("ring_full", 8, 1, 256, 520, 520, 3000, 3520, 0, 8, 1.0, "heads"),
    ("ring_gap1", 8, 1, 256, 100, 100, 150, 249, 0, 8, 1.0, "heads"),
    ("ring_row", 8, 1, 256, 520, 520, 1301, 1813, 0, 8, 1.0, "row"),
    ("ring_odd", 8, 1, 256, 77, 77, 60, 120, 0, 8, 1.0, "heads"),
    ("empty", 8, 1, 256, 64, 0, 10, 10, 0, 8, 1.0, "heads"),
    ("empty_row", 8, 1, 256, 64, 0, 10, 10, 0, 8, 1.0, "row"),
]


def attn_inputs(name: str, n_heads: int, kv_heads: int, head_dim: int, cap: int, qmul: float):
    """Seeded query and cache: K, V ~ U[-1, 1) per element, quantised per slot
    as the forward pass writes them; q ~ qmul * U[-1, 1) (qmul sets how peaked
    the softmax is, as in the reference's bench/kernels/attn_test.c).  Head 1
    of the query is all zeros (qamax = 0: uniform attention)."""
    seed = sum(ord(c) * (i + 1) for i, c in enumerate(name)) & 0xFFFF
    kvd = kv_heads * head_dim
    kv = oracle.KvLayer(cap, kv_heads, head_dim)
    kf = oracle.gen_uniform(0xA77E0 + seed, cap * kvd, -1.0, 1.0).reshape(cap, kvd)
    vf = oracle.gen_uniform(0xA77E1 + seed, cap * kvd, -1.0, 1.0).reshape(cap, kvd)
    for t in range(cap):
        kv.store(t, kf[t], vf[t])
    q = oracle.gen_uniform(0xA77E2 + seed, n_heads * head_dim, -1.0, 1.0) * np.float32(qmul)
    q = q.astype(np.float32)
    if n_heads > 1:
        q[head_dim:2 * head_dim] = 0.0
    return q, kv


# BASELINE-shaped cases (seeded splitmix64 inputs through the oracle's
# generators): prep_rows (hsz 0) of fp32 rows, then the GEMM.  The reference's
# bytes for them are recorded by make_golden.py; the negative controls
# (tests/test_negative_controls.py) show that plausible wrong epilogues and
# nibble conventions change them.
#   name: (kind, M, N, K, group, activation)
BASELINE_CASES = {
    "cfg1_q8c_m1": ("q8c", 1, 8192, 2048, 0, "normal"),
    "cfg2_up_q4g_m8": ("q4g", 8, 8192, 2048, 64, "normal"),
    "cfg2_down_q4g_m8": ("q4g", 8, 2048, 8192, 64, "normal"),
    # accumulators past 2^24 whose per-64-k partial sums are not round: the
    # case that tells a single int32 -> float conversion from float partials
    "bigacc_q8c_m16": ("q8c", 16, 256, 8192, 0, "bigacc"),
    # int4 group sums near 2^16 (|a| ~ 120, |w| in 5..8, signs matched), so
    # (float)acc_g * s needs more than 24 bits: the case that tells the fused
    # per-group fma from a multiply and an add
    "bigacc_q4g_m16": ("q4g", 16, 256, 2048, 64, "bigacc"),
    # cfg5's heavy tail (Student-t nu=3, 0.1% of channels x20), 64 rows
    "cfg5_down_q8c_m64": ("q8c", 64, 256, 8192, 0, "heavy"),
}


def baseline_inputs(name: str):
    """(x f32 [M, K], B, bs) of one BASELINE_CASES entry."""
    kind, M, N, K, group, act = BASELINE_CASES[name]
    seed = 1000 + sum(ord(c) for c in name)
    if act == "normal":
        x = oracle.gen_normal(seed, M * K).reshape(M, K)
    elif act == "heavy":
        x = oracle.gen_student_t(seed, M * K, 3).reshape(M, K)
        hot = np.arange(K) % 1000 == 7             # 0.1% of the channels
        x[:, hot] *= np.float32(20.0)
    else:                                          # |x| in [0.8, 1] with random signs
        mag = oracle.gen_uniform(seed, M * K, 0.8, 1.0)
        sgn = np.where(oracle.gen_u8(seed + 1, M * K) & 1, 1.0, -1.0).astype(np.float32)
        x = (mag * sgn).reshape(M, K)
    if kind == "q8c":
        if act == "bigacc":                        # weights in +-[100, 127] with A's signs per k
            w = oracle.gen_i8(seed + 2, N * K, 100, 127).reshape(N, K).astype(np.int16)
            w = (w * np.where(x[0] < 0, -1, 1)[None, :]).astype(np.int8)
        else:
            w = oracle.gen_i8(seed + 2, N * K, -127, 127).reshape(N, K)
        B = oracle.pack_b_tiles(w)
        bs = oracle.gen_uniform(seed + 3, N, 1e-3, 1e-2)
    elif act == "bigacc":                          # int4 in +-[5, 8] with A's signs per k
        w = oracle.gen_i8(seed + 2, N * K, 5, 8).reshape(N, K).astype(np.int16)
        w = np.where(x[0] < 0, -1, 1)[None, :] * w
        w = np.where(w == 8, 7, w).astype(np.int8)     # int4 holds -8..7
        B = oracle.pack_nibbles(oracle.pack_b_tiles(w))
        bs = oracle.f32_to_f16(oracle.gen_uniform(seed + 3, (K // group) * N, 5e-3, 5e-2)).reshape(K // group, N)
    else:
        B = oracle.gen_u8(seed + 2, N * K // 2)
        bs = oracle.f32_to_f16(oracle.gen_uniform(seed + 3, (K // group) * N, 5e-3, 5e-2)).reshape(K // group, N)
    return np.ascontiguousarray(x, np.float32), B, bs
