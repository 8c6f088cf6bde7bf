"""CPU oracle for the fgm-kernels quantized-matmul path -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker; the product library
(``fastgemma_amd``) never touches it.

Two CPU implementations are reachable from here:

* ``liboracle.so`` -- ``fgm_oracle.c``, a scalar C restatement of the reference
  algorithm (file:line citations in that file), plus the pthread pool in
  ``cpu_pool.c`` that reproduces the reference's N-split.
* ``_ref/libfgmref.so`` / ``_ref/libfgmref_amx.so`` -- the reference's own
  ``vnni_gemm.c`` + ``ops.c`` / ``amx_gemm.c`` compiled from their sources by
  ``oracle/Makefile`` (built only where ``/root/reference`` exists; the built
  files travel with the tree).  ``ref()`` / ``ref_amx()`` return ``None`` when a
  library is missing or the host CPU lacks the ISA it needs.

How each oracle function is pinned (reference outputs, known answers, closed
forms, brute force) is documented and checked in ``tests/test_oracle.py``.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None
_REF_AMX = None

_i = C.c_int
_p = C.c_void_p
_u64 = C.c_uint64
_sz = C.c_size_t
_f = C.c_float


def _build_oracle() -> None:
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)


def lib() -> C.CDLL:
    """The oracle library (built on first use if absent)."""
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            _build_oracle()
        L = C.CDLL(path)
        L.orc_f16_to_f32.restype = _f
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [_f]
        L.orc_quant_act.argtypes = [_p, _i, _i, _p, _p]
        L.orc_packed_a_len.restype = _sz
        L.orc_packed_a_len.argtypes = [_i, _i]
        L.orc_pack_a.argtypes = [_i, _i, _p, _p]
        L.orc_fwht.argtypes = [_p, _i, _i]
        L.orc_prep_rows.argtypes = [_p, _i, _p, _p, _p, _p, _i, _i, _i, _i, _i]
        L.orc_pack_b_tiles.argtypes = [_p, _i, _i, _p]
        L.orc_pack_nibbles.argtypes = [_p, _sz, _p]
        L.orc_unpack_nibbles.argtypes = [_p, _sz, _p]
        L.orc_acc_q8c.argtypes = [_i, _i, _p, _p, _p, _i, _i, _i]
        L.orc_gemm_q8c.argtypes = [_i, _i, _i, _p, _p, _p, _p, _p, _i, _i, _i]
        L.orc_acc_q4g.argtypes = [_i, _i, _p, _p, _i, _p, _i, _i, _i]
        L.orc_gemm_q4g.argtypes = [_i, _i, _i, _p, _p, _p, _p, _i, _p, _i, _i, _i]
        L.orc_epilogue_q8c.argtypes = [_i, _p, _i, _p, _p, _p, _i, _i, _i]
        L.orc_epilogue_q4g.argtypes = [_i, _i, _i, _p, _i, _p, _p, _p, _i, _i, _i]
        L.orc_gen_i8.argtypes = [_u64, _sz, _i, _i, _p]
        L.orc_gen_u8.argtypes = [_u64, _sz, _p]
        L.orc_gen_uniform.argtypes = [_u64, _sz, _f, _f, _p]
        L.orc_gen_normal.argtypes = [_u64, _sz, _p]
        L.orc_gen_student_t.argtypes = [_u64, _sz, _i, _p]
        L.orc_exp16.restype = _f
        L.orc_exp16.argtypes = [_f]
        L.orc_rmsnorm.argtypes = [_p, _p, _p, _i, _f]
        L.orc_rmsnorm_noscale.argtypes = [_p, _p, _i, _f]
        L.orc_gelu_mul.argtypes = [_p, _p, _p, _i]
        L.orc_gelu.argtypes = [_p, _i]
        L.orc_rope.argtypes = [_p, _i, _i, _p, _i]
        L.orc_add.argtypes = [_p, _p, _i]
        L.orc_mul.argtypes = [_p, _p, _i]
        L.orc_scale.argtypes = [_p, _f, _i]
        L.orc_softcap.argtypes = [_p, _i, _f]
        L.orc_attend_q8_heads.argtypes = [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i,
                                          _i, _i]
        L.orc_attend_q8.argtypes = [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i]
        L.orc_attend_q8_row.argtypes = [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i]
        L.orc_store_v_t.argtypes = [_p, _p, _i, _i]
        L.orc_rowbatch_scratch.restype = _i
        L.orc_gather_q8r.argtypes = [_p, _p, _p, _i, _i]
        L.orc_gather_q4r.argtypes = [_p, _p, _p, _i, _i]
        L.orc_rowbatch_scratch.argtypes = [_i, _i, _i]
        L.orc_xorshift_fill.restype = _u64
        L.orc_xorshift_fill.argtypes = [_u64, _sz, _i, _i, _p]
        L.orc_lcg_fill.restype = C.c_uint32
        L.orc_lcg_fill.argtypes = [C.c_uint32, _sz, _i, _i, _p]
        L.orc_pool_start.restype = _i
        L.orc_pool_start.argtypes = [_i]
        L.orc_pool_q8c.argtypes = [_p, _i, _i, _i, _p, _p, _p, _p, _p, _i, _i, _p]
        L.orc_pool_q4g.argtypes = [_p, _i, _i, _i, _p, _p, _p, _p, _i, _p, _i, _i, _p]
        L.orc_pool_prep.argtypes = [_p, _p, _i, _p, _p, _p, _p, _i, _i, _i, _i, _p]
        _LIB = L
    return _LIB


class fault:
    """Context manager that makes the oracle compute one deliberately wrong
    variant (see the orc_fault table in fgm_oracle.c), for negative controls:
    ``with oracle.fault(1): ...``.  Test infrastructure only."""

    def __init__(self, kind: int):
        self.kind = kind

    def __enter__(self):
        v = C.c_int.in_dll(lib(), "orc_fault")
        self.prev = v.value
        v.value = self.kind
        return self

    def __exit__(self, *exc):
        C.c_int.in_dll(lib(), "orc_fault").value = self.prev
        return False


def _bind_ref(L: C.CDLL) -> None:
    L.fgm_cpu_has_amx.restype = _i
    L.fgm_cpu_has_avx512_vnni.restype = _i
    for name in ("fgm_gemm_q8c_vnni",):
        getattr(L, name).argtypes = [_i, _i, _i, _p, _p, _p, _p, _p, _i, _i, _i]
    L.fgm_gemm_q4g_vnni.argtypes = [_i, _i, _i, _p, _p, _p, _p, _i, _p, _i, _i, _i]
    L.fgm_quant_act.argtypes = [_p, _i, _i, _p, _p]
    L.fgm_pack_a.argtypes = [_i, _i, _p, _p]
    L.fgm_fwht.argtypes = [_p, _i, _i]
    L.fgm_prep_rows.argtypes = [_p, _i, _p, _p, _p, _p, _i, _i, _i, _i, _i]
    L.fgm_rmsnorm.argtypes = [_p, _p, _p, _i, _f]
    L.fgm_rmsnorm_noscale.argtypes = [_p, _p, _i, _f]
    L.fgm_gelu_mul.argtypes = [_p, _p, _p, _i]
    L.fgm_gelu.argtypes = [_p, _i]
    L.fgm_rope.argtypes = [_p, _i, _i, _p, _i]
    L.fgm_add.argtypes = [_p, _p, _i]
    L.fgm_mul.argtypes = [_p, _p, _i]
    L.fgm_scale.argtypes = [_p, _f, _i]
    L.fgm_softcap.argtypes = [_p, _i, _f]
    L.fgm_attend_q8.argtypes = [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p]
    L.fgm_attend_q8_heads.argtypes = [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _i, _i,
                                      _i, _i]
    L.fgm_attend_q8_row.argtypes = [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _i, _i]
    L.fgm_store_v_t.argtypes = [_p, _p, _i, _i]
    L.fgm_rowbatch_scratch.restype = _i
    L.fgm_gather_q8r.argtypes = [_p, _p, _p, _i, _i]
    L.fgm_gather_q4r.argtypes = [_p, _p, _p, _i, _i]
    L.fgm_rowbatch_scratch.argtypes = [_i, _i, _i]


def ref() -> C.CDLL | None:
    """The reference's own VNNI path (vnni_gemm.c + ops.c), or None."""
    global _REF
    if _REF is None:
        path = os.path.join(HERE, "_ref", "libfgmref.so")
        if not os.path.exists(path):
            return None
        L = C.CDLL(path)
        _bind_ref(L)
        if not L.fgm_cpu_has_avx512_vnni():
            return None
        _REF = L
    return _REF


def ref_amx() -> C.CDLL | None:
    """The reference's own AMX path (amx_gemm.c), or None (no file / no AMX)."""
    global _REF_AMX
    if _REF_AMX is None:
        r = ref()
        path = os.path.join(HERE, "_ref", "libfgmref_amx.so")
        if r is None or not r.fgm_cpu_has_amx() or not os.path.exists(path):
            return None
        L = C.CDLL(path)
        L.fgm_amx_init.restype = _i
        L.fgm_gemm_q8c.argtypes = [_i, _i, _i, _p, _p, _p, _p, _p, _i, _i, _i]
        L.fgm_gemm_q4g.argtypes = [_i, _i, _i, _p, _p, _p, _p, _i, _p, _i, _i, _i]
        if not L.fgm_amx_init():
            return None
        _REF_AMX = L
    return _REF_AMX


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


# --------------------------------------------------------------- generators
def gen_i8(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    out = np.empty(n, np.int8)
    lib().orc_gen_i8(seed, n, lo, hi, _ptr(out))
    return out


def gen_u8(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint8)
    lib().orc_gen_u8(seed, n, _ptr(out))
    return out


def gen_uniform(seed: int, n: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_gen_uniform(seed, n, lo, hi, _ptr(out))
    return out


def gen_normal(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_gen_normal(seed, n, _ptr(out))
    return out


def gen_student_t(seed: int, n: int, nu: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_gen_student_t(seed, n, nu, _ptr(out))
    return out


class XorShift:
    """vnni_test.c:39-43's generator with its running state."""

    def __init__(self, state: int = 0x243F6A8885A308D3):
        self.s = state

    def ints(self, n: int, lo: int, hi: int) -> np.ndarray:
        out = np.empty(n, np.int32)
        self.s = lib().orc_xorshift_fill(self.s, n, lo, hi, _ptr(out))
        return out


class Lcg:
    """gemm_test.c:30-31's generator with its running state."""

    def __init__(self, state: int = 12345):
        self.s = state

    def ints(self, n: int, lo: int, hi: int) -> np.ndarray:
        out = np.empty(n, np.int32)
        self.s = lib().orc_lcg_fill(self.s, n, lo, hi, _ptr(out))
        return out


# ------------------------------------------------------------------ helpers
def f16_to_f32(h: np.ndarray) -> np.ndarray:
    L = lib()
    h = np.ascontiguousarray(h, np.uint16)
    return np.array([L.orc_f16_to_f32(int(v)) for v in h.ravel()], np.float32).reshape(h.shape)


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    L = lib()
    x = np.ascontiguousarray(x, np.float32)
    return np.array([L.orc_f32_to_f16(float(v)) for v in x.ravel()], np.uint16).reshape(x.shape)


def packed_a_len(m: int, k: int) -> int:
    return (m + 15) // 16 * 16 * k


# ----------------------------------------------------------------- the path
def quant_act(x: np.ndarray, rows: int, k: int):
    """fgm_quant_act (ops.c:181-204) -> (q int8 [rows, k], scale f32 [rows])."""
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty((rows, k), np.int8)
    s = np.empty(rows, np.float32)
    lib().orc_quant_act(_ptr(x), rows, k, _ptr(q), _ptr(s))
    return q, s


def pack_a(m: int, k: int, a: np.ndarray) -> np.ndarray:
    """fgm_pack_a (ops.c:279-290)."""
    a = np.ascontiguousarray(a, np.int8)
    ap = np.empty(packed_a_len(m, k), np.int8)
    lib().orc_pack_a(m, k, _ptr(a), _ptr(ap))
    return ap


def fwht(x: np.ndarray, hsz: int) -> np.ndarray:
    """fgm_fwht (ops.c:153-175), returns a rotated copy."""
    y = np.array(x, np.float32, copy=True, order="C")
    lib().orc_fwht(_ptr(y), y.size, hsz)
    return y


def prep_rows(src, lda, rot, qa, qs, pa, m, k, hsz, r0, r1) -> None:
    """fgm_prep_rows (ops.c:293-314), in place on caller buffers."""
    lib().orc_prep_rows(_ptr(src), lda, _ptr(rot), _ptr(qa), _ptr(qs), _ptr(pa),
                        m, k, hsz, r0, r1)


def pack_b_tiles(q: np.ndarray) -> np.ndarray:
    """pack_b_tiles (quant.py:96-107): q [N, K] int8 -> VNNI tile stream."""
    q = np.ascontiguousarray(q, np.int8)
    n, k = q.shape
    out = np.empty(n * k, np.int8)
    lib().orc_pack_b_tiles(_ptr(q), n, k, _ptr(out))
    return out


def pack_nibbles(flat: np.ndarray) -> np.ndarray:
    """pack_nibbles (quant.py:76-82)."""
    flat = np.ascontiguousarray(flat, np.int8)
    out = np.empty(flat.size // 2, np.uint8)
    lib().orc_pack_nibbles(_ptr(flat), flat.size, _ptr(out))
    return out


def unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    """unpack_nibbles (quant.py:85-92)."""
    packed = np.ascontiguousarray(packed, np.uint8)
    out = np.empty(packed.size * 2, np.int8)
    lib().orc_unpack_nibbles(_ptr(packed), out.size, _ptr(out))
    return out


def acc_q8c(m, k, ap, b, n0, n1, ldacc):
    acc = np.zeros((m, ldacc), np.int32)
    lib().orc_acc_q8c(m, k, _ptr(ap), _ptr(b), _ptr(acc), ldacc, n0, n1)
    return acc


def acc_q4g(m, k, ap, bq, group, n0, n1, ldacc):
    acc = np.zeros((k // group, m, ldacc), np.int32)
    lib().orc_acc_q4g(m, k, _ptr(ap), _ptr(bq), group, _ptr(acc), ldacc, n0, n1)
    return acc


def epilogue_q8c(m, acc, ldacc, a_scale, b_scale, c, ldc, n0, n1) -> None:
    """q8c epilogue (vnni_gemm.c:206-219) on given int32 accumulators."""
    lib().orc_epilogue_q8c(m, _ptr(acc), ldacc, _ptr(a_scale), _ptr(b_scale), _ptr(c), ldc,
                           n0, n1)


def epilogue_q4g(m, n, ng, acc, ldacc, a_scale, b_scale, c, ldc, n0, n1) -> None:
    """q4g group chain (vnni_gemm.c:258-285, 316-321) on given per-group
    accumulators acc[(g*m + row)*ldacc + col]."""
    lib().orc_epilogue_q4g(m, n, ng, _ptr(acc), ldacc, _ptr(a_scale), _ptr(b_scale), _ptr(c),
                           ldc, n0, n1)


def gemm_q8c(m, n, k, ap, a_scale, b, b_scale, c, ldc, n0, n1) -> None:
    """fgm_gemm_q8c_vnni (vnni_gemm.c:224-245), in place on c."""
    lib().orc_gemm_q8c(m, n, k, _ptr(ap), _ptr(a_scale), _ptr(b), _ptr(b_scale), _ptr(c),
                       ldc, n0, n1)


def gemm_q4g(m, n, k, ap, a_scale, bq, b_scale, group, c, ldc, n0, n1) -> None:
    """fgm_gemm_q4g_vnni (vnni_gemm.c:291-322), in place on c."""
    lib().orc_gemm_q4g(m, n, k, _ptr(ap), _ptr(a_scale), _ptr(bq), _ptr(b_scale), group,
                       _ptr(c), ldc, n0, n1)


def gemm_pooled(bits, m, n, k, ap, a_scale, b, b_scale, group, c, ldc, use_ref=True) -> str:
    """gemm_q8c / gemm_q4g over all of [0, n/16), split across host threads
    the way fgm-core's pool splits a GEMM (cpu_pool.c, pool.rs:110-145): the
    reference's own VNNI kernels when oracle/_ref is built and the host has
    AVX-512 VNNI (use_ref), else the oracle's scalar restatement.  Columns are
    independent, so the bytes equal one call over the whole range.  Returns
    which ran ("reference" / "oracle")."""
    L = lib()
    R = ref() if use_ref else None
    nt = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    L.orc_pool_start(max(1, min(nt, 64)))
    t1 = np.empty(1, np.float64)
    try:
        if bits == 8:
            fn = C.cast(R.fgm_gemm_q8c_vnni if R is not None else L.orc_gemm_q8c, C.c_void_p).value
            L.orc_pool_q8c(fn, m, n, k, _ptr(ap), _ptr(a_scale), _ptr(b), _ptr(b_scale), _ptr(c), ldc, 1,
                           _ptr(t1))
        else:
            fn = C.cast(R.fgm_gemm_q4g_vnni if R is not None else L.orc_gemm_q4g, C.c_void_p).value
            L.orc_pool_q4g(fn, m, n, k, _ptr(ap), _ptr(a_scale), _ptr(b), _ptr(b_scale), group, _ptr(c),
                           ldc, 1, _ptr(t1))
    finally:
        L.orc_pool_stop()
    return "reference" if R is not None else "oracle"


# ------------------------------------------------------- elementwise ops
# Restatements of ops.c's f32 primitives (fgm_oracle.c cites the lines).  All
# take and return numpy float32 arrays; the in-place reference functions get
# a copy.
def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def exp16(x: float) -> float:
    return lib().orc_exp16(x)


def rmsnorm(x: np.ndarray, w: np.ndarray | None, eps: float) -> np.ndarray:
    """One row (``fgm_rmsnorm``); ``w=None`` is ``fgm_rmsnorm_noscale``."""
    x = _f32(x)
    out = np.empty_like(x)
    if w is None:
        lib().orc_rmsnorm_noscale(_ptr(out), _ptr(x), x.size, eps)
    else:
        w = _f32(w)
        lib().orc_rmsnorm(_ptr(out), _ptr(x), _ptr(w), x.size, eps)
    return out


def gelu_mul(gate: np.ndarray, up: np.ndarray | None) -> np.ndarray:
    """``fgm_gelu_mul`` (``up=None``: ``fgm_gelu``)."""
    g = _f32(gate)
    if up is None:
        out = g.copy()
        lib().orc_gelu(_ptr(out), out.size)
        return out
    u = _f32(up)
    out = np.empty_like(g)
    lib().orc_gelu_mul(_ptr(out), _ptr(g), _ptr(u), g.size)
    return out


def rope(x: np.ndarray, n_heads: int, head_dim: int, inv_freq: np.ndarray, pos: int) -> np.ndarray:
    out = _f32(x).copy()
    inv = _f32(inv_freq)
    lib().orc_rope(_ptr(out), n_heads, head_dim, _ptr(inv), pos)
    return out


def add(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    out = _f32(a).copy()
    lib().orc_add(_ptr(out), _ptr(_f32(b)), out.size)
    return out


def mul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    out = _f32(a).copy()
    lib().orc_mul(_ptr(out), _ptr(_f32(b)), out.size)
    return out


def scale(a: np.ndarray, s: float) -> np.ndarray:
    out = _f32(a).copy()
    lib().orc_scale(_ptr(out), s, out.size)
    return out


def softcap(x: np.ndarray, cap: float) -> np.ndarray:
    out = _f32(x).copy()
    lib().orc_softcap(_ptr(out), out.size, cap)
    return out



# ------------------------------------------------------ int8-KV attention
class KvLayer:
    """One layer's int8 KV cache in the reference's layout (kv.rs:13-50):
    kc [cap][kvd] int8, ks [cap] f32, vt transposed in groups of four slots
    ([ceil(cap/4)][kvd][4] int8), vs [cap] f32."""

    def __init__(self, cap: int, kv_heads: int, head_dim: int):
        self.cap, self.kvh, self.hd = cap, kv_heads, head_dim
        kvd = kv_heads * head_dim
        self.kc = np.zeros(cap * kvd, np.int8)
        self.ks = np.zeros(cap, np.float32)
        self.vt = np.zeros((cap + 3) // 4 * 4 * kvd, np.int8)
        self.vs = np.zeros(cap, np.float32)

    def store(self, slot: int, krow: np.ndarray, vrow: np.ndarray) -> None:
        """The forward pass's write (forward.rs:515-548): quant_act each row,
        K in place, V through store_v_t."""
        kvd = self.kvh * self.hd
        q, s = quant_act(krow, 1, kvd)
        self.kc[slot * kvd:(slot + 1) * kvd] = q[0]
        self.ks[slot] = s[0]
        q, s = quant_act(vrow, 1, kvd)
        store_v_t(self.vt, q[0], slot)
        self.vs[slot] = s[0]


def store_v_t(vt: np.ndarray, src: np.ndarray, slot: int) -> None:
    src = np.ascontiguousarray(src, np.int8)
    lib().orc_store_v_t(_ptr(vt), _ptr(src), src.size, slot)


def tail_noncr() -> int:
    """Tail expf values (since the last reset) that were not the correctly
    rounded exp."""
    return C.c_int.in_dll(lib(), "orc_attn_tail_noncr").value


def reset_tail_noncr() -> None:
    C.c_int.in_dll(lib(), "orc_attn_tail_noncr").value = 0


def attend_heads(q, kv: KvLayer, n_heads: int, start: int, end: int, h0: int = 0,
                 h1: int | None = None, ring: int = 0, out=None) -> np.ndarray:
    """fgm_attend_q8_heads (ops.c:378-637) on a KvLayer; out [n_heads * hd]
    (heads outside [h0, h1) keep `out`'s values)."""
    h1 = n_heads if h1 is None else h1
    q = _f32(q)
    out = np.zeros(n_heads * kv.hd, np.float32) if out is None else out
    lib().orc_attend_q8_heads(_ptr(out), _ptr(q), _ptr(kv.kc), _ptr(kv.ks), _ptr(kv.vt),
                              _ptr(kv.vs), n_heads, kv.kvh, kv.hd, start, end, h0, h1, ring,
                              kv.cap)
    return out


def attend_row(q, kv: KvLayer, n_heads: int, start: int, end: int, ring: int = 0,
               out=None) -> np.ndarray:
    """fgm_attend_q8_row (ops.c:729-872)."""
    q = _f32(q)
    out = np.zeros(n_heads * kv.hd, np.float32) if out is None else out
    lib().orc_attend_q8_row(_ptr(out), _ptr(q), _ptr(kv.kc), _ptr(kv.ks), _ptr(kv.vt),
                            _ptr(kv.vs), n_heads, kv.kvh, kv.hd, start, end, ring, kv.cap)
    return out


def ref_attend(kind: str, q, kv: KvLayer, n_heads: int, start: int, end: int, h0: int = 0,
               h1: int | None = None, ring: int = 0, out=None) -> np.ndarray | None:
    """The reference's own fgm_attend_q8{,_heads,_row} (oracle/_ref), or None."""
    R = ref()
    if R is None:
        return None
    h1 = n_heads if h1 is None else h1
    q = _f32(q)
    out = np.zeros(n_heads * kv.hd, np.float32) if out is None else out
    scratch = np.zeros(R.fgm_rowbatch_scratch(n_heads, kv.cap, kv.hd) + 4 * kv.cap + 256,
                       np.float32)
    args = (_ptr(out), _ptr(q), _ptr(kv.kc), _ptr(kv.ks), _ptr(kv.vt), _ptr(kv.vs), n_heads,
            kv.kvh, kv.hd, start, end, _ptr(scratch))
    if kind == "q8":
        R.fgm_attend_q8(*args)
    elif kind == "heads":
        R.fgm_attend_q8_heads(*args, h0, h1, ring, kv.cap)
    else:
        R.fgm_attend_q8_row(*args, ring, kv.cap)
    return out


# ---------------------------------------------------------- gather tables
def gather(bits: int, tbl: np.ndarray, sc: np.ndarray, row: int, k: int) -> np.ndarray:
    """fgm_gather_q8r / fgm_gather_q4r (ops.c:208-251)."""
    out = np.empty(k, np.float32)
    f = lib().orc_gather_q8r if bits == 8 else lib().orc_gather_q4r
    f(_ptr(out), _ptr(tbl), _ptr(sc), row, k)
    return out


def ref_gather(bits: int, tbl: np.ndarray, sc: np.ndarray, row: int, k: int):
    R = ref()
    if R is None:
        return None
    out = np.empty(k, np.float32)
    f = R.fgm_gather_q8r if bits == 8 else R.fgm_gather_q4r
    f(_ptr(out), _ptr(tbl), _ptr(sc), row, k)
    return out
