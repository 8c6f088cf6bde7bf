"""Python mirror of the reference's kernel wrapper layer.

Each function has the name, argument order, argument meaning and checks of
the safe wrapper it mirrors in crates/fgm-kernels/src/lib.rs; the reference's
``debug_assert!``s are always-on assertions here.  Buffers may be

* numpy arrays (host memory): the call goes to the drop-in ``fgm_*_hip``
  symbol, which moves A / C per call and caches weights on the GPU;
* torch tensors on the GPU: the call goes to the device API
  (``fgm_hip_*_dev``) on torch's current stream, asynchronously.

Mixing the two in one call is an error.
"""
from __future__ import annotations

import enum
import os

import numpy as np

from . import check, lib, HipUnavailable


class Backend(enum.Enum):
    """Which GEMM kernel the process uses (lib.rs:84-100).  The reference's
    Amx / Vnni CPU backends live in the reference; this library is Hip."""

    Hip = "hip"

    def name_str(self) -> str:
        return "hip-gfx950"


_BACKEND = None


def backend() -> Backend:
    """The backend for this process, decided once (lib.rs:112-137).

    ``FGM_BACKEND=hip`` or unset selects the GPU; the reference's CPU values
    (``amx``, ``vnni``) are refused, since those kernels are not in this
    library.  Raises HipUnavailable without a usable gfx950 device."""
    global _BACKEND
    if _BACKEND is None:
        want = os.environ.get("FGM_BACKEND", "hip")
        if want != "hip":
            raise HipUnavailable(f"FGM_BACKEND={want}: this library provides only the hip backend")
        if not lib().fgm_hip_available():
            raise HipUnavailable(lib().fgm_hip_last_error().decode() or "no gfx950 device")
        _BACKEND = Backend.Hip
    return _BACKEND


# ------------------------------------------------------------------ helpers
def _is_dev(x) -> bool:
    return type(x).__module__.startswith("torch") and x.is_cuda


def _kind(*bufs) -> str:
    kinds = {("dev" if _is_dev(b) else "host") for b in bufs if b is not None}
    if len(kinds) != 1:
        raise TypeError("pass either all numpy arrays or all GPU torch tensors")
    return kinds.pop()


def _hp(a: np.ndarray) -> int:
    if not isinstance(a, np.ndarray) or not a.flags["C_CONTIGUOUS"]:
        raise TypeError("host buffers must be C-contiguous numpy arrays")
    return a.ctypes.data


def _dp(t) -> int:
    if not t.is_contiguous():
        raise TypeError("device buffers must be contiguous")
    return t.data_ptr()


def _stream():
    import torch
    return torch.cuda.current_stream().cuda_stream


def _len(x) -> int:
    return x.size if isinstance(x, np.ndarray) else x.numel()


# --------------------------------------------------------------- wrappers
def packed_a_len(m: int, k: int) -> int:
    """Bytes of the tile-packed copy of an m x k activation (lib.rs:153-157)."""
    return (m + 15) // 16 * 16 * k


def pack_a(m: int, k: int, a, ap) -> None:
    """Tile-pack int8 A (lib.rs:159-165)."""
    assert k % 64 == 0
    assert _len(a) >= m * k
    assert _len(ap) >= packed_a_len(m, k)
    backend()
    if _kind(a, ap) == "host":
        lib().fgm_pack_a_hip(m, k, _hp(a), _hp(ap))
    else:
        check(lib().fgm_hip_pack_a_dev(m, k, _dp(a), _dp(ap), _stream()))


def gemm_q4g(m, n, k, a, a_scale, bq, b_scale, group, c, ldc, n0, n1) -> None:
    """C[m, n] = (A int8 * a_scale) . (int4-grouped B * b_scale), columns
    [n0*16, n1*16); `a` tile-packed (lib.rs:167-192).  b_scale: f16 bits."""
    assert k % 64 == 0 and n % 16 == 0
    assert (n1 - n0) % 4 == 0, "n-block range must be a multiple of 4"
    backend()
    if _kind(a, a_scale, bq, b_scale, c) == "host":
        lib().fgm_gemm_q4g_hip(m, n, k, _hp(a), _hp(a_scale), _hp(bq), _hp(b_scale), group,
                               _hp(c), ldc, n0, n1)
    else:
        check(lib().fgm_hip_gemm_q4g_dev(m, n, k, _dp(a), _dp(a_scale), _dp(bq), _dp(b_scale),
                                         group, _dp(c), ldc, n0, n1, _stream()))


def gemm_q8c(m, n, k, a, a_scale, b, b_scale, c, ldc, n0, n1) -> None:
    """C[m, n] = (A int8 * a_scale) . (int8 per-channel B * b_scale)
    (lib.rs:194-217)."""
    assert k % 64 == 0 and n % 16 == 0
    assert (n1 - n0) % 4 == 0, "n-block range must be a multiple of 4"
    backend()
    if _kind(a, a_scale, b, b_scale, c) == "host":
        lib().fgm_gemm_q8c_hip(m, n, k, _hp(a), _hp(a_scale), _hp(b), _hp(b_scale), _hp(c),
                               ldc, n0, n1)
    else:
        check(lib().fgm_hip_gemm_q8c_dev(m, n, k, _dp(a), _dp(a_scale), _dp(b), _dp(b_scale),
                                         _dp(c), ldc, n0, n1, _stream()))


def fwht(x, hsz: int) -> None:
    """In-place normalised fast Walsh-Hadamard transform on blocks of hsz
    (lib.rs:246-252)."""
    n = _len(x)
    assert hsz > 0 and n % hsz == 0 and (hsz & (hsz - 1)) == 0
    backend()
    if _kind(x) == "host":
        lib().fgm_fwht_hip(_hp(x), n, hsz)
    else:
        check(lib().fgm_hip_fwht_dev(_dp(x), n, hsz, _stream()))


def quant_act(x, rows: int, k: int, q, scale) -> None:
    """Per-row symmetric int8 quantisation (lib.rs:254-257)."""
    backend()
    if _kind(x, q, scale) == "host":
        lib().fgm_quant_act_hip(_hp(x), rows, k, _hp(q), _hp(scale))
    else:
        check(lib().fgm_hip_quant_act_dev(_dp(x), rows, k, _dp(q), _dp(scale), _stream()))


def prep_rows(src, lda, rot, qa, qs, pa, m, k, hsz, r0, r1) -> None:
    """Rotate + quantise + tile-pack rows [r0, r1) of a GEMM activation
    (lib.rs:510-529).  On the device path rot / qa may be None (not written)."""
    assert r0 % 16 == 0, "prep row start must be tile-aligned"
    backend()
    if _kind(src, rot, qa, qs, pa) == "host":
        lib().fgm_prep_rows_hip(_hp(src), lda, _hp(rot), _hp(qa), _hp(qs), _hp(pa), m, k, hsz,
                                r0, r1)
    else:
        check(lib().fgm_hip_prep_rows_dev(_dp(src), lda, _dp(rot) if rot is not None else None,
                                          _dp(qa) if qa is not None else None, _dp(qs), _dp(pa),
                                          m, k, hsz, r0, r1, _stream()))


def _opt(t):
    return _dp(t) if t is not None else None


def prep_rmsnorm(x, lda: int, w, eps: float, qs, pa, m: int, k: int, hsz: int, xn=None, rot=None,
                 qa=None, stream=None) -> None:
    """rmsnorm (w None: rmsnorm_noscale) fused with prep_rows over rows
    [0, m) of x: the bytes of rmsnorm (lib.rs:220-228) per row into xn
    followed by prep_rows(xn, k, ...) (lib.rs:517-529), in one launch
    (device tensors; xn, rot and qa are optional outputs)."""
    backend()
    check(lib().fgm_hip_prep_rmsnorm_dev(_dp(x), lda, _opt(w), eps, _opt(xn), _opt(rot), _opt(qa),
                                         _dp(qs), _dp(pa), m, k, hsz,
                                         _stream() if stream is None else stream))


def prep_gelu_mul(gate, up, lda: int, qs, pa, m: int, k: int, hsz: int, act=None, rot=None,
                  qa=None, stream=None) -> None:
    """gelu_mul (lib.rs:231-233) fused with prep_rows over rows [0, m)
    (device tensors; act, rot and qa are optional outputs)."""
    backend()
    check(lib().fgm_hip_prep_gelu_mul_dev(_dp(gate), _dp(up), lda, _opt(act), _opt(rot), _opt(qa),
                                          _dp(qs), _dp(pa), m, k, hsz,
                                          _stream() if stream is None else stream))


# ------------------------------------------------- device-only extensions
def acc_q8c(m, n, k, a, b, acc, ldacc, n0, n1) -> None:
    """Raw int32 accumulators of the q8c GEMM (device tensors)."""
    check(lib().fgm_hip_acc_q8c_dev(m, n, k, _dp(a), _dp(b), _dp(acc), ldacc, n0, n1, _stream()))


def acc_q4g(m, n, k, a, bq, group, acc, ldacc, n0, n1) -> None:
    """Raw per-group int32 accumulators of the q4g GEMM (device tensors),
    acc[(g*m + row)*ldacc + col]."""
    check(lib().fgm_hip_acc_q4g_dev(m, n, k, _dp(a), _dp(bq), group, _dp(acc), ldacc, n0, n1,
                                    _stream()))


def _ptr_or_none(t):
    return None if t is None else _dp(t)


def gemm_batch(problems, stream=None) -> None:
    """Several GEMMs on device tensors in as few launches as possible.

    `problems`: iterable of dicts with keys bits (4 or 8), m, n, k, a, a_scale,
    b, b_scale, c, ldc, n0, n1 and, for bits == 4, group."""
    from . import GemmDesc
    probs = list(problems)
    arr = (GemmDesc * max(1, len(probs)))()
    for i, p in enumerate(probs):
        assert p["k"] % 64 == 0 and p["n"] % 16 == 0
        assert (p["n1"] - p["n0"]) % 4 == 0, "n-block range must be a multiple of 4"
        arr[i] = GemmDesc(p["bits"], p["m"], p["n"], p["k"], p.get("group", 64), _dp(p["a"]),
                          _dp(p["a_scale"]), _dp(p["b"]), _dp(p["b_scale"]), _dp(p["c"]),
                          p["ldc"], p["n0"], p["n1"])
    check(lib().fgm_hip_gemm_batch_dev(arr, len(probs), _stream() if stream is None else stream))


def prep_batch(problems, stream=None) -> None:
    """fgm_prep_rows for several device activations in one launch.  Each dict:
    src, lda, rot, qa, qs, pa, m, k, hsz, r0, r1 (rot / qa may be None)."""
    from . import PrepDesc
    probs = list(problems)
    arr = (PrepDesc * max(1, len(probs)))()
    for i, p in enumerate(probs):
        assert p["r0"] % 16 == 0, "prep row start must be tile-aligned"
        arr[i] = PrepDesc(_dp(p["src"]), p["lda"], _ptr_or_none(p.get("rot")),
                          _ptr_or_none(p.get("qa")), _dp(p["qs"]), _dp(p["pa"]), p["m"], p["k"],
                          p.get("hsz", 0), p["r0"], p["r1"])
    check(lib().fgm_hip_prep_batch_dev(arr, len(probs), _stream() if stream is None else stream))


def gemm_path(bits: int, m: int, k: int, group: int = 64) -> str:
    """'skinny' or 'dense': which kernel family serves this shape."""
    return ("skinny", "dense")[lib().fgm_hip_gemm_path(bits, m, k, group)]


def gemm_plan(bits: int, m: int, n: int, k: int, group: int = 64, n0: int = 0, n1=None) -> int:
    """Launch calls one GEMM of this shape makes (host-only dry run of the
    dispatch, with the drop-ins' shape validation; raises FgmHipError on a
    shape they refuse)."""
    import ctypes
    out = ctypes.c_int(-1)
    check(lib().fgm_hip_gemm_plan(bits, m, n, k, group, n0, n // 16 if n1 is None else n1,
                                  ctypes.byref(out)))
    return out.value


# ------------------------------------------------------ elementwise ops
# lib.rs:220-291.  Host (numpy) buffers go to the drop-ins, GPU tensors to the
# device API on torch's current stream.
def rmsnorm(out, x, w, eps: float) -> None:
    """out = x * (mean(x^2) + eps)^-0.5 * w over n = len(w) (lib.rs:220-223)."""
    n = _len(w)
    assert _len(x) >= n and _len(out) >= n
    backend()
    if _kind(out, x, w) == "host":
        lib().fgm_rmsnorm_hip(_hp(out), _hp(x), _hp(w), n, eps)
    else:
        check(lib().fgm_hip_rmsnorm_dev(_dp(out), _dp(x), _dp(w), 1, n, eps, _stream()))


def rmsnorm_noscale(out, x, n: int, eps: float) -> None:
    """rmsnorm without the learned scale (lib.rs:226-228)."""
    assert _len(x) >= n and _len(out) >= n
    backend()
    if _kind(out, x) == "host":
        lib().fgm_rmsnorm_noscale_hip(_hp(out), _hp(x), n, eps)
    else:
        check(lib().fgm_hip_rmsnorm_dev(_dp(out), _dp(x), None, 1, n, eps, _stream()))


def rmsnorm_rows(out, x, w, rows: int, n: int, eps: float) -> None:
    """Device API only: rmsnorm of `rows` contiguous rows (the forward pass
    calls rmsnorm once per row or head, forward.rs:480-511)."""
    backend()
    if _kind(out, x, w) != "dev":
        raise TypeError("rmsnorm_rows takes GPU tensors")
    check(lib().fgm_hip_rmsnorm_dev(_dp(out), _dp(x), _ptr_or_none(w), rows, n, eps, _stream()))


def gelu_mul(out, gate, up, n: int) -> None:
    """out = gelu_tanh(gate) * up (lib.rs:231-233)."""
    assert _len(gate) >= n and _len(up) >= n and _len(out) >= n
    backend()
    if _kind(out, gate, up) == "host":
        lib().fgm_gelu_mul_hip(_hp(out), _hp(gate), _hp(up), n)
    else:
        check(lib().fgm_hip_gelu_mul_dev(_dp(out), _dp(gate), _dp(up), n, _stream()))


def gelu(x) -> None:
    """In-place gelu_tanh (lib.rs:236-239)."""
    n = _len(x)
    backend()
    if _kind(x) == "host":
        lib().fgm_gelu_hip(_hp(x), n)
    else:
        check(lib().fgm_hip_gelu_mul_dev(_dp(x), _dp(x), None, n, _stream()))


def rope_table(inv_freq: np.ndarray, head_dim: int, pos: int) -> np.ndarray:
    """(cos, sin) pairs for one position, computed on the host with the
    host's libm exactly as ops.c:138-139 does: float32 [head_dim // 2, 2]."""
    inv = np.ascontiguousarray(inv_freq, dtype=np.float32)
    cs = np.empty((head_dim // 2, 2), np.float32)
    lib().fgm_hip_rope_table(cs.ctypes.data, inv.ctypes.data, head_dim, pos)
    return cs


def rope(x, n_heads: int, head_dim: int, inv_freq, pos: int) -> None:
    """In-place half-split rotary embedding of one token's heads
    (lib.rs:242-244).  On the device path inv_freq is a numpy array (host
    side, where the angles are computed)."""
    assert _len(x) >= n_heads * head_dim and head_dim % 2 == 0
    backend()
    if _kind(x) == "host":
        inv = np.ascontiguousarray(inv_freq, dtype=np.float32)
        lib().fgm_rope_hip(_hp(x), n_heads, head_dim, _hp(inv), pos)
    else:
        import torch
        cs = torch.from_numpy(rope_table(inv_freq, head_dim, pos)).to(x.device)
        check(lib().fgm_hip_rope_dev(_dp(x), 1, n_heads, head_dim, _dp(cs), _stream()))
        x._fgm_keep = cs  # keep the table alive until the launch has run


def add(a, b) -> None:
    """a += b over min(len(a), len(b)) (lib.rs:270-273)."""
    n = min(_len(a), _len(b))
    backend()
    if _kind(a, b) == "host":
        lib().fgm_add_hip(_hp(a), _hp(b), n)
    else:
        check(lib().fgm_hip_add_dev(_dp(a), _dp(b), n, _stream()))


def mul(a, b) -> None:
    """a *= b (lib.rs:276-279)."""
    n = min(_len(a), _len(b))
    backend()
    if _kind(a, b) == "host":
        lib().fgm_mul_hip(_hp(a), _hp(b), n)
    else:
        check(lib().fgm_hip_mul_dev(_dp(a), _dp(b), n, _stream()))


def scale(a, s: float) -> None:
    """a *= s (lib.rs:282-285)."""
    n = _len(a)
    backend()
    if _kind(a) == "host":
        lib().fgm_scale_hip(_hp(a), s, n)
    else:
        check(lib().fgm_hip_scale_dev(_dp(a), s, n, _stream()))


def softcap(x, cap: float) -> None:
    """x = cap * tanh(x / cap) (lib.rs:288-291)."""
    n = _len(x)
    backend()
    if _kind(x) == "host":
        lib().fgm_softcap_hip(_hp(x), n, cap)
    else:
        check(lib().fgm_hip_softcap_dev(_dp(x), n, cap, _stream()))



# ------------------------------------------------------ int8-KV attention
# lib.rs:293-372, 428-438.  Host arrays go to the drop-ins (the caches are
# uploaded per call); GPU tensors go to the device API with a scratch buffer
# from torch's allocator.
def attend_scratch(cap: int, head_dim: int) -> int:
    """Floats of scratch attend_q8_heads needs for a cache of `cap` positions
    (lib.rs:340-344)."""
    return cap + (cap + 1) // 2 + 2 * head_dim + 64


def rowbatch_scratch(n_heads: int, cap: int, head_dim: int) -> int:
    """lib.rs:371-373."""
    return int(lib().fgm_rowbatch_scratch_hip(n_heads, cap, head_dim))


def set_scalar_wfill(on: bool) -> None:
    """lib.rs:428-430: an A/B switch the reference's kernels no longer read."""
    lib().fgm_set_scalar_wfill_hip(1 if on else 0)


def _dev_scratch(nbytes: int, like):
    import torch
    return torch.empty(max(nbytes, 256) + 256, dtype=torch.uint8, device=like.device)


def _aligned(t) -> int:
    return (t.data_ptr() + 255) & ~255


def attend_q8_heads(out, q, kc, ks, vc, vs, n_heads: int, kv_heads: int, head_dim: int,
                    start: int, end: int, scratch, h0: int, h1: int, ring: int, cap: int) -> None:
    """Attention of one query row over positions [start, end), heads [h0, h1)
    (lib.rs:317-338; ops.c:378-637).  `scratch` is the reference's host
    scratch (unused by this library; may be None)."""
    assert ring == 0 or _len(kc) >= ring * kv_heads * head_dim
    assert _len(vc) >= (cap + 3) // 4 * 4 * kv_heads * head_dim
    backend()
    if _kind(out, q, kc, ks, vc, vs) == "host":
        lib().fgm_attend_q8_heads_hip(_hp(out), _hp(q), _hp(kc), _hp(ks), _hp(vc), _hp(vs),
                                      n_heads, kv_heads, head_dim, start, end, None, h0, h1,
                                      ring, cap)
    else:
        span = max(end - start, ring, 1)
        nb = lib().fgm_hip_attend_scratch_bytes(1, n_heads, kv_heads, head_dim, span)
        sc = _dev_scratch(nb, out)
        check(lib().fgm_hip_attend_heads_dev(_dp(out), _dp(q), _dp(kc), _dp(ks), _dp(vc),
                                             _dp(vs), n_heads, kv_heads, head_dim, start,
                                             max(end, start), h0, h1, ring, cap, _aligned(sc),
                                             nb, _stream()))
        out._fgm_keep = sc


def attend_q8(out, q, kc, ks, vc, vs, n_heads: int, kv_heads: int, head_dim: int, start: int,
              end: int, scratch=None) -> None:
    """lib.rs:293-309; ops.c:363-368."""
    if _kind(out, q, kc, ks, vc, vs) == "host":
        backend()
        lib().fgm_attend_q8_hip(_hp(out), _hp(q), _hp(kc), _hp(ks), _hp(vc), _hp(vs), n_heads,
                                kv_heads, head_dim, start, end, None)
    else:
        attend_q8_heads(out, q, kc, ks, vc, vs, n_heads, kv_heads, head_dim, start, end,
                        scratch, 0, n_heads, 0, max(end, 1))


def attend_q8_row(out, q, kc, ks, vc, vs, n_heads: int, kv_heads: int, head_dim: int,
                  start: int, end: int, scratch, ring: int, cap: int) -> None:
    """All heads of one query row (lib.rs:353-369; ops.c:729-872): an empty
    range zeroes every head; with one kv head at most eight heads are
    computed, as there."""
    if _kind(out, q, kc, ks, vc, vs) == "host":
        backend()
        lib().fgm_attend_q8_row_hip(_hp(out), _hp(q), _hp(kc), _hp(ks), _hp(vc), _hp(vs),
                                    n_heads, kv_heads, head_dim, start, end, None, ring, cap)
    else:
        h1 = n_heads if (end - start <= 0 or kv_heads != 1) else min(n_heads, 8)
        attend_q8_heads(out, q, kc, ks, vc, vs, n_heads, kv_heads, head_dim, start,
                        max(end, start), scratch, 0, h1, ring, cap)


def store_v_t(vt, src, n: int, slot: int) -> None:
    """One quantised V row into the transposed cache (lib.rs:432-438)."""
    assert _len(vt) >= (slot // 4 + 1) * n * 4 and _len(src) >= n
    backend()
    if _kind(vt, src) == "host":
        lib().fgm_store_v_t_hip(_hp(vt), _hp(src), n, slot)
    else:
        check(lib().fgm_hip_store_v_t_dev(_dp(vt), _dp(src), n, slot, _stream()))


def attend(out, q, seqs, n_heads: int, kv_heads: int, head_dim: int, window: int = 0,
           scratch=None) -> None:
    """Device API only: the reference's AttnJob (pool.rs:36-65) in one call.

    `seqs`: list of (kc, ks, vc, vs, k_len, ring, pos, rows) with GPU tensors
    for the caches; sequence i owns the next `rows` rows of q / out
    ([rows][n_heads][head_dim]) at positions pos, pos + 1, ...  `scratch`: a
    uint8 GPU tensor of at least attend_scratch_bytes(...) + 256 bytes, or None
    to allocate one."""
    import fastgemma_amd as F
    backend()
    arr = (F.AttnSeq * max(len(seqs), 1))()
    rows, span = 0, 1
    for i, (kc, ks, vc, vs, k_len, ring, pos, nr) in enumerate(seqs):
        arr[i] = F.AttnSeq(_dp(kc), _dp(ks), _dp(vc), _dp(vs), k_len, ring, pos, nr)
        rows += nr
        span = max(span, ring, min(pos + nr, window) if window > 0 else pos + nr)
    nb = lib().fgm_hip_attend_scratch_bytes(max(rows, 1), n_heads, kv_heads, head_dim, span)
    sc = scratch if scratch is not None else _dev_scratch(nb, out)
    check(lib().fgm_hip_attend_dev(_dp(out), _dp(q), arr, len(seqs), n_heads, kv_heads, head_dim,
                                   window, _aligned(sc), nb, _stream()))
    out._fgm_keep = sc


def attend_scratch_bytes(rows: int, n_heads: int, kv_heads: int, head_dim: int,
                         max_span: int) -> int:
    return int(lib().fgm_hip_attend_scratch_bytes(rows, n_heads, kv_heads, head_dim, max_span))


def kv_store(k, v, m: int, row_len: int, kc, ks, vt, vs, cap: int, pos: int,
             ring: int = 0) -> None:
    """Device API only: quantise m K / V rows into a layer cache of `cap`
    slots at positions pos .. pos + m - 1 (forward.rs:515-548)."""
    backend()
    check(lib().fgm_hip_kv_store_dev(_dp(k), _dp(v), m, row_len, _dp(kc), _dp(ks), _dp(vt),
                                     _dp(vs), cap, pos, ring, _stream()))
