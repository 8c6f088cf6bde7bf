"""fastgemma_amd -- MI355X (gfx950) implementation of fastgemma's fgm-kernels
quantized-matmul path.

The product is the C-ABI library ``libfgm_hip.so`` (declared in
``include/fgm_hip.h``); this package loads it and mirrors, in Python, the
reference's safe wrapper layer over that ABI (crates/fgm-kernels/src/lib.rs),
so host code and tests can call the path with the reference's names, argument
meaning and checks.

There is no CPU fallback: if the library is missing, or no gfx950 device is
usable when a kernel is called, the call raises.
"""
from __future__ import annotations

import ctypes as _C
import os as _os

HERE = _os.path.dirname(_os.path.abspath(__file__))
LIB_PATH = _os.path.join(HERE, "libfgm_hip.so")
_LIB = None


class HipUnavailable(RuntimeError):
    """The HIP library is not built or no gfx950 device is usable."""


class FgmHipError(RuntimeError):
    """A device-API call returned a non-zero status."""


def lib() -> _C.CDLL:
    """Load libfgm_hip.so (raises HipUnavailable if it was not built)."""
    global _LIB
    if _LIB is None:
        if not _os.path.exists(LIB_PATH):
            raise HipUnavailable(
                f"{LIB_PATH} is missing: build it with `make -C fastgemma_amd/csrc` "
                "or __graft_entry__.build()")
        # torch (the test and benchmark plumbing) ships its own HIP runtime
        # under the same soname as the system one this library links; the
        # first one loaded serves the whole process, and torch only
        # initialises the GPU through its own.  Load it first when present.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = _C.CDLL(LIB_PATH)
        _bind(L)
        _LIB = L
    return _LIB


def _bind(L: _C.CDLL) -> None:
    i, p, f = _C.c_int, _C.c_void_p, _C.c_float
    L.fgm_hip_last_error.restype = _C.c_char_p
    L.fgm_hip_available.restype = i
    L.fgm_hip_init.argtypes = [i]
    L.fgm_hip_gemm_path.argtypes = [i, i, i, i]
    L.fgm_hip_gemm_plan.argtypes = [i, i, i, i, i, i, i, _C.POINTER(i)]
    L.fgm_hip_weight_cache_bytes.argtypes = [i]
    L.fgm_hip_weight_cache_bytes.restype = _C.c_size_t
    dev_q8c = [i, i, i, p, p, p, p, p, i, i, i, p]
    dev_q4g = [i, i, i, p, p, p, p, i, p, i, i, i, p]
    L.fgm_hip_gemm_q8c_dev.argtypes = dev_q8c
    L.fgm_hip_gemm_q4g_dev.argtypes = dev_q4g
    L.fgm_hip_acc_q8c_dev.argtypes = [i, i, i, p, p, p, i, i, i, p]
    L.fgm_hip_acc_q4g_dev.argtypes = [i, i, i, p, p, i, p, i, i, i, p]
    L.fgm_hip_prep_rows_dev.argtypes = [p, i, p, p, p, p, i, i, i, i, i, p]
    L.fgm_hip_quant_act_dev.argtypes = [p, i, i, p, p, p]
    L.fgm_hip_pack_a_dev.argtypes = [i, i, p, p, p]
    L.fgm_hip_fwht_dev.argtypes = [p, i, i, p]
    L.fgm_gemm_q8c_hip.argtypes = [i, i, i, p, p, p, p, p, i, i, i]
    L.fgm_gemm_q4g_hip.argtypes = [i, i, i, p, p, p, p, i, p, i, i, i]
    L.fgm_pack_a_hip.argtypes = [i, i, p, p]
    L.fgm_prep_rows_hip.argtypes = [p, i, p, p, p, p, i, i, i, i, i]
    L.fgm_quant_act_hip.argtypes = [p, i, i, p, p]
    L.fgm_fwht_hip.argtypes = [p, i, i]
    L.fgm_hip_gemm_batch_dev.argtypes = [p, i, p]
    L.fgm_hip_prep_batch_dev.argtypes = [p, i, p]
    L.fgm_hip_prep_rmsnorm_dev.argtypes = [p, i, p, f, p, p, p, p, p, i, i, i, p]
    L.fgm_hip_prep_gelu_mul_dev.argtypes = [p, p, i, p, p, p, p, p, i, i, i, p]
    L.fgm_rmsnorm_hip.argtypes = [p, p, p, i, f]
    L.fgm_rmsnorm_noscale_hip.argtypes = [p, p, i, f]
    L.fgm_gelu_mul_hip.argtypes = [p, p, p, i]
    L.fgm_gelu_hip.argtypes = [p, i]
    L.fgm_rope_hip.argtypes = [p, i, i, p, i]
    L.fgm_add_hip.argtypes = [p, p, i]
    L.fgm_mul_hip.argtypes = [p, p, i]
    L.fgm_scale_hip.argtypes = [p, f, i]
    L.fgm_softcap_hip.argtypes = [p, i, f]
    L.fgm_hip_rmsnorm_dev.argtypes = [p, p, p, i, i, f, p]
    L.fgm_hip_gelu_mul_dev.argtypes = [p, p, p, i, p]
    L.fgm_hip_softcap_dev.argtypes = [p, i, f, p]
    L.fgm_hip_rope_table.argtypes = [p, p, i, i]
    L.fgm_hip_rope_dev.argtypes = [p, i, i, i, p, p]
    L.fgm_hip_add_dev.argtypes = [p, p, i, p]
    L.fgm_hip_mul_dev.argtypes = [p, p, i, p]
    L.fgm_hip_scale_dev.argtypes = [p, f, i, p]
    L.fgm_attend_q8_hip.argtypes = [p, p, p, p, p, p, i, i, i, i, i, p]
    L.fgm_attend_q8_heads_hip.argtypes = [p, p, p, p, p, p, i, i, i, i, i, p, i, i, i, i]
    L.fgm_attend_q8_row_hip.argtypes = [p, p, p, p, p, p, i, i, i, i, i, p, i, i]
    L.fgm_store_v_t_hip.argtypes = [p, p, i, i]
    L.fgm_set_scalar_wfill_hip.argtypes = [i]
    L.fgm_rowbatch_scratch_hip.argtypes = [i, i, i]
    L.fgm_rowbatch_scratch_hip.restype = i
    L.fgm_hip_attend_scratch_bytes.argtypes = [i, i, i, i, i]
    L.fgm_hip_attend_scratch_bytes.restype = _C.c_size_t
    L.fgm_hip_attend_dev.argtypes = [p, p, p, i, i, i, i, i, p, _C.c_size_t, p]
    L.fgm_hip_attend_heads_dev.argtypes = [p, p, p, p, p, p, i, i, i, i, i, i, i, i, i, p,
                                           _C.c_size_t, p]
    L.fgm_hip_store_v_t_dev.argtypes = [p, p, i, i, p]
    L.fgm_hip_kv_store_dev.argtypes = [p, p, i, i, p, p, p, p, i, i, i, p]
    L.fgm_hip_model_open.argtypes = [_C.c_char_p, i]
    L.fgm_hip_model_open.restype = p
    L.fgm_hip_model_close.argtypes = [p]
    L.fgm_hip_model_close.restype = None
    L.fgm_hip_model_has.argtypes = [p, _C.c_char_p]
    L.fgm_hip_model_config.argtypes = [p]
    L.fgm_hip_model_config.restype = _C.c_char_p
    L.fgm_hip_model_meta.argtypes = [p]
    L.fgm_hip_model_meta.restype = _C.c_char_p
    L.fgm_hip_model_total_bytes.argtypes = [p]
    L.fgm_hip_model_total_bytes.restype = _C.c_size_t
    L.fgm_hip_model_tensor_count.argtypes = [p]
    L.fgm_hip_model_tensor_name.argtypes = [p, i]
    L.fgm_hip_model_tensor_name.restype = _C.c_char_p
    L.fgm_hip_model_tensor.argtypes = [p, _C.c_char_p, p]
    L.fgm_hip_model_linear.argtypes = [p, _C.c_char_p, p]
    L.fgm_hip_weight_sel.argtypes = [_C.c_char_p, p]
    L.fgm_hip_model_dual.argtypes = [p, _C.c_char_p, i, i, i, p]
    L.fgm_hip_model_gather_dev.argtypes = [p, _C.c_char_p, p, i, p, p]
    L.fgm_hip_gather_dev.argtypes = [i, p, p, p, i, i, p, p]
    L.fgm_gather_q8r_hip.argtypes = [p, p, p, i, i]
    L.fgm_gather_q4r_hip.argtypes = [p, p, p, i, i]
    L.fgm_hip_pool_gemm_dev.argtypes = [p, p]
    L.fgm_hip_pool_prep_dev.argtypes = [p, p]
    L.fgm_hip_linear_scratch_bytes.argtypes = [i, i]
    L.fgm_hip_linear_scratch_bytes.restype = _C.c_size_t
    L.fgm_hip_linear_run_dev.argtypes = [p, p, i, i, p, p, _C.c_size_t, p]
    L.fgm_hip_linear_run_noalloc_dev.argtypes = [p, p, i, i, p, p]
    L.fgm_hip_linear_noalloc_max_bytes.argtypes = []
    L.fgm_hip_linear_noalloc_max_bytes.restype = _C.c_size_t
    for name in ("fgm_hip_model_has", "fgm_hip_model_tensor_count", "fgm_hip_model_tensor",
                 "fgm_hip_model_linear", "fgm_hip_weight_sel", "fgm_hip_model_dual",
                 "fgm_hip_model_gather_dev", "fgm_hip_gather_dev", "fgm_hip_pool_gemm_dev",
                 "fgm_hip_pool_prep_dev", "fgm_hip_linear_run_dev",
                 "fgm_hip_linear_run_noalloc_dev"):
        getattr(L, name).restype = i
    for name in ("fgm_hip_attend_dev", "fgm_hip_attend_heads_dev", "fgm_hip_store_v_t_dev",
                 "fgm_hip_kv_store_dev", "fgm_hip_gemm_batch_dev", "fgm_hip_prep_batch_dev",
                 "fgm_hip_prep_rmsnorm_dev", "fgm_hip_prep_gelu_mul_dev", "fgm_hip_gemm_q8c_dev",
                 "fgm_hip_gemm_q4g_dev", "fgm_hip_acc_q8c_dev",
                 "fgm_hip_acc_q4g_dev", "fgm_hip_prep_rows_dev", "fgm_hip_quant_act_dev",
                 "fgm_hip_pack_a_dev", "fgm_hip_fwht_dev", "fgm_hip_init", "fgm_hip_gemm_path", "fgm_hip_gemm_plan",
                 "fgm_hip_rmsnorm_dev", "fgm_hip_gelu_mul_dev", "fgm_hip_softcap_dev",
                 "fgm_hip_rope_dev", "fgm_hip_add_dev", "fgm_hip_mul_dev", "fgm_hip_scale_dev"):
        getattr(L, name).restype = i


def check(status: int) -> None:
    """Raise FgmHipError with the library's message for a non-zero status."""
    if status != 0:
        raise FgmHipError(f"status {status}: {lib().fgm_hip_last_error().decode()}")


class GemmDesc(_C.Structure):
    """fgm_hip_gemm_desc (include/fgm_hip.h)."""
    _fields_ = [("bits", _C.c_int), ("m", _C.c_int), ("n", _C.c_int), ("k", _C.c_int),
                ("group", _C.c_int), ("a", _C.c_void_p), ("a_scale", _C.c_void_p),
                ("b", _C.c_void_p), ("b_scale", _C.c_void_p), ("c", _C.c_void_p),
                ("ldc", _C.c_int), ("n0", _C.c_int), ("n1", _C.c_int)]


class PrepDesc(_C.Structure):
    """fgm_hip_prep_desc (include/fgm_hip.h)."""
    _fields_ = [("src", _C.c_void_p), ("lda", _C.c_int), ("rot", _C.c_void_p),
                ("qa", _C.c_void_p), ("qs", _C.c_void_p), ("pa", _C.c_void_p),
                ("m", _C.c_int), ("k", _C.c_int), ("hsz", _C.c_int), ("r0", _C.c_int),
                ("r1", _C.c_int)]


class TensorInfo(_C.Structure):
    """fgm_hip_tensor (include/fgm_hip.h)."""
    _fields_ = [("dtype", _C.c_char * 16), ("ndim", _C.c_int), ("shape", _C.c_int64 * 4),
                ("offset", _C.c_size_t), ("nbytes", _C.c_size_t), ("host", _C.c_void_p),
                ("dev", _C.c_void_p), ("hadamard", _C.c_int), ("group", _C.c_int)]


class LinearInfo(_C.Structure):
    """fgm_hip_linear (include/fgm_hip.h)."""
    _fields_ = [("bits", _C.c_int), ("n", _C.c_int), ("k", _C.c_int), ("group", _C.c_int),
                ("hadamard", _C.c_int), ("b", _C.c_void_p), ("b_scale", _C.c_void_p),
                ("b_host", _C.c_void_p), ("b_scale_host", _C.c_void_p)]


class GemmJob(_C.Structure):
    """fgm_hip_gemm_job (include/fgm_hip.h; pool.rs:19-34)."""
    _fields_ = [("m", _C.c_int), ("n", _C.c_int), ("kdim", _C.c_int), ("a", _C.c_void_p),
                ("a_scale", _C.c_void_p), ("bq", _C.c_void_p), ("b8", _C.c_void_p),
                ("s4", _C.c_void_p), ("s8", _C.c_void_p), ("bits", _C.c_int),
                ("group", _C.c_int), ("c", _C.c_void_p), ("ldc", _C.c_int)]


class PrepJob(_C.Structure):
    """fgm_hip_prep_job (include/fgm_hip.h; pool.rs:67-79)."""
    _fields_ = [("src", _C.c_void_p), ("lda", _C.c_int), ("rot", _C.c_void_p),
                ("qa", _C.c_void_p), ("qs", _C.c_void_p), ("pa", _C.c_void_p), ("m", _C.c_int),
                ("k", _C.c_int), ("hsz", _C.c_int)]


class AttnSeq(_C.Structure):
    """fgm_hip_attn_seq (include/fgm_hip.h)."""
    _fields_ = [("kc", _C.c_void_p), ("ks", _C.c_void_p), ("vc", _C.c_void_p),
                ("vs", _C.c_void_p), ("k_len", _C.c_int), ("ring", _C.c_int), ("pos", _C.c_int),
                ("rows", _C.c_int)]


from .kernels import (  # noqa: E402,F401
    Backend, backend, fwht, gemm_batch, gemm_q4g, gemm_q8c, pack_a, packed_a_len, prep_batch,
    prep_rows, quant_act)
