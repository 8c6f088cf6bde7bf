"""CPU checks of the C-ABI library: it loads, exports every symbol that
include/fgm_hip.h declares, refuses bad shapes before touching a device, and
reports the absence of a GPU instead of falling back to anything."""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np
import pytest

import fastgemma_amd as F
from fastgemma_amd import kernels as K

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fgm_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fgm_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = F.lib()
    names = declared_symbols()
    assert len(names) >= 18
    for name in names:
        assert hasattr(L, name), name


def test_dropin_symbols_mirror_reference_names():
    """Every GEMM-path symbol the reference's Rust crate binds (lib.rs:19-53)
    has a _hip twin."""
    ref = ["fgm_pack_a", "fgm_prep_rows", "fgm_gemm_q4g", "fgm_gemm_q8c", "fgm_fwht",
           "fgm_quant_act"]
    names = declared_symbols()
    for r in ref:
        assert r + "_hip" in names


BAD_Q8C = [
    dict(m=8, n=256, k=100, ldc=256, n0=0, n1=16),   # k % 64
    dict(m=8, n=250, k=128, ldc=256, n0=0, n1=15),   # n % 16
    dict(m=8, n=256, k=128, ldc=256, n0=0, n1=6),    # (n1 - n0) % 4
    dict(m=8, n=256, k=128, ldc=256, n0=4, n1=20),   # n1 > n / 16
    dict(m=8, n=256, k=128, ldc=100, n0=0, n1=16),   # ldc < 16 n1
    dict(m=-1, n=256, k=128, ldc=256, n0=0, n1=16),  # negative
]


@pytest.mark.parametrize("args", BAD_Q8C)
def test_bad_shapes_are_refused_with_einval(args):
    L = F.lib()
    rc = L.fgm_hip_gemm_q8c_dev(args["m"], args["n"], args["k"], None, None, None, None, None,
                                args["ldc"], args["n0"], args["n1"], None)
    assert rc == 1, L.fgm_hip_last_error()
    assert L.fgm_hip_last_error()


def test_operand_ranges_past_2g_are_refused():
    """The kernels' buffer descriptors carry 32-bit byte ranges and mask lanes
    with the offset 2^31: packed A or an int4 scale table of 2^31 bytes or
    more is refused on the host (B itself is cut into launches along N)."""
    L = F.lib()
    # packed A: 16 * ceil(m / 16) * k >= 2^31
    rc = L.fgm_hip_gemm_q8c_dev(4096, 256, 524288, None, None, None, None, None, 256, 0, 16, None)
    assert rc == 1 and b"packed A" in L.fgm_hip_last_error()
    # int4 scales: (k / group) * n * 2 >= 2^31
    rc = L.fgm_hip_gemm_q4g_dev(8, 1 << 24, 8192, None, None, None, None, 64, None, 1 << 24, 0, 16, None)
    assert rc == 1 and b"scale table" in L.fgm_hip_last_error()
    # just below the limits the shape checks pass (ENODEV without a GPU)
    rc = L.fgm_hip_gemm_q8c_dev(4096, 256, 524224, None, None, None, None, None, 256, 0, 16, None)
    assert rc in (0, 3) or b"packed A" not in L.fgm_hip_last_error()


@pytest.mark.parametrize("group", [0, 32, 96, 192])
def test_bad_group_is_refused(group):
    L = F.lib()
    rc = L.fgm_hip_gemm_q4g_dev(8, 256, 1024, None, None, None, None, group, None, 256, 0, 16,
                                None)
    assert rc == 1 and b"group" in L.fgm_hip_last_error()


def test_other_preconditions():
    L = F.lib()
    assert L.fgm_hip_prep_rows_dev(None, 64, None, None, None, None, 32, 64, 0, 8, 16, None) == 1
    assert L.fgm_hip_prep_rows_dev(None, 64, None, None, None, None, 32, 100, 0, 0, 16, None) == 1
    assert L.fgm_hip_prep_rows_dev(None, 128, None, None, None, None, 32, 128, 48, 0, 16, None) == 1
    assert L.fgm_hip_fwht_dev(None, 96, 12, None) == 1
    assert L.fgm_hip_fwht_dev(None, 96, 64, None) == 1
    assert L.fgm_hip_pack_a_dev(4, 100, None, None, None) == 1
    # fused producers: prep_rows' shape rules, and gelu_mul needs up
    fake = C.c_void_p(4096)
    assert L.fgm_hip_prep_rmsnorm_dev(fake, 100, None, 1e-6, None, None, None, fake, fake, 4, 100,
                                      0, None) == 1
    assert L.fgm_hip_prep_rmsnorm_dev(fake, 64, None, 1e-6, None, None, None, fake, fake, -1, 64,
                                      0, None) == 1
    assert L.fgm_hip_prep_gelu_mul_dev(fake, None, 128, None, None, None, fake, fake, 4, 128, 0,
                                       None) == 1
    assert b"up is NULL" in L.fgm_hip_last_error()


def test_no_gpu_means_no_backend():
    """On a host without a gfx950 device the library says so; nothing runs on
    the CPU in its place."""
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:
        has_gpu = False
    if has_gpu:
        pytest.skip("a GPU is present")
    L = F.lib()
    assert L.fgm_hip_available() == 0
    rc = L.fgm_hip_gemm_q8c_dev(8, 256, 128, None, None, None, None, None, 256, 0, 16, None)
    assert rc == 3  # FGM_HIP_ENODEV, after the shape checks passed
    with pytest.raises(F.HipUnavailable):
        K.backend()


def test_skinny_dense_dispatch_thresholds():
    """The switch points measured on MI355X (bench.py --only sweep): the
    skinny kernel up to 32 rows for int8, 48 for int4 group 64, 16 for wider
    int4 groups; the dense kernel beyond."""
    assert K.gemm_path(8, 1, 2048) == "skinny"
    assert K.gemm_path(4, 8, 8192, 64) == "skinny"
    assert K.gemm_path(8, 32, 2048) == "skinny"
    assert K.gemm_path(8, 33, 2048) == "dense"
    assert K.gemm_path(4, 48, 2048, 64) == "skinny"
    assert K.gemm_path(4, 49, 2048, 64) == "dense"
    assert K.gemm_path(4, 16, 2048, 128) == "skinny"
    assert K.gemm_path(4, 17, 2048, 256) == "dense"
    assert K.gemm_path(8, 65, 2048) == "dense"
    assert K.gemm_path(4, 256, 2048, 64) == "dense"
    # the int4 skinny kernel keeps every group's sums in LDS; past 160 KB it goes dense
    assert K.gemm_path(4, 64, 65536, 64) == "dense"


def test_gemm_plan_cuts_weights_past_1gib():
    """The GEMM dispatch's cuts along N, checked on the host alone (a dry run:
    no device, no operand read): weights up to 1 GiB go in one launch, larger
    ones in launches of at most 1 GiB, and an int8 n-block that alone passes
    1 GiB (K > 2^26) is launched whole -- the case that once recursed without
    end on the host.  The int4 cut covers the scale table's rebased columns
    (the GPU side of both cuts: test_edge_gpu.py)."""
    assert K.gemm_plan(4, 8, 8192, 2048) == 1                     # cfg2 up
    assert K.gemm_plan(8, 8, 262144, 2048) == 1                   # LM head, 512 MiB
    assert K.gemm_plan(8, 8, 524288, 2048) == 1                   # exactly 1 GiB
    assert K.gemm_plan(8, 8, 524288 + 64, 2048) == 2              # 1 GiB + 4 n-blocks
    assert K.gemm_plan(4, 8, 163840, 16384, 64) == 2              # int4 1.25 GiB, skinny
    assert K.gemm_plan(4, 128, 163840, 16384, 64) == 2            # the same, dense
    kl = (1 << 26) + 64                                           # one n-block: 1 GiB + 1 KiB
    assert K.gemm_plan(8, 8, 64, kl) == 4
    assert K.gemm_plan(8, 8, 128, kl, 64, 4, 8) == 4              # a range not at n-block 0
    assert K.gemm_plan(8, 16, 64, kl) == 4                        # 16 rows: packed A 1 GiB
    assert K.gemm_plan(8, 0, 8192, 2048) == 0                     # nothing to do
    assert K.gemm_plan(8, 8, 8192, 0) == 1                        # k = 0: one zero fill
    with pytest.raises(F.FgmHipError):
        K.gemm_plan(8, 8, 64, 1 << 27)                            # packed A reaches 2^31
    with pytest.raises(F.FgmHipError):
        K.gemm_plan(4, 8, 8192, 2048, 96)                         # bad group
