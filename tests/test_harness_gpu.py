"""The drop-in C ABI driven from C the way fgm-core drives the reference
kernels (tests/harness/gemm_run.c): Gemm::run with the prep split over 16-row
tile blocks and the GEMM over n-block ranges on concurrent host threads
(pool.rs:110-145, 206-225), every output byte checked against the oracle.
The harness is a separate process with no Python or torch, so the library
runs on the system HIP runtime, as a Rust caller's would."""
from __future__ import annotations

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

HARNESS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "harness", "gemm_run")


@pytest.mark.parametrize("threads", [8, 16])
def test_c_harness_threads_match_oracle(threads):
    assert os.path.exists(HARNESS), "build it first: make -C tests/harness (or __graft_entry__.build())"
    r = subprocess.run([HARNESS, str(threads)], capture_output=True, text=True, timeout=240)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("all ok")
    assert "MISMATCH" not in r.stdout
