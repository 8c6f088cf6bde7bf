"""The skinny kernel's group chains read LDS through inline asm (the reads are
issued ahead and waited for with s_waitcnt lgkmcnt), so the compiler believes
their destination registers hold the data as soon as the asm statement ends.
If it copies or reuses such a register before the wait -- which it may do
where the register reaches a branch's join or a loop's back edge -- the copy
reads stale bits or the late data overwrites a new value: a wrong result that
depends on timing.  This test compiles fgm_decode.hip to gfx950 assembly with
the library's flags and checks, kernel by kernel, that no instruction touches
a register of an inline-asm LDS read before an lgkmcnt wait has retired that
read.  It also checks that no inline asm loads registers from global memory
(those loads must stay visible to the compiler, whose own waits cover them).

The scan is linear in layout order (the pending reads carry across labels),
with LDS operations retiring in issue order, as lgkmcnt counts them."""
from __future__ import annotations

import os
import re
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "fastgemma_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"


def _regs(tok: str) -> set[int]:
    tok = tok.strip().split()[0] if tok.strip() else ""
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", tok)
    return {int(m.group(1))} if m else set()


def scan_kernel(lines: list[str]) -> list[str]:
    """Problems in one kernel's assembly (empty when clean)."""
    bad = []
    pending: list[set[int]] = []      # LDS operations in flight, oldest first
    in_asm = False
    for ln in lines:
        if ";;#ASMSTART" in ln:
            in_asm = True
            continue
        if ";;#ASMEND" in ln:
            in_asm = False
            continue
        t = ln.split(";")[0].strip()
        if not t or t.startswith("."):
            continue
        op = t.split()[0]
        args = t[len(op):].split(",")
        if op == "s_waitcnt":
            m = re.search(r"lgkmcnt\((\d+)\)", t)
            if m:
                n = int(m.group(1))
                pending = pending[-n:] if n else []
            continue
        if op.startswith("s_"):
            continue
        live = set().union(*pending) if pending else set()
        touched = set().union(*(_regs(a) for a in args))
        if touched & live:
            bad.append(f"{t}  (registers {sorted(touched & live)} of an LDS read still in flight)")
        if in_asm and (op.startswith("buffer_load") or op.startswith("global_load")) and " lds" not in t:
            bad.append(f"{t}  (a register load from global memory in inline asm)")
        if op.startswith("ds_"):
            # only the inline-asm reads are invisible to the compiler; its own
            # LDS operations still count in the in-order retirement
            pending.append(_regs(args[0]) if (in_asm and op.startswith("ds_read")) else set())
    return bad


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="no hipcc")
def test_no_register_of_an_asm_lds_read_is_touched_before_its_wait(tmp_path):
    out = tmp_path / "decode.s"
    flags = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Xclang",
             "-target-feature", "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form",
             "--cuda-device-only", "-S", "-o", str(out), "fgm_decode.hip"]
    r = subprocess.run([HIPCC] + flags, cwd=CSRC, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    text = out.read_text()
    parts = re.split(r"\n(_ZN\w*decode_(?:pir2_)?kernel\w+):", text)
    assert len(parts) > 10, "no decode kernels found in the assembly"
    problems = {}
    for i in range(1, len(parts), 2):
        body = parts[i + 1].split(".Lfunc_end")[0].split("\n")
        bad = scan_kernel(body)
        if bad:
            problems[parts[i]] = bad[:5]
    assert not problems, problems


def test_scanner_flags_a_copy_before_the_wait():
    """The scanner itself: a copy of a pending asm read's register is caught,
    the same copy after the wait is not."""
    racy = ["\t;;#ASMSTART", "\tds_read_b128 v[10:13], v2", "\t;;#ASMEND",
            "\tv_mov_b32_e32 v20, v11", "\t;;#ASMSTART", "\ts_waitcnt lgkmcnt(0)", "\t;;#ASMEND"]
    clean = ["\t;;#ASMSTART", "\tds_read_b128 v[10:13], v2", "\t;;#ASMEND",
             "\t;;#ASMSTART", "\ts_waitcnt lgkmcnt(0)", "\t;;#ASMEND", "\tv_mov_b32_e32 v20, v11"]
    newer = ["\t;;#ASMSTART", "\tds_read_b128 v[10:13], v2", "\tds_read_b128 v[14:17], v2 offset:16",
             "\t;;#ASMEND", "\t;;#ASMSTART", "\ts_waitcnt lgkmcnt(1)", "\t;;#ASMEND",
             "\tv_mov_b32_e32 v20, v11", "\tv_mov_b32_e32 v21, v15"]
    asm_load = ["\t;;#ASMSTART", "\tbuffer_load_dwordx4 v[2:5], v1, s[4:7], 0 offen", "\t;;#ASMEND"]
    assert scan_kernel(racy)
    assert not scan_kernel(clean)
    bad = scan_kernel(newer)
    assert len(bad) == 1 and "[15]" in bad[0]
    assert scan_kernel(asm_load)
