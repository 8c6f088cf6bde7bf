"""The device API under HIP graph capture: the calls a decode step issues
(the batched prep, the int4 pair GEMM on the skinny kernel, a dense M=256
GEMM, an empty contraction's zero fill, the allocation-free Gemm::run) are
captured once and replayed several times, with eager work between the
replays and new inputs written into the captured buffers; every replay must
equal, byte for byte, the same calls run eagerly on the same inputs.  (No
memset node is captured: an empty contraction writes its zeros with a fill
kernel.)"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import fastgemma_amd as F
import oracle
from fastgemma_amd import LinearInfo, check, lib
from tests import hip_util as H

pytestmark = pytest.mark.gpu


def _ptr(t):
    return t.data_ptr()


class Step:
    """Device buffers and the calls of one synthetic decode + prefill step."""

    def __init__(self, t):
        self.t = t
        dev = "cuda"
        # decode: M = 8, up (8192 x 2048) and down (2048 x 8192), int4 g64
        self.x2 = t.zeros((8, 2048), dtype=t.float32, device=dev)
        self.x8 = t.zeros((8, 8192), dtype=t.float32, device=dev)
        self.qs2, self.qs8 = t.zeros(8, device=dev), t.zeros(8, device=dev)
        self.pa2 = t.zeros(16 * 2048, dtype=t.int8, device=dev)
        self.pa8 = t.zeros(16 * 8192, dtype=t.int8, device=dev)
        self.wu = H.dev(oracle.gen_u8(1, 8192 * 1024))
        self.su = H.dev(oracle.gen_uniform(2, 32 * 8192, 5e-3, 5e-2).astype(np.float16).view(np.uint16))
        self.wd = H.dev(oracle.gen_u8(3, 2048 * 4096))
        self.sd = H.dev(oracle.gen_uniform(4, 128 * 2048, 5e-3, 5e-2).astype(np.float16).view(np.uint16))
        self.cu = t.zeros((8, 8192), device=dev)
        self.cd = t.zeros((8, 2048), device=dev)
        # prefill: M = 256, int8 1024 x 2048 on the dense kernel
        self.xp = t.zeros((256, 2048), dtype=t.float32, device=dev)
        self.qsp = t.zeros(256, device=dev)
        self.pap = t.zeros(256 * 2048, dtype=t.int8, device=dev)
        self.w8 = H.dev(oracle.gen_i8(5, 1024 * 2048, -127, 127))
        self.s8 = H.dev(oracle.gen_uniform(6, 1024, 1e-3, 1e-2))
        self.cp = t.zeros((256, 1024), device=dev)
        # an empty contraction (k = 0) into the middle columns of cz
        self.cz = t.zeros((4, 256), device=dev)
        # the allocation-free Gemm::run on the int8 weight, M = 3
        self.info = LinearInfo(8, 1024, 2048, 0, 0, self.w8.data_ptr(), self.s8.data_ptr(), None, None)
        self.xn = t.zeros((3, 2048), device=dev)
        self.cn = t.zeros((3, 1024), device=dev)

    def outputs(self):
        return [self.cu, self.cd, self.cp, self.cz, self.cn, self.qs2, self.qs8, self.pa2, self.pa8]

    def fill_inputs(self, seed):
        t = self.t
        self.x2.copy_(t.from_numpy(oracle.gen_normal(seed, 8 * 2048).reshape(8, 2048)))
        self.x8.copy_(t.from_numpy(oracle.gen_student_t(seed + 1, 8 * 8192, 3).reshape(8, 8192)))
        self.xp.copy_(t.from_numpy(oracle.gen_normal(seed + 2, 256 * 2048).reshape(256, 2048)))
        self.xn.copy_(t.from_numpy(oracle.gen_normal(seed + 3, 3 * 2048).reshape(3, 2048)))

    def run(self, stream):
        L = lib()
        st = stream
        pd = (F.PrepDesc * 2)()
        pd[0] = F.PrepDesc(_ptr(self.x2), 2048, None, None, _ptr(self.qs2), _ptr(self.pa2), 8, 2048, 0, 0, 8)
        pd[1] = F.PrepDesc(_ptr(self.x8), 8192, None, None, _ptr(self.qs8), _ptr(self.pa8), 8, 8192, 0, 0, 8)
        check(L.fgm_hip_prep_batch_dev(pd, 2, st))
        gd = (F.GemmDesc * 2)()
        gd[0] = F.GemmDesc(4, 8, 8192, 2048, 64, _ptr(self.pa2), _ptr(self.qs2), _ptr(self.wu), _ptr(self.su),
                           _ptr(self.cu), 8192, 0, 512)
        gd[1] = F.GemmDesc(4, 8, 2048, 8192, 64, _ptr(self.pa8), _ptr(self.qs8), _ptr(self.wd), _ptr(self.sd),
                           _ptr(self.cd), 2048, 0, 128)
        check(L.fgm_hip_gemm_batch_dev(gd, 2, st))
        check(L.fgm_hip_prep_rows_dev(_ptr(self.xp), 2048, None, None, _ptr(self.qsp), _ptr(self.pap), 256, 2048,
                                      0, 0, 256, st))
        check(L.fgm_hip_gemm_q8c_dev(256, 1024, 2048, _ptr(self.pap), _ptr(self.qsp), _ptr(self.w8),
                                     _ptr(self.s8), _ptr(self.cp), 1024, 0, 64, st))
        check(L.fgm_hip_gemm_q8c_dev(4, 256, 0, _ptr(self.pap), _ptr(self.qsp), _ptr(self.w8), _ptr(self.s8),
                                     _ptr(self.cz), 256, 4, 12, st))
        check(L.fgm_hip_linear_run_noalloc_dev(C.byref(self.info), _ptr(self.xn), 3, 2048, _ptr(self.cn), st))


def snapshot(step):
    return [H.host(o).copy() for o in step.outputs()]


def same(a, b):
    return all(np.array_equal(np.ascontiguousarray(x).view(np.uint8), np.ascontiguousarray(y).view(np.uint8))
               for x, y in zip(a, b))


def scramble(step):
    """Eager work between replays: every output overwritten."""
    for o in step.outputs():
        o.fill_(7 if o.dtype == step.t.int8 else 3.25)


def test_captured_step_replays_equal_eager_runs():
    t = H.torch()
    s = Step(t)
    side = t.cuda.Stream()
    s.fill_inputs(11)
    scramble(s)
    s.run(t.cuda.current_stream().cuda_stream)  # eager (also first-use set-up, outside capture)
    t.cuda.synchronize()
    want = {11: snapshot(s)}
    # the empty contraction wrote zeros into columns [64, 192) only
    assert np.all(want[11][3][:, 64:192] == 0) and np.all(want[11][3][:, :64] == 3.25)

    g = t.cuda.CUDAGraph()
    side.wait_stream(t.cuda.current_stream())
    with t.cuda.stream(side):
        scramble(s)
        t.cuda.synchronize()
        with t.cuda.graph(g, stream=side):
            s.run(side.cuda_stream)
    t.cuda.synchronize()

    for seed in (11, 23, 11, 37):
        s.fill_inputs(seed)
        scramble(s)
        t.cuda.synchronize()
        g.replay()
        t.cuda.synchronize()
        got = snapshot(s)
        if seed not in want:
            # the eager result for these inputs, computed after the replay
            scramble(s)
            s.run(t.cuda.current_stream().cuda_stream)
            t.cuda.synchronize()
            want[seed] = snapshot(s)
        assert same(got, want[seed]), f"replay with inputs {seed} differs from the eager run"
        # eager work between replays
        junk = t.randn(1 << 20, device="cuda")
        (junk * 2).sum().item()
