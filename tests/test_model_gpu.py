"""The .fgm model resident in HBM (fgm_model.hip): Gemm::run through the
file's own weights (forward.rs:140-158), the int8-twin selection on the
device, the gathers (model.rs:203-213; ops.c:208-251) and the pool jobs
(pool.rs:19-79), against the oracle -- bit-exact."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import fastgemma_amd as F
import oracle
from fastgemma_amd.model import Model, Selection, WeightSel, linear_run
from tests import fgm_file
from tests import hip_util as H

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    p = tmp_path_factory.mktemp("fgm") / "tiny.fgm"
    arrays = fgm_file.synthetic_model(str(p))
    m = Model(str(p), resident=True)
    yield m, arrays
    m.close()


def oracle_linear(w, a: np.ndarray, m: int, lda: int) -> np.ndarray:
    """forward.rs:140-158 on the CPU oracle: prep_rows (FWHT of w.hadamard,
    quantise, pack) then the GEMM on the file's bytes."""
    k = w.k
    rot = np.zeros(m * k, np.float32)
    qa = np.zeros(m * k, np.int8)
    qs = np.zeros(m, np.float32)
    pa = np.zeros(oracle.packed_a_len(m, k), np.int8)
    oracle.prep_rows(np.ascontiguousarray(a, np.float32), lda, rot, qa, qs, pa, m, k, w.hadamard, 0, m)
    c = np.zeros(m * w.n, np.float32)
    if w.bits == 4:
        oracle.gemm_q4g(m, w.n, k, pa, qs, np.ascontiguousarray(w.blob()), np.ascontiguousarray(w.scales()),
                        w.group, c, w.n, 0, w.n // 16)
    else:
        oracle.gemm_q8c(m, w.n, k, pa, qs, np.ascontiguousarray(w.blob()), np.ascontiguousarray(w.scales()),
                        c, w.n, 0, w.n // 16)
    return c.reshape(m, w.n)


@pytest.mark.parametrize("name", ["layers.0.mlp.gate", "layers.0.mlp.gate.i8", "layers.0.mlp.down",
                                  "layers.0.attn.q"])
@pytest.mark.parametrize("m", [1, 8, 40])
def test_linear_run_resident(model, name, m):
    mdl, _ = model
    w = mdl.linear(name)
    assert w.info.b and w.info.b_scale
    lda = w.k + 3
    a = oracle.gen_student_t(7 + m, m * lda, 3).reshape(m, lda)
    t = H.torch()
    out = t.zeros((m, w.n), dtype=t.float32, device="cuda")
    linear_run(w, H.dev(a), m, lda, out)
    want = oracle_linear(w, a.ravel(), m, lda)
    assert np.array_equal(H.host(out).view(np.uint32), want.view(np.uint32))


def test_dual_pick_runs_the_chosen_weight(model):
    mdl, _ = model
    d = mdl.dual("layers.0.mlp.gate")
    t = H.torch()
    for rows, bits in ((8, 4), (16, 8)):
        w = d.pick(rows, Selection(WeightSel.Above, 16))
        assert w.bits == bits
        a = oracle.gen_normal(77 + rows, rows * w.k).reshape(rows, w.k)
        out = t.zeros((rows, w.n), dtype=t.float32, device="cuda")
        linear_run(w, H.dev(a), rows, w.k, out)
        want = oracle_linear(w, a.ravel(), rows, w.k)
        assert np.array_equal(H.host(out).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name,bits", [("embed", 8), ("ple", 4)])
def test_gathers(model, name, bits):
    mdl, arrays = model
    t = H.torch()
    k = mdl.shape(name)[1]
    rows = [0, 5, mdl.shape(name)[0] - 1, 5]
    tbl, sc = arrays[name], arrays[name + ".scale"].ravel()
    want = np.stack([oracle.gather(bits, tbl, sc, r, k) for r in rows])
    out = t.zeros((len(rows), k), dtype=t.float32, device="cuda")
    mrows = t.tensor(rows, dtype=t.int32, device="cuda")
    mdl.gather(name, mrows, out)
    assert np.array_equal(H.host(out).view(np.uint32), want.view(np.uint32))
    # device API on caller tables
    out2 = t.zeros_like(out)
    dtbl, dsc = H.dev(tbl), H.dev(sc)              # referenced until the call has run
    drows = t.tensor(rows, dtype=t.int32, device="cuda")
    F.check(F.lib().fgm_hip_gather_dev(bits, dtbl.data_ptr(), dsc.data_ptr(), drows.data_ptr(),
                                       len(rows), k, out2.data_ptr(), t.cuda.current_stream().cuda_stream))
    assert np.array_equal(H.host(out2).view(np.uint32), want.view(np.uint32))
    # host-pointer drop-in, the reference's signature (lib.rs:54-55)
    for r in rows:
        o = np.empty(k, np.float32)
        f = F.lib().fgm_gather_q8r_hip if bits == 8 else F.lib().fgm_gather_q4r_hip
        f(o.ctypes.data, np.ascontiguousarray(tbl).ctypes.data, np.ascontiguousarray(sc).ctypes.data, r, k)
        assert np.array_equal(o.view(np.uint32), oracle.gather(bits, tbl, sc, r, k).view(np.uint32))


def test_pool_jobs_equal_linear_run(model):
    """Pool::prep + Pool::gemm jobs (pool.rs:19-79) on the device give the
    same bytes as Gemm::run."""
    mdl, _ = model
    w = mdl.linear("layers.0.mlp.gate")
    m = 24
    t = H.torch()
    a = H.dev(oracle.gen_normal(5, m * w.k).reshape(m, w.k))
    qs = t.zeros(m, dtype=t.float32, device="cuda")
    pa = t.zeros(oracle.packed_a_len(m, w.k), dtype=t.int8, device="cuda")
    rot = t.zeros(m * w.k, dtype=t.float32, device="cuda")
    qa = t.zeros(m * w.k, dtype=t.int8, device="cuda")
    F.check(F.lib().fgm_hip_pool_prep_dev(C.byref(F.PrepJob(a.data_ptr(), w.k, rot.data_ptr(), qa.data_ptr(),
                                                             qs.data_ptr(), pa.data_ptr(), m, w.k, w.hadamard)),
                                          t.cuda.current_stream().cuda_stream))
    c = t.zeros((m, w.n), dtype=t.float32, device="cuda")
    job = F.GemmJob(m, w.n, w.k, pa.data_ptr(), qs.data_ptr(), w.info.b, None, w.info.b_scale, None, 4,
                    w.group, c.data_ptr(), w.n)
    F.check(F.lib().fgm_hip_pool_gemm_dev(C.byref(job), t.cuda.current_stream().cuda_stream))
    out = t.zeros((m, w.n), dtype=t.float32, device="cuda")
    linear_run(w, a, m, w.k, out)
    assert np.array_equal(H.host(c).view(np.uint32), H.host(out).view(np.uint32))


def test_reference_written_file_on_the_gpu():
    """The file written by the reference's own FgmWriter (tests/golden/
    ref_writer.fgm), resident: Gemm::run through both weights of the dual and
    both gathers equal the oracle on the file's bytes."""
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_writer.fgm")
    t = H.torch()
    with Model(path, resident=True) as m:
        for name in ("layers.0.mlp.up", "layers.0.mlp.up.i8"):
            w = m.linear(name)
            for rows in (3, 20):
                a = oracle.gen_student_t(31 + rows, rows * w.k, 3).reshape(rows, w.k)
                out = t.zeros((rows, w.n), dtype=t.float32, device="cuda")
                linear_run(w, H.dev(a), rows, w.k, out)
                want = oracle_linear(w, a.ravel(), rows, w.k)
                assert np.array_equal(H.host(out).view(np.uint32), want.view(np.uint32)), (name, rows)
        for name, bits in (("embed", 8), ("ple", 4)):
            shape = m.shape(name)
            k = shape[1]
            tbl = m.i8s(name) if bits == 8 else m.u8s(name)
            sc = m.f32s(name + ".scale") if bits == 8 else m.f16s(name + ".scale").view(np.uint16)
            rows = [0, shape[0] - 1, 1]
            want = np.stack([oracle.gather(bits, np.ascontiguousarray(tbl), np.ascontiguousarray(sc).ravel(), r, k)
                             for r in rows])
            out = t.zeros((len(rows), k), dtype=t.float32, device="cuda")
            m.gather(name, t.tensor(rows, dtype=t.int32, device="cuda"), out)
            assert np.array_equal(H.host(out).view(np.uint32), want.view(np.uint32)), name
