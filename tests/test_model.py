"""The .fgm reader (fgm_model.hip; model.rs:1-220, forward.rs:26-89) on the CPU:
header parsing, typed tensor views, Model::linear, the int8-twin selection and
FGM_WEIGHTS parsing, error paths.  The file is written by tests/fgm_file.py in
the layout convert/fgm.py documents; no GPU is touched (resident=False)."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from fastgemma_amd import FgmHipError
from fastgemma_amd.model import Model, Selection, WeightSel
from tests import fgm_file


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    p = tmp_path_factory.mktemp("fgm") / "tiny.fgm"
    arrays = fgm_file.synthetic_model(str(p))
    return str(p), arrays


def test_header_and_tensor_table(model_file):
    path, arrays = model_file
    with Model(path) as m:
        assert m.cfg == fgm_file.CONFIG
        assert m.meta == {"source": "synthetic"}
        assert sorted(m.names()) == sorted(arrays)
        assert m.has("embed") and not m.has("embed2")
        assert m.shape("layers.0.mlp.gate.scale") == [8, 256]
        assert m.total_bytes() == sum(np.asarray(a).nbytes for a in arrays.values())
        for name, a in arrays.items():
            raw = m.u8s(name)
            assert raw.tobytes() == np.ascontiguousarray(a).tobytes(), name
            assert m.tensor(name).offset % 64 == 0
        assert np.array_equal(m.f32s("layers.0.input_ln"), arrays["layers.0.input_ln"])
        assert m.tensor("embed").dev is None          # not resident


def test_linear_geometry_and_views(model_file):
    """model.rs:167-192: bits, n, k; group from meta (default 64, 0 for q8c);
    hadamard from meta (default 0); blobs and scales are the file's bytes."""
    path, arrays = model_file
    with Model(path) as m:
        g = m.linear("layers.0.mlp.gate")
        assert (g.bits, g.n, g.k, g.group, g.hadamard) == (4, 256, 512, 64, 128)
        assert np.array_equal(g.blob(), arrays["layers.0.mlp.gate"])
        assert np.array_equal(g.scales(), arrays["layers.0.mlp.gate.scale"].ravel())
        d = m.linear("layers.0.mlp.down")
        assert (d.bits, d.group, d.hadamard) == (4, 128, 0)
        q = m.linear("layers.0.attn.q")
        assert (q.bits, q.n, q.k, q.group, q.hadamard) == (8, 128, 256, 0, 128)
        assert np.array_equal(q.scales(), arrays["layers.0.attn.q.scale"])
        with pytest.raises(FgmHipError, match="non-linear dtype"):
            m.linear("embed")
        with pytest.raises(FgmHipError, match="missing tensor"):
            m.linear("nope")


@pytest.mark.parametrize("value,want", [
    (None, (WeightSel.Above, 16)), ("", (WeightSel.Above, 16)), ("int4", (WeightSel.Lo, 16)),
    ("int8", (WeightSel.Hi, 16)), ("INT8", (WeightSel.Above, 16)), ("auto", (WeightSel.Above, 16)),
    ("auto:", (WeightSel.Above, 16)), ("auto:32", (WeightSel.Above, 32)), ("auto:+7", (WeightSel.Above, 7)),
    ("auto:0", (WeightSel.Above, 0)), ("auto:abc", (WeightSel.Above, 16)), ("auto:-1", (WeightSel.Above, 16)),
    ("auto:18446744073709551615", (WeightSel.Above, 2**31 - 1)),
    ("auto:18446744073709551616", (WeightSel.Above, 16)),
])
def test_weight_selection_parse(value, want):
    """FGM_WEIGHTS=int4|int8|auto[:M] (forward.rs:58-69; Rust's usize parse)."""
    s = Selection.parse(value)
    assert (s.sel, s.threshold) == want


def test_dual_pick(model_file):
    """DualW::pick (forward.rs:74-81): the twin for Hi, or Above(t) with
    rows >= t; the primary otherwise and whenever there is no twin."""
    path, _ = model_file
    with Model(path) as m:
        gate, down = m.dual("layers.0.mlp.gate"), m.dual("layers.0.mlp.down")
        assert gate.has_hi() and not down.has_hi()
        cases = [(Selection(WeightSel.Lo), 1, 4), (Selection(WeightSel.Lo), 512, 4),
                 (Selection(WeightSel.Hi), 1, 8), (Selection(WeightSel.Above, 16), 15, 4),
                 (Selection(WeightSel.Above, 16), 16, 8), (Selection(WeightSel.Above, 0), 0, 8)]
        for sel, rows, bits in cases:
            w = gate.pick(rows, sel)
            assert w.bits == bits
            assert w.name == ("layers.0.mlp.gate.i8" if bits == 8 else "layers.0.mlp.gate")
            assert down.pick(rows, sel).bits == 4


def test_bad_files(tmp_path):
    p = tmp_path / "bad.fgm"
    p.write_bytes(b"NOTAFGM!" + struct.pack("<I", 2) + b"{}")
    with pytest.raises(FgmHipError, match="magic"):
        Model(str(p))
    p.write_bytes(b"FASTGEM1" + struct.pack("<I", 1000) + b"{}")
    with pytest.raises(FgmHipError, match="past the end"):
        Model(str(p))
    hdr = b'{"config":{},"tensors":{"x":{"dtype":"f32","shape":[4],"offset":64,'
    p.write_bytes(b"FASTGEM1" + struct.pack("<I", len(hdr)) + hdr)
    with pytest.raises(FgmHipError, match="not valid JSON"):
        Model(str(p))
    hdr = b'{"config":{},"tensors":{"x":{"dtype":"f32","shape":[4],"offset":4096,"nbytes":16}}}'
    p.write_bytes(b"FASTGEM1" + struct.pack("<I", len(hdr)) + hdr)
    with pytest.raises(FgmHipError, match="past the end of the file"):
        Model(str(p))
    with pytest.raises(FgmHipError, match="cannot open"):
        Model(str(tmp_path / "missing.fgm"))


def _linear_file(path, n, k, wbytes, sbytes, dtype="q4g", group=64):
    out = [("w", np.zeros(wbytes, np.uint8), dtype, (n, k), {"group": group} if dtype == "q4g" else {}),
           ("w.scale", np.zeros(sbytes, np.uint8), "f16" if dtype == "q4g" else "f32",
            ((k // max(group, 1)), n) if dtype == "q4g" else (n,), None)]
    fgm_file.write_fgm(str(path), {}, out)


@pytest.mark.parametrize("n,k,wb,sb,dtype,group,msg", [
    (256, 512, 256 * 512 // 2 - 1, (512 // 64) * 256 * 2, "q4g", 64, "its shape needs"),   # short blob
    (256, 512, 256 * 512 // 2, (512 // 64) * 256 * 2 - 2, "q4g", 64, "needs"),             # short scales
    (256, 512, 256 * 512, 256 * 4 - 4, "q8c", 0, "needs"),                                  # short f32 scales
    (250, 512, 250 * 512, 250 * 4, "q8c", 0, "n % 16"),                                     # n not tiled
    (256, 500, 256 * 500, 256 * 4, "q8c", 0, "k % 64"),                                     # k not tiled
    (256, 512, 256 * 512 // 2, 4096, "q4g", 96, "group"),                                   # bad group
    (0, 512, 64, 64, "q8c", 0, "shape"),                                                    # empty
])
def test_linear_refuses_malformed_tensors(tmp_path, n, k, wb, sb, dtype, group, msg):
    """Model::linear on a tensor whose bytes or shape the GEMM cannot read
    safely: refused with EINVAL on the host instead of a device read past the
    tensor's end."""
    p = tmp_path / "lin.fgm"
    _linear_file(p, n, k, wb, sb, dtype, group)
    with Model(str(p)) as m:
        with pytest.raises(FgmHipError, match=msg):
            m.linear("w")


def test_linear_accepts_exact_sizes(tmp_path):
    p = tmp_path / "ok.fgm"
    _linear_file(p, 256, 512, 256 * 512 // 2, (512 // 64) * 256 * 2)
    with Model(str(p)) as m:
        w = m.linear("w")
        assert (w.bits, w.n, w.k, w.group) == (4, 256, 512, 64)
