"""The library's .fgm reader on a file written by the reference's own writer
(convert/fgm.py FgmWriter, via tests/golden/make_fgm_fixture.py): the header
the reference writes (arch, config, meta, tensors with offsets and sizes), the
payload bytes, and model.rs's typed views (Model::linear, DualW::pick) --
CPU only; the GPU side is in tests/test_model_gpu.py."""
from __future__ import annotations

import ctypes as C
import hashlib
import json
import os

import numpy as np

from fastgemma_amd.model import Model, Selection, WeightSel

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
PATH = os.path.join(GOLD, "ref_writer.fgm")
EXPECT = json.load(open(os.path.join(GOLD, "ref_writer.json")))


def test_reader_returns_the_reference_writers_layout():
    with Model(PATH) as m:
        assert m.cfg == EXPECT["config"]
        assert m.meta == EXPECT["meta"]
        assert sorted(m.names()) == sorted(t["name"] for t in EXPECT["tensors"])
        for t in EXPECT["tensors"]:
            info = m.tensor(t["name"])
            assert info.dtype.decode() == t["dtype"]
            assert list(info.shape[: info.ndim]) == t["shape"]
            assert (info.offset, info.nbytes) == (t["offset"], t["nbytes"])
            assert info.offset % 64 == 0
            assert info.hadamard == t["meta"].get("hadamard", 0)
            assert info.group == t["meta"].get("group", -1)
            body = C.string_at(info.host, info.nbytes)
            assert hashlib.sha256(body).hexdigest() == t["sha256"], t["name"]


def test_linear_and_dual_on_the_reference_writers_file():
    with Model(PATH) as m:
        w = m.linear("layers.0.mlp.up")
        assert (w.bits, w.n, w.k, w.group, w.hadamard) == (4, 64, 256, 64, 128)
        w8 = m.linear("layers.0.mlp.up.i8")
        assert (w8.bits, w8.n, w8.k, w8.group, w8.hadamard) == (8, 64, 256, 0, 128)
        d = m.dual("layers.0.mlp.up")
        assert d.has_hi()
        assert d.pick(8, Selection(WeightSel.Above, 16)).bits == 4
        assert d.pick(16, Selection(WeightSel.Above, 16)).bits == 8
        assert d.pick(1, Selection(WeightSel.Hi, 16)).bits == 8
        assert d.pick(500, Selection(WeightSel.Lo, 16)).bits == 4
        scales = np.asarray(w.scales()).view(np.float16).astype(np.float32)
        assert scales.shape == (4 * 64,) and np.all(scales > 0)
