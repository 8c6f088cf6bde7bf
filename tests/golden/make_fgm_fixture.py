"""Writes tests/golden/ref_writer.fgm: a small .fgm container written by the
reference's own writer (convert/fgm.py, FgmWriter), so that the library's C++
reader is checked against the reference's bytes, not only against this
repository's restatement of the format (fastgemma_amd/fgm_format.py).

The reference's fgm.py has no tests or stored files of its own, so nothing
else pins the container; the tensor payloads are this repository's oracle
packers (pinned in tests/test_oracle.py) and seeded generators.  Run in the
build container only (it imports the reference from /root/reference):

    python tests/golden/make_fgm_fixture.py

The expected tensors (name, dtype, shape, meta, a sha256 of each payload) go
to tests/golden/ref_writer.json beside the file.
"""
from __future__ import annotations

import hashlib
import importlib.util
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

REF_FGM = "/root/reference/convert/fgm.py"


def load_writer():
    spec = importlib.util.spec_from_file_location("ref_fgm", REF_FGM)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def payloads():
    """(name, array, dtype, shape, meta): a q4g linear with its f16 scales and
    int8 twin, an int8 per-row gather table, an int4 one, a norm weight."""
    n, k, g = 64, 256, 64
    q = oracle.gen_i8(901, n * k, -8, 7).reshape(n, k)
    q4 = oracle.pack_nibbles(oracle.pack_b_tiles(q))
    s4 = oracle.gen_uniform(902, (k // g) * n, 5e-3, 5e-2).astype(np.float16)
    q8 = oracle.pack_b_tiles(oracle.gen_i8(903, n * k, -127, 127).reshape(n, k))
    s8 = oracle.gen_uniform(904, n, 1e-3, 1e-2)
    tbl8 = oracle.gen_i8(905, 10 * 128, -127, 127)
    tsc8 = oracle.gen_uniform(906, 10, 1e-3, 1e-2)
    tbl4 = oracle.gen_u8(907, 6 * 128 // 2)
    tsc4 = oracle.gen_uniform(908, 6 * 2, 1e-3, 1e-2).astype(np.float16)
    norm = oracle.gen_uniform(909, 256, 0.5, 1.5)
    return [
        ("layers.0.mlp.up", q4, "q4g", (n, k), {"hadamard": 128, "group": g}),
        ("layers.0.mlp.up.scale", s4, "f16", (k // g, n), None),
        ("layers.0.mlp.up.i8", q8, "q8c", (n, k), {"hadamard": 128, "group": 0}),
        ("layers.0.mlp.up.i8.scale", s8, "f32", (n,), None),
        ("embed", tbl8, "q8r", (10, 128), None),
        ("embed.scale", tsc8, "f32", (10,), None),
        ("ple", tbl4, "q4r", (6, 128), None),
        ("ple.scale", tsc4, "f16", (6, 2), None),
        ("norm", norm, "f32", (256,), None),
    ]


def main():
    fgm = load_writer()
    path = os.path.join(HERE, "ref_writer.fgm")
    w = fgm.FgmWriter(path)
    w.start_body(4096)
    expect = []
    for name, arr, dtype, shape, meta in payloads():
        e = w.add(name, arr, dtype, shape=shape, meta=meta)
        expect.append({"name": name, "dtype": dtype, "shape": list(shape), "offset": e["offset"],
                       "nbytes": e["nbytes"], "meta": meta or {},
                       "sha256": hashlib.sha256(np.ascontiguousarray(arr).tobytes()).hexdigest()})
    config = {"hidden_size": 256, "num_hidden_layers": 1}
    w.meta = {"converter": "reference convert/fgm.py FgmWriter"}
    w.close(config)
    with open(os.path.join(HERE, "ref_writer.json"), "w") as f:
        json.dump({"config": config, "meta": w.meta, "tensors": expect}, f, indent=1, sort_keys=True)
    print(f"wrote {path} ({os.path.getsize(path)} bytes), {len(expect)} tensors")


if __name__ == "__main__":
    main()
