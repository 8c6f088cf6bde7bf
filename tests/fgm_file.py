"""Test infrastructure: writes .fgm files in the layout convert/fgm.py:1-16
documents -- magic b"FASTGEM1", u32 little-endian header length, the compact
JSON header {arch, config, meta, tensors}, tensor blobs 64-byte aligned at
absolute offsets after a reserved header area -- plus a small synthetic model
with the tensor kinds the converter writes (convert_gemma4.py:150-225)."""
from __future__ import annotations

import numpy as np

import oracle

from fastgemma_amd.fgm_format import write_fgm  # noqa: E402


CONFIG = {"hidden_size": 256, "num_hidden_layers": 1, "intermediate_size": 512,
          "num_attention_heads": 8, "num_key_value_heads": 1, "head_dim": 256,
          "global_head_dim": 512, "sliding_window": 512, "rms_norm_eps": 1e-6,
          "final_logit_softcapping": 30.0, "hadamard": 128, "layer_types": ["sliding_attention"],
          "quant": {"ffn": 4, "attn": 8, "ple": 4, "emb": 8}, "note": "qé \"quoted\" \\ /"}


def synthetic_model(path):
    """A file with every tensor kind: q4g linears (group 64 and 128, with and
    without an int8 twin), a q8c linear, q8r / q4r gather tables, f32 norms.
    Returns the arrays written, by name."""
    t = {}
    out = []

    def add(name, arr, dtype, shape, meta=None):
        t[name] = arr
        out.append((name, arr, dtype, shape, meta))

    # gate: q4g group 64, Hadamard 128, with an int8 twin
    n, k = 256, 512
    add("layers.0.mlp.gate", oracle.gen_u8(101, n * k // 2), "q4g", (n, k), {"hadamard": 128, "group": 64})
    add("layers.0.mlp.gate.scale",
        oracle.f32_to_f16(oracle.gen_uniform(102, (k // 64) * n, 0.005, 0.05)), "f16", (k // 64, n))
    add("layers.0.mlp.gate.i8", oracle.gen_i8(103, n * k, -127, 127), "q8c", (n, k), {"hadamard": 128, "group": 0})
    add("layers.0.mlp.gate.i8.scale", oracle.gen_uniform(104, n, 1e-3, 1e-2), "f32", (n,))
    # down: q4g group 128, no twin, no Hadamard
    n, k = 128, 512
    add("layers.0.mlp.down", oracle.gen_u8(111, n * k // 2), "q4g", (n, k), {"hadamard": 0, "group": 128})
    add("layers.0.mlp.down.scale",
        oracle.f32_to_f16(oracle.gen_uniform(112, (k // 128) * n, 0.005, 0.05)), "f16", (k // 128, n))
    # q: q8c, Hadamard 128, meta without a group key
    n, k = 128, 256
    add("layers.0.attn.q", oracle.gen_i8(121, n * k, -127, 127), "q8c", (n, k), {"hadamard": 128})
    add("layers.0.attn.q.scale", oracle.gen_uniform(122, n, 1e-3, 1e-2), "f32", (n,))
    # gather tables
    rows, k = 100, 256
    add("embed", oracle.gen_i8(131, rows * k, -127, 127), "q8r", (rows, k))
    add("embed.scale", oracle.gen_uniform(132, rows, 1e-3, 1e-2), "f32", (rows,))
    rows, k = 50, 256
    add("ple", oracle.gen_u8(141, rows * k // 2), "q4r", (rows, k))
    add("ple.scale", oracle.f32_to_f16(oracle.gen_uniform(142, rows * (k // 64), 0.005, 0.05)), "f16",
        (rows, k // 64))
    add("layers.0.input_ln", oracle.gen_normal(151, 256), "f32", (256,))
    add("odd \"name\" é", np.arange(7, dtype=np.int8), "i8", (7,))
    write_fgm(path, CONFIG, out, meta={"source": "synthetic"})
    return t
