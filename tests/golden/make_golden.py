"""Record the reference's own outputs for the golden cases.

Runs the reference's C -- vnni_gemm.c + ops.c (and amx_gemm.c where the host
has AMX), compiled from /root/reference's sources into oracle/_ref by
oracle/Makefile -- on the inputs built by tests/golden/cases.py, and writes
tests/golden/ref_outputs.json: per case a SHA-256 of the output bytes plus a
few sampled values (the inputs are regenerated from the recorded seeds, so no
input data is stored).

    make -C oracle ref && python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import oracle  # noqa: E402
import cases  # noqa: E402

P = oracle._ptr


def digest(*arrays: np.ndarray) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def samples(a: np.ndarray, n: int = 24) -> dict:
    flat = np.ascontiguousarray(a).ravel()
    idx = np.linspace(0, flat.size - 1, min(n, flat.size)).astype(np.int64)
    vals = flat[idx]
    if vals.dtype == np.float32:
        vals = vals.view(np.uint32)
    return {"idx": idx.tolist(), "bits": [int(v) for v in vals]}


def run_gemm(L, kind, M, N, K, group, n0, n1, inp, amx=False):
    C = np.zeros((M, N), np.float32)
    if kind == "q8c":
        f = L.fgm_gemm_q8c if amx else L.fgm_gemm_q8c_vnni
        f(M, N, K, P(inp["Ap"]), P(inp["a_s"]), P(inp["B"]), P(inp["bs"]), P(C), N, n0, n1)
    else:
        f = L.fgm_gemm_q4g if amx else L.fgm_gemm_q4g_vnni
        f(M, N, K, P(inp["Ap"]), P(inp["a_s"]), P(inp["B"]), P(inp["bs"]), group, P(C), N,
          n0, n1)
    return C


def main() -> None:
    R = oracle.ref()
    if R is None:
        sys.exit("oracle/_ref/libfgmref.so missing or host lacks AVX-512 VNNI: "
                 "run `make -C oracle ref` in the build container")
    RA = oracle.ref_amx()
    out: dict = {"source": "reference vnni_gemm.c/ops.c (+amx_gemm.c) built by oracle/Makefile",
                 "vnni": [], "amx": None}

    for case, inp in cases.vnni_inputs():
        kind, M, N, K, group, n0, n1 = case
        C = run_gemm(R, kind, M, N, K, group, n0, n1, inp)
        rec = {"case": list(case), "sha256": digest(C), "samples": samples(C)}
        if RA is not None:
            CA = run_gemm(RA, kind, M, N, K, group, n0, n1, inp, amx=True)
            rec["amx_sha256"] = digest(CA)
        out["vnni"].append(rec)

    a = cases.amx_inputs()
    M, N, K, g = a["M"], a["N"], a["K"], a["group"]
    amx = {}
    for m in (M, 8):
        Ap = oracle.pack_a(m, K, a["A"][:m])
        for kind in ("q8c", "q4g"):
            inp = dict(Ap=Ap, a_s=a["a_s"][:m].copy(),
                       B=a["B8"] if kind == "q8c" else a["Bq"],
                       bs=a["bs8"] if kind == "q8c" else a["bs4"])
            C = run_gemm(R, kind, m, N, K, g, 0, N // 16, inp)
            amx[f"{kind}_M{m}"] = {"sha256": digest(C), "samples": samples(C)}
            if RA is not None:
                amx[f"{kind}_M{m}"]["amx_sha256"] = digest(
                    run_gemm(RA, kind, m, N, K, g, 0, N // 16, inp, amx=True))
    out["amx"] = amx

    lay = cases.layout_inputs()
    ones8 = np.ones(lay["N"], np.float32)
    ones4 = np.full((lay["K"] // 64, lay["N"]), 0x3C00, np.uint16)  # f16 1.0
    Ap = oracle.pack_a(lay["M"], lay["K"], lay["A"])
    a1 = np.ones(lay["M"], np.float32)
    C8 = run_gemm(R, "q8c", lay["M"], lay["N"], lay["K"], 0, 0, lay["N"] // 16,
                  dict(Ap=Ap, a_s=a1, B=oracle.pack_b_tiles(lay["Q8"]), bs=ones8))
    C4 = run_gemm(R, "q4g", lay["M"], lay["N"], lay["K"], 64, 0, lay["N"] // 16,
                  dict(Ap=Ap, a_s=a1, B=oracle.pack_nibbles(oracle.pack_b_tiles(lay["Q4"])),
                       bs=ones4))
    out["layout"] = {"q8c_sha256": digest(C8), "q4g_sha256": digest(C4)}

    d = cases.dbg_inputs()
    inp = dict(Ap=oracle.pack_a(d["M"], d["K"], d["A"]), a_s=d["a_s"], B=d["Bq"], bs=d["bs"])
    C = run_gemm(R, "q4g", d["M"], d["N"], d["K"], d["group"], 0, d["N"] // 16, inp)
    out["dbg"] = {"sha256": digest(C), "samples": samples(C)}

    x, tail = cases.quant_rows()
    q = np.empty(x.shape, np.int8)
    s = np.empty(x.shape[0], np.float32)
    R.fgm_quant_act(P(x), x.shape[0], x.shape[1], P(q), P(s))
    qt = np.empty(tail.shape, np.int8)
    st = np.empty(tail.shape[0], np.float32)
    R.fgm_quant_act(P(tail), tail.shape[0], tail.shape[1], P(qt), P(st))
    out["quant_act"] = {"q_sha256": digest(q), "s_sha256": digest(s),
                        "tail_q_sha256": digest(qt), "tail_s_sha256": digest(st),
                        "s_bits": [int(v) for v in s.view(np.uint32)],
                        "tail_s_bits": [int(v) for v in st.view(np.uint32)]}

    fw = {}
    for hsz in (8, 16, 128, 256):
        y = cases.fwht_input(hsz).copy()
        R.fgm_fwht(P(y), y.size, hsz)
        fw[str(hsz)] = {"sha256": digest(y), "samples": samples(y)}
    out["fwht"] = fw

    m, k, lda, src = cases.prep_input()
    prep = {}
    for hsz in (0, 128):
        for split in ((0, m), (0, 16, 32, m)):
            rot = np.zeros((m, k), np.float32)
            qa = np.zeros((m, k), np.int8)
            qs = np.zeros(m, np.float32)
            pa = np.zeros(oracle.packed_a_len(m, k), np.int8)
            for r0, r1 in zip(split[:-1], split[1:]):
                R.fgm_prep_rows(P(src), lda, P(rot), P(qa), P(qs), P(pa), m, k, hsz, r0, r1)
            prep[f"hsz{hsz}_split{len(split) - 1}"] = {
                "sha256": digest(rot, qa, qs, pa), "pa_sha256": digest(pa),
                "qs_bits": [int(v) for v in qs.view(np.uint32)]}
    out["prep_rows"] = prep

    elem = {}
    for n in cases.ELEM_NS:
        e = cases.elem_inputs(n)
        o1 = np.empty(n, np.float32)
        R.fgm_rmsnorm(P(o1), P(e["x"]), P(e["w"]), n, 1e-6)
        o2 = np.empty(n, np.float32)
        R.fgm_rmsnorm_noscale(P(o2), P(e["x"]), n, 1e-6)
        o3 = np.empty(n, np.float32)
        R.fgm_gelu_mul(P(o3), P(e["gate"]), P(e["up"]), n)
        o4 = e["gate"].copy()
        R.fgm_gelu(P(o4), n)
        o5 = e["sc"].copy()
        R.fgm_softcap(P(o5), n, 30.0)
        o6 = e["x"].copy()
        R.fgm_add(P(o6), P(e["w"]), n)
        o7 = e["x"].copy()
        R.fgm_mul(P(o7), P(e["w"]), n)
        o8 = e["x"].copy()
        R.fgm_scale(P(o8), 0.7071067811865476, n)
        elem[str(n)] = {name: digest(a) for name, a in (
            ("rmsnorm", o1), ("rmsnorm_noscale", o2), ("gelu_mul", o3), ("gelu", o4),
            ("softcap", o5), ("add", o6), ("mul", o7), ("scale", o8))}
    rope = {}
    for nh, hd, pos in cases.ROPE_CASES:
        x, inv = cases.rope_inputs(nh, hd)
        y = x.copy()
        R.fgm_rope(P(y), nh, hd, P(inv), pos)
        rope[f"{nh}x{hd}@{pos}"] = digest(y)
    out["elem"] = elem
    out["rope"] = rope

    attn = {}
    for (name, nh, kvh, hd, cap, ring, st, en, h0, h1, qmul, path) in cases.ATTN_CASES:
        q, kv = cases.attn_inputs(name, nh, kvh, hd, cap, qmul)
        o = np.full(nh * hd, 7.0, np.float32)   # heads a call leaves alone keep 7.0
        oracle.ref_attend(path, q, kv, nh, st, en, h0, h1, ring, out=o)
        attn[name] = {"sha256": digest(o), "samples": samples(o)}
    out["attn"] = attn

    base = {}
    for name, (kind, M, N, K, group, _act) in cases.BASELINE_CASES.items():
        x, B, bs = cases.baseline_inputs(name)
        qa = np.zeros((M, K), np.int8)
        qs = np.zeros(M, np.float32)
        pa = np.zeros(oracle.packed_a_len(M, K), np.int8)
        rot = np.zeros((M, K), np.float32)
        R.fgm_prep_rows(P(x), K, P(rot), P(qa), P(qs), P(pa), M, K, 0, 0, M)
        C = run_gemm(R, kind, M, N, K, group, 0, N // 16, dict(Ap=pa, a_s=qs, B=B, bs=bs))
        base[name] = {"prep_sha256": digest(qs, pa), "c_sha256": digest(C), "samples": samples(C)}
    out["baseline"] = base

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_outputs.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main()
