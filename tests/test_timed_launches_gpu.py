"""The launches bench.py times, issued through bench.py's own call wrappers
(`bench.Gpu.prep_many`, `gemm_many`, `prep`, `q8c`) at the timed shapes, on
host-generated inputs, every output against the oracle:

* the headline step: one fgm_hip_prep_batch_dev call
  for both activations (M=8, k=2048 and k=8192), then one
  fgm_hip_gemm_batch_dev call with up (N=8192, K=2048) and down (N=2048,
  K=8192), int4 group 64;
* the decode step's batches: q/k/v (N=2048/512/512, K=2048) in
  one call, gate/up (N=8192 twice) in one call, int4 group 64, the int8 down
  projection (N=2048, K=8192);
* the prefill layer's batches: q/k/v, o, gate/up, down at M=256,
  int8, as bench.py's cfg3 layer issues them.

Bar: bit-exact (fp32 outputs, packed A and row scales).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests import hip_util as H

pytestmark = pytest.mark.gpu


def _bits_equal(x, y):
    return np.array_equal(np.ascontiguousarray(x).view(np.uint32), np.ascontiguousarray(y).view(np.uint32))


@pytest.fixture(scope="module")
def gpu():
    import bench
    return bench.Gpu()


def _act(gpu, seed, M, K):
    t = gpu.t
    x = oracle.gen_normal(seed, M * K).reshape(M, K)
    qs = t.full((M,), 7.0, device=gpu.dev)
    pa = t.full(((M + 15) // 16 * 16 * K,), 5, dtype=t.int8, device=gpu.dev)
    return x, H.dev(x), qs, pa


def _w4(seed, N, K):
    B = oracle.gen_u8(seed, N * K // 2)
    bs = oracle.gen_uniform(seed + 1, (K // 64) * N, 5e-3, 5e-2).astype(np.float16).view(np.uint16)
    return B, bs


def _w8(seed, N, K):
    return oracle.gen_i8(seed, N * K, -127, 127), oracle.gen_uniform(seed + 1, N, 1e-3, 1e-2)


def _want_prep(x, M, K):
    rq, rs = oracle.quant_act(x, M, K)
    return rs, oracle.pack_a(M, K, rq)


def _want_gemm(bits, M, N, K, pa, qs, B, bs):
    """All of [0, N/16) on the host threads: the reference's own VNNI kernels
    where oracle/_ref is built, else the oracle (same bytes, pinned)."""
    R = np.zeros((M, N), np.float32)
    oracle.gemm_pooled(bits, M, N, K, pa, qs, B, bs, 64, R, N)
    return R


def test_headline_step_prep_batch_and_pair_launch(gpu):
    """The cfg2 step as bench.py's step() issues it: prep_many over both
    activations, then gemm_many over up + down (one launch each)."""
    t = gpu.t
    xu, dxu, qsu, pau = _act(gpu, 501, 8, 2048)
    xd, dxd, qsd, pad_ = _act(gpu, 502, 8, 8192)
    print("cfg2 prep batch", flush=True)
    gpu.prep_many([(dxu, qsu, pau, 8, 2048), (dxd, qsd, pad_, 8, 8192)])
    for x, qs, pa, K in ((xu, qsu, pau, 2048), (xd, qsd, pad_, 8192)):
        rs, rpa = _want_prep(x, 8, K)
        assert _bits_equal(H.host(qs), rs), K
        assert np.array_equal(H.host(pa), rpa), K
    Bu, bsu = _w4(511, 8192, 2048)
    Bd, bsd = _w4(513, 2048, 8192)
    cu = t.full((8, 8192), 9.0, device=gpu.dev)
    cd = t.full((8, 2048), 9.0, device=gpu.dev)
    print("cfg2 pair launch", flush=True)
    gpu.gemm_many([(4, 8, 8192, 2048, pau, qsu, H.dev(Bu), H.dev(bsu), cu),
                   (4, 8, 2048, 8192, pad_, qsd, H.dev(Bd), H.dev(bsd), cd)])
    for c, B, bs, N, K, qs, pa in ((cu, Bu, bsu, 8192, 2048, qsu, pau), (cd, Bd, bsd, 2048, 8192, qsd, pad_)):
        R = _want_gemm(4, 8, N, K, H.host(pa), H.host(qs), B, bs)
        assert _bits_equal(H.host(c), R), N


def _layer_check(gpu, M, bits_of, batches, seed0):
    """Run bench.LAYER's projections in the given batches (lists of names)
    through gemm_many on two activations (K=2048 and K=8192) prepared by
    gpu.prep, and compare every output with the oracle."""
    import bench
    t = gpu.t
    shapes = {name: (N, K) for name, N, K in bench.LAYER}
    acts = {}
    for i, K in enumerate((2048, 8192)):
        x, dx, qs, pa = _act(gpu, seed0 + i, M, K)
        gpu.prep(dx, qs, pa, M, K)
        acts[K] = (qs, pa)
    ws, outs = {}, {}
    for i, (name, (N, K)) in enumerate(shapes.items()):
        bits = bits_of(name)
        ws[name] = (_w4 if bits == 4 else _w8)(seed0 + 10 + 2 * i, N, K)
        outs[name] = t.full((M, N), 9.0, device=gpu.dev)
    dws = {name: (H.dev(B), H.dev(bs)) for name, (B, bs) in ws.items()}
    for names in batches:
        print("batch", M, names, flush=True)
        items = []
        for name in names:
            N, K = shapes[name]
            qs, pa = acts[K]
            items.append((bits_of(name), M, N, K, pa, qs, dws[name][0], dws[name][1], outs[name]))
        gpu.gemm_many(items)
    for name, (N, K) in shapes.items():
        qs, pa = acts[K]
        R = _want_gemm(bits_of(name), M, N, K, H.host(pa), H.host(qs), *ws[name])
        assert _bits_equal(H.host(outs[name]), R), name


def test_decode_step_batches(gpu):
    """cfg4's per-layer launches at M=8: q/k/v int4 in one call, o, gate/up
    int4 in one call, down int8 (bench.py extra_cfg4)."""
    _layer_check(gpu, 8, lambda n: 8 if n == "down" else 4,
                 [["q", "k", "v"], ["o"], ["gate", "up"], ["down"]], 600)


def test_prefill_layer_batches(gpu):
    """cfg3's layer at M=256, int8: q/k/v in one call, o, gate/up in one
    call, down (bench.py extra_cfg3 layer())."""
    _layer_check(gpu, 256, lambda n: 8, [["q", "k", "v"], ["o"], ["gate", "up"], ["down"]], 700)


def test_decode_lm_head(gpu):
    """cfg4's int8 LM head, N=262144 K=2048 at M=8, through gpu.q8c: every
    output against the oracle."""
    t = gpu.t
    x, dx, qs, pa = _act(gpu, 801, 8, 2048)
    gpu.prep(dx, qs, pa, 8, 2048)
    B, bs = _w8(803, 262144, 2048)
    c = t.full((8, 262144), 9.0, device=gpu.dev)
    print("lm head", flush=True)
    gpu.q8c(8, 262144, 2048, pa, qs, H.dev(B), H.dev(bs), c)
    R = _want_gemm(8, 8, 262144, 2048, H.host(pa), H.host(qs), B, bs)
    assert _bits_equal(H.host(c), R)
