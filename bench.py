"""Benchmark of the fgm-kernels quantized-matmul path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra] [--no-cpu]

Headline workload: batched decode skinny GEMM,
M = 8 activation rows ~ N(0,1) fp32, int4 weights group 64 with f16 scales,
two shapes -- up N=8192 K=2048 and down N=2048 K=8192.  One step = the hot
path over one batch: for each shape, quantise + tile-pack the fp32 rows
(prep kernel) and run the int4 GEMM with its fp32 epilogue.  Weights rotate
over 48 distinct copies (~870 MB), so no step finds its weights in the
256 MB MALL; inputs are resident in HBM before the timed region.  Steps are
launched as HIP graphs (torch.cuda.CUDAGraph is only the capture/replay
plumbing) so host launch overhead stays off the GPU timeline.

`value` = algorithmic bytes per step / step time, in GB/s, where the bytes are
weights + f16 scales + packed A + a_scale + f32 C of both GEMMs plus the
prep's fp32 read and packed-A write.

`roofline` is for the dominant kernel, the step's GEMM launch (the int4
skinny GEMM serving up and down in one launch): the average duration of one
launch, measured with HIP events around a graph of 48 back-to-back launches
on the launch stream; `traffic` comes from the committed rocprofv3 PMC
summary (profiles/decode_q4g_m8_pair_traffic.txt).

`cpu_baseline` runs the reference's own VNNI kernels (oracle/_ref, compiled
from the reference sources) on this host's cores with the reference's thread
split, on the same shapes, for about 10 s; falls back to the oracle port.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12        # B/s, MI355X HBM3E
I8_PEAK = 5.0e15         # dense int8 MFMA ops/s (MI355X, no sparsity)
NCOPY = 48


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------- byte counts
def gemm_bytes(bits, M, N, K, group=64):
    """Algorithmic bytes of one GEMM launch: weights + scales + the M rows of
    int8 A + a_scale + C (fp32).  The packed layout's pad rows (up to the next
    multiple of 16) carry no data and are not counted."""
    w = N * K if bits == 8 else N * K // 2
    s = N * 4 if bits == 8 else (K // group) * N * 2
    return w + s + M * K + 4 * M + 4 * M * N


def prep_bytes(M, K):
    """fp32 rows read + int8 rows and row scales written."""
    return 4 * M * K + M * K + 4 * M


# ---------------------------------------------------------------- plumbing
class Gpu:
    def __init__(self):
        import torch
        import fastgemma_amd as F
        from fastgemma_amd import kernels
        self.t = torch
        self.F = F
        self.L = F.lib()
        kernels.backend()
        self.dev = torch.device("cuda:0")

    def stream(self):
        return self.t.cuda.current_stream().cuda_stream

    def prep(self, x, qs, pa, M, K):
        rc = self.L.fgm_hip_prep_rows_dev(x.data_ptr(), K, None, None, qs.data_ptr(),
                                          pa.data_ptr(), M, K, 0, 0, M, self.stream())
        self.F.check(rc)

    def prep_many(self, items):
        """items: (x, qs, pa, M, K) -- one launch for all."""
        arr = (self.F.PrepDesc * len(items))()
        for i, (x, qs, pa, M, K) in enumerate(items):
            arr[i] = self.F.PrepDesc(x.data_ptr(), K, None, None, qs.data_ptr(), pa.data_ptr(),
                                     M, K, 0, 0, M)
        self.F.check(self.L.fgm_hip_prep_batch_dev(arr, len(items), self.stream()))

    def gemm_many(self, items):
        """items: (bits, M, N, K, pa, qs, w, s, c) -- as few launches as possible."""
        arr = (self.F.GemmDesc * len(items))()
        for i, (bits, M, N, K, pa, qs, w, s, c) in enumerate(items):
            arr[i] = self.F.GemmDesc(bits, M, N, K, 64, pa.data_ptr(), qs.data_ptr(), w.data_ptr(),
                                     s.data_ptr(), c.data_ptr(), N, 0, N // 16)
        self.F.check(self.L.fgm_hip_gemm_batch_dev(arr, len(items), self.stream()))

    def q4g(self, M, N, K, pa, qs, w, s, c, group=64):
        rc = self.L.fgm_hip_gemm_q4g_dev(M, N, K, pa.data_ptr(), qs.data_ptr(), w.data_ptr(),
                                         s.data_ptr(), group, c.data_ptr(), N, 0, N // 16,
                                         self.stream())
        self.F.check(rc)

    def q8c(self, M, N, K, pa, qs, w, s, c):
        rc = self.L.fgm_hip_gemm_q8c_dev(M, N, K, pa.data_ptr(), qs.data_ptr(), w.data_ptr(),
                                         s.data_ptr(), c.data_ptr(), N, 0, N // 16, self.stream())
        self.F.check(rc)

    # synthetic operands, generated on the device
    def w4(self, N, K, group=64):
        t = self.t
        w = t.randint(0, 256, (N * K // 2,), dtype=t.uint8, device=self.dev)
        s = (t.rand((K // group) * N, device=self.dev) * 0.045 + 0.005).half().view(t.int16)
        return w, s

    def w8(self, N, K):
        t = self.t
        w = t.randint(-127, 128, (N * K,), dtype=t.int8, device=self.dev)
        s = t.rand(N, device=self.dev) * 0.009 + 0.001
        return w, s

    def act(self, M, K):
        t = self.t
        x = t.randn(M, K, device=self.dev)
        qs = t.empty(M, device=self.dev)
        pa = t.empty((M + 15) // 16 * 16 * K, dtype=t.int8, device=self.dev)
        return x, qs, pa

    def graphs(self, fn, nsteps, chunk):
        """Capture fn(i) for i in [0, nsteps) as graphs of `chunk` steps."""
        t = self.t
        s = t.cuda.Stream()
        s.wait_stream(t.cuda.current_stream())
        with t.cuda.stream(s):
            for i in range(min(3, nsteps)):
                fn(i)
        t.cuda.current_stream().wait_stream(s)
        t.cuda.synchronize()
        out = []
        for b in range(0, nsteps, chunk):
            g = t.cuda.CUDAGraph()
            with t.cuda.graph(g):
                for i in range(b, min(nsteps, b + chunk)):
                    fn(i)
            out.append(g)
        t.cuda.synchronize()
        return out

    def time_graphs(self, gs, reps=1):
        """Seconds for `reps` passes over the graph list, HIP events on the
        replay stream, synchronize on both sides."""
        t = self.t
        t.cuda.synchronize()
        e0, e1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            for g in gs:
                g.replay()
        e1.record()
        t.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3

    def time_each(self, gs, reps):
        """Seconds of each of `reps` passes over the graph list, every pass
        bracketed by synchronize and HIP events on the replay stream."""
        return [self.time_graphs(gs, 1) for _ in range(reps)]


# ------------------------------------------------------------- workloads
def cfg2_setup(gpu):
    ups = [gpu.w4(8192, 2048) for _ in range(NCOPY)]
    downs = [gpu.w4(2048, 8192) for _ in range(NCOPY)]
    xu, qsu, pau = gpu.act(8, 2048)
    xd, qsd, pad_ = gpu.act(8, 8192)
    cu = gpu.t.empty(8, 8192, device=gpu.dev)
    cd = gpu.t.empty(8, 2048, device=gpu.dev)

    def gemms(c):
        return [(4, 8, 8192, 2048, pau, qsu, ups[c][0], ups[c][1], cu),
                (4, 8, 2048, 8192, pad_, qsd, downs[c][0], downs[c][1], cd)]

    def step(i):
        # one prep launch for both activations, one GEMM launch for both shapes
        gpu.prep_many([(xu, qsu, pau, 8, 2048), (xd, qsd, pad_, 8, 8192)])
        gpu.gemm_many(gemms(i % NCOPY))

    def gemv_pair(i):
        gpu.gemm_many(gemms(i % NCOPY))

    def gemv_up(i):
        c = i % NCOPY
        gpu.q4g(8, 8192, 2048, pau, qsu, ups[c][0], ups[c][1], cu)

    def gemv_down(i):
        c = i % NCOPY
        gpu.q4g(8, 2048, 8192, pad_, qsd, downs[c][0], downs[c][1], cd)

    step_bytes = (gemm_bytes(4, 8, 8192, 2048) + gemm_bytes(4, 8, 2048, 8192)
                  + prep_bytes(8, 2048) + prep_bytes(8, 8192))
    host = dict(up=(ups[0][0].cpu().numpy(), ups[0][1].cpu().numpy()),
                down=(downs[0][0].cpu().numpy(), downs[0][1].cpu().numpy()))
    return step, gemv_pair, gemv_up, gemv_down, step_bytes, host


def med_range(ts):
    """(median, min, max) of a list of times."""
    s = sorted(ts)
    return s[len(s) // 2], s[0], s[-1]


def kernel_time(gpu, fn, n=NCOPY, reps=5):
    """Seconds per launch of fn, from `reps` timed replays of a graph of n
    back-to-back launches: (median, min, max) over the replays."""
    gs = gpu.graphs(fn, n, n)
    gpu.time_graphs(gs, 2)
    return tuple(x / n for x in med_range(gpu.time_each(gs, reps)))


def kernel_avg(gpu, fn, n=NCOPY, reps=5):
    """Median seconds per launch of fn (kernel_time)."""
    return kernel_time(gpu, fn, n, reps)[0]


def extra_cfg1(gpu):
    ws = [gpu.w8(8192, 2048) for _ in range(24)]   # 24 x 16.8 MB = 403 MB > MALL
    x, qs, pa = gpu.act(1, 2048)
    c = gpu.t.empty(1, 8192, device=gpu.dev)
    gpu.prep(x, qs, pa, 1, 2048)
    dt, lo, hi = kernel_time(gpu, lambda i: gpu.q8c(1, 8192, 2048, pa, qs, ws[i % 24][0], ws[i % 24][1], c), 24)
    b = gemm_bytes(8, 1, 8192, 2048)
    return {"workload": "int8 GEMV M=1 N=8192 K=2048", "us_per_launch": dt * 1e6,
            "us_range": [lo * 1e6, hi * 1e6],
            "GB_s": b / dt / 1e9, "frac_hbm": b / dt / HBM_PEAK, "bytes_per_launch": b}


def extra_int4_stream(gpu):
    """The int4 skinny kernel's sustained rate on one large weight (M=8,
    N=131072, K=2048, 134 MB; two copies > MALL): what the kernel streams
    once the fixed per-launch cost (~2-3 us) is amortised.  Not a BASELINE
    config; it bounds what a fused forward pass could reach."""
    N, K = 131072, 2048
    ws = [gpu.w4(N, K) for _ in range(2)]
    x, qs, pa = gpu.act(8, K)
    gpu.prep(x, qs, pa, 8, K)
    c = gpu.t.empty(8, N, device=gpu.dev)
    dt, lo, hi = kernel_time(gpu, lambda i: gpu.q4g(8, N, K, pa, qs, ws[i % 2][0], ws[i % 2][1], c), 8, 5)
    b = gemm_bytes(4, 8, N, K)
    return {"workload": "int4 g64 M=8 N=131072 K=2048 (134 MB weights), one launch",
            "us_per_launch": dt * 1e6, "us_range": [lo * 1e6, hi * 1e6], "GB_s": b / dt / 1e9,
            "frac_hbm": b / dt / HBM_PEAK}


LAYER = [("q", 2048, 2048), ("k", 512, 2048), ("v", 512, 2048), ("o", 2048, 2048),
         ("gate", 8192, 2048), ("up", 8192, 2048), ("down", 2048, 8192)]


def attainable(bits, M, N, K, group=64):
    """min(peak, AI x 8 TB/s) for one GEMM: AI = 2 M N K ops over the bytes it
    must move at least once (weights + scales + packed A + a_scale + f32 C)."""
    ai = 2.0 * M * N * K / gemm_bytes(bits, M, N, K, group)
    return min(I8_PEAK, ai * HBM_PEAK)


COLD = 320 * 1000 * 1000   # bytes of rotating weight copies: more than the 256 MB MALL


def extra_cfg3(gpu):
    """The seven M=256 int8 projections, each on weights rotating over more
    than the MALL holds (a prefill reads its layer's weights from HBM), and
    the layer as the forward pass issues it (four launches)."""
    res, tot_ops, tot_t = {}, 0.0, 0.0
    xs = {K: gpu.act(256, K) for K in (2048, 8192)}
    for K, (x, qs, pa) in xs.items():
        gpu.prep(x, qs, pa, 256, K)
    for name, N, K in LAYER:
        ncp = -(-COLD // (N * K))
        ws = [gpu.w8(N, K) for _ in range(ncp)]
        x, qs, pa = xs[K]
        c = gpu.t.empty(256, N, device=gpu.dev)
        dt, lo, hi = kernel_time(gpu, lambda i: gpu.q8c(256, N, K, pa, qs, ws[i % ncp][0], ws[i % ncp][1], c),
                                 max(20, ncp))
        # the same launch on one weight copy (L2 / MALL resident), for reference
        wt = kernel_time(gpu, lambda i: gpu.q8c(256, N, K, pa, qs, ws[0][0], ws[0][1], c), 20)[0]
        ops = 2.0 * 256 * N * K
        res[name] = {"us": dt * 1e6, "us_range": [lo * 1e6, hi * 1e6], "TOPS": ops / dt / 1e12,
                     "frac_mfma": ops / dt / I8_PEAK, "frac_attainable": ops / dt / attainable(8, 256, N, K),
                     "weight_copies": ncp, "us_one_copy": wt * 1e6}
        tot_ops += ops
        tot_t += dt
        del ws
        gpu.t.cuda.empty_cache()
    # the layer as the forward pass issues it: q/k/v on one activation in one
    # launch, o, gate/up in one launch, down (forward.rs:484-641); six copies
    # of the layer's 58 MB
    nl = 6
    lw = [{name: gpu.w8(N, K) for name, N, K in LAYER} for _ in range(nl)]
    outs = {name: gpu.t.empty(256, N, device=gpu.dev) for name, N, K in LAYER}

    def item(i, name):
        N, K = next((N, K) for nm, N, K in LAYER if nm == name)
        x, qs, pa = xs[K]
        w = lw[i % nl][name]
        return (8, 256, N, K, pa, qs, w[0], w[1], outs[name])

    def layer(i):
        gpu.gemm_many([item(i, "q"), item(i, "k"), item(i, "v")])
        gpu.gemm_many([item(i, "o")])
        gpu.gemm_many([item(i, "gate"), item(i, "up")])
        gpu.gemm_many([item(i, "down")])
    gs = gpu.graphs(layer, 12, 12)
    gpu.time_graphs(gs, 2)
    lt, llo, lhi = (x / 12 for x in med_range(gpu.time_each(gs, 7)))
    g1 = gpu.graphs(lambda i: layer(0), 12, 12)
    gpu.time_graphs(g1, 2)
    l1 = med_range(gpu.time_each(g1, 7))[0] / 12
    return {"workload": "int8 prefill M=256, 7 projection shapes of one layer, weights rotating over "
                        "> 256 MB (from HBM)",
            "per_shape": res, "layer_us": tot_t * 1e6, "TOPS": tot_ops / tot_t / 1e12,
            "frac_mfma": tot_ops / tot_t / I8_PEAK,
            "layer_batched": {"launches": 4, "us": lt * 1e6, "us_range": [llo * 1e6, lhi * 1e6],
                              "TOPS": tot_ops / lt / 1e12, "frac_mfma": tot_ops / lt / I8_PEAK,
                              "note": "q/k/v and gate/up each share one launch",
                              "us_one_copy": l1 * 1e6},
            "tokens_per_s_30_layers": 256 / (30 * lt)}


def extra_cfg4(gpu):
    """30 synthetic layers (q,k,v,o,gate,up int4 g64; down int8) + int8 LM
    head [262144, 2048], M = 8, distinct buffers, one graph per step."""
    layers = []
    for _ in range(30):
        L = {}
        for name, N, K in LAYER:
            L[name] = gpu.w8(N, K) if name == "down" else gpu.w4(N, K)
        layers.append(L)
    head = gpu.w8(262144, 2048)
    a2 = gpu.act(8, 2048)
    a8 = gpu.act(8, 8192)
    outs = {name: gpu.t.empty(8, N, device=gpu.dev) for name, N, K in LAYER}
    logits = gpu.t.empty(8, 262144, device=gpu.dev)

    def w(L, name, bits, pa, qs):
        N, K = next((N, K) for nm, N, K in LAYER if nm == name)
        return (bits, 8, N, K, pa, qs, L[name][0], L[name][1], outs[name])

    def step(_i, prep=True):
        # the reference forward's GEMM sequence per layer (forward.rs:484-641):
        # q/k/v on one activation, o, gate/up on one activation, down
        x, qs, pa = a2
        xd, qsd, pad_ = a8
        for L in layers:
            if prep:
                gpu.prep(x, qs, pa, 8, 2048)              # attention input
            gpu.gemm_many([w(L, "q", 4, pa, qs), w(L, "k", 4, pa, qs), w(L, "v", 4, pa, qs)])
            if prep:
                gpu.prep(x, qs, pa, 8, 2048)              # attention output
            gpu.gemm_many([w(L, "o", 4, pa, qs)])
            if prep:
                gpu.prep(x, qs, pa, 8, 2048)              # FFN input
            gpu.gemm_many([w(L, "gate", 4, pa, qs), w(L, "up", 4, pa, qs)])
            if prep:
                gpu.prep(xd, qsd, pad_, 8, 8192)         # FFN hidden
            gpu.gemm_many([w(L, "down", 8, pad_, qsd)])
        if prep:
            gpu.prep(x, qs, pa, 8, 2048)
        gpu.q8c(8, 262144, 2048, pa, qs, head[0], head[1], logits)

    gs = gpu.graphs(step, 1, 1)
    gpu.time_graphs(gs, 3)
    dt, lo, hi = med_range(gpu.time_each(gs, 20))
    # GEMM-only, as the reference's bench also times it (the packed
    # activations the preps above left behind)
    gg = gpu.graphs(lambda i: step(i, prep=False), 1, 1)
    gpu.time_graphs(gg, 3)
    gt, glo, ghi = med_range(gpu.time_each(gg, 20))
    wbytes = 0
    for name, N, K in LAYER:
        wbytes += (N * K + N * 4) if name == "down" else (N * K // 2 + (K // 64) * N * 2)
    wbytes = wbytes * 30 + 262144 * 2048 + 262144 * 4
    allb = 0
    for name, N, K in LAYER:
        allb += gemm_bytes(8 if name == "down" else 4, 8, N, K)
    allb = allb * 30 + gemm_bytes(8, 8, 262144, 2048) + 30 * (3 * prep_bytes(8, 2048) + prep_bytes(8, 8192)) + prep_bytes(8, 2048)
    return {"workload": "decode step M=8: 30 layers + int8 LM head, 242 launches (q/k/v and "
                        "gate/up batched), one graph",
            "us_per_step": dt * 1e6, "us_range": [lo * 1e6, hi * 1e6], "weight_bytes": wbytes,
            "gemm_only": {"launches": 121, "us_per_step": gt * 1e6, "us_range": [glo * 1e6, ghi * 1e6],
                          "GB_s_weights": wbytes / gt / 1e9},
            "GB_s_weights": wbytes / dt / 1e9,
            "GB_s_all": allb / dt / 1e9, "frac_hbm": allb / dt / HBM_PEAK,
            "tokens_per_s": 8 / dt}


def extra_cfg5(gpu):
    res = {}
    x2, qs2, pa2 = gpu.act(2048, 2048)
    x8, qs8, pa8 = gpu.act(2048, 8192)
    gpu.prep(x2, qs2, pa2, 2048, 2048)
    gpu.prep(x8, qs8, pa8, 2048, 8192)
    for name, bits, N, K in (("gate", 4, 8192, 2048), ("up", 4, 8192, 2048), ("down", 8, 2048, 8192)):
        ws = [gpu.w4(N, K) if bits == 4 else gpu.w8(N, K) for _ in range(2)]
        c = gpu.t.empty(2048, N, device=gpu.dev)
        if bits == 4:
            fn = lambda i: gpu.q4g(2048, N, K, pa2, qs2, ws[i % 2][0], ws[i % 2][1], c)
        else:
            fn = lambda i: gpu.q8c(2048, N, K, pa8, qs8, ws[i % 2][0], ws[i % 2][1], c)
        dt, lo, hi = kernel_time(gpu, fn, 8, 5)
        ops = 2.0 * 2048 * N * K
        res[name] = {"bits": bits, "us": dt * 1e6, "us_range": [lo * 1e6, hi * 1e6], "TOPS": ops / dt / 1e12,
                     "frac_mfma": ops / dt / I8_PEAK,
                     "frac_attainable": ops / dt / attainable(bits, 2048, N, K)}
    return {"workload": "long prefill M=2048 (gate/up int4 g64, down int8)", "per_shape": res}


def extra_ceilings(gpu):
    """The floors the roofline fractions are read against, measured on this box
    by fastgemma_amd/csrc/fgm_ceil.hip: the back-to-back launch floor, pure-read
    floors at the decode sizes (rotating buffers, so each read comes from
    HBM), a plain copy (the kernel that calibrates FETCH_SIZE / WRITE_SIZE),
    and the dense int8 MFMA rate with independent chains on every SIMD."""
    import ctypes as C
    L = C.CDLL(os.path.join(ROOT, "fastgemma_amd", "libfgm_ceil.so"))
    L.fgm_ceil_empty.argtypes = [C.c_int, C.c_int, C.c_void_p]
    L.fgm_ceil_read.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.c_void_p, C.c_void_p]
    L.fgm_ceil_copy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
    L.fgm_ceil_read_lds.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    L.fgm_ceil_mfma.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    t = gpu.t

    def ok(rc):
        if rc != 0:
            raise RuntimeError(f"fgm_ceil call failed: {rc}")

    res = {}
    for nwg, thr in ((1, 64), (256, 256), (256, 1024)):
        dt = kernel_avg(gpu, lambda i: ok(L.fgm_ceil_empty(nwg, thr, gpu.stream())), 64, 5)
        res[f"empty_launch_{nwg}x{thr}_us"] = dt * 1e6
    chunk = 16 * 8 * 1024  # a multiple of every probe's per-workgroup bytes
    sink = t.zeros(600 * 1000 * 1000 // 4096, dtype=t.int32, device=gpu.dev)
    reads = {}
    for mb, copies in ((18, 48), (134, 6), (537, 2)):
        nbytes = (mb * 1000 * 1000) // chunk * chunk
        bufs = [t.empty(nbytes, dtype=t.uint8, device=gpu.dev) for _ in range(copies)]
        best, best_lds = None, None
        for u in (1, 2, 4, 8):
            dt = kernel_avg(gpu, lambda i: ok(L.fgm_ceil_read(bufs[i % copies].data_ptr(), nbytes, u,
                                                              sink.data_ptr(), gpu.stream())),
                            max(copies, 8), 3)
            if best is None or dt < best[0]:
                best = (dt, f"register loads, {4 * u} KiB per 4-wave workgroup")
        # the skinny GEMM's path: 1 KB LDS-DMA units, 16-wave workgroups
        for nw, u in ((16, 4), (16, 2), (16, 8), (8, 8), (8, 4)):
            dt = kernel_avg(gpu, lambda i: ok(L.fgm_ceil_read_lds(bufs[i % copies].data_ptr(), nbytes, nw, u,
                                                                  sink.data_ptr(), gpu.stream())),
                            max(copies, 8), 3)
            if best_lds is None or dt < best_lds[0]:
                best_lds = (dt, f"LDS-DMA, {nw} waves x {u} KiB per workgroup")
        top = min(best, best_lds)
        reads[f"{mb}MB"] = {"bytes": nbytes, "us": top[0] * 1e6, "GB_s": nbytes / top[0] / 1e9,
                            "frac_hbm": nbytes / top[0] / HBM_PEAK, "path": top[1],
                            "register_loads_us": best[0] * 1e6, "lds_dma_us": best_lds[0] * 1e6}
        del bufs
        t.cuda.empty_cache()
    res["read_one_launch"] = reads
    nbytes = 512 << 20
    src = t.empty(nbytes, dtype=t.uint8, device=gpu.dev)
    dst = t.empty(nbytes, dtype=t.uint8, device=gpu.dev)
    dt = kernel_avg(gpu, lambda i: ok(L.fgm_ceil_copy(src.data_ptr(), dst.data_ptr(), nbytes, 4096,
                                                      gpu.stream())), 4, 3)
    res["copy_512MiB"] = {"bytes_read": nbytes, "bytes_written": nbytes, "us": dt * 1e6,
                          "GB_s": 2 * nbytes / dt / 1e9}
    del src, dst
    t.cuda.empty_cache()
    res["grid_barrier"] = ceil_gridbar(gpu, L, ok)
    iters = 2000
    for shape, ops1 in ((32, 65536), (16, 32768)):
        nwg = 1024
        dt = kernel_avg(gpu, lambda i: ok(L.fgm_ceil_mfma(shape, nwg, iters, sink.data_ptr(),
                                                          gpu.stream())), 4, 3)
        ops = nwg * 4 * iters * 4 * ops1
        res[f"mfma_i8_{shape}"] = {"TOPS": ops / dt / 1e12, "frac_of_5000": ops / dt / I8_PEAK,
                                   "us": dt * 1e6}
    return {"workload": "ceiling probes (fgm_ceil.hip): launch floor, one-launch read floors, "
                        "copy, int8 MFMA rate", **res}


def extra_sweep(gpu):
    """Where the paths cross on this GPU (bench/kernels/gemm_bench.c:105-133
    measures the same on the CPU): the cfg2 up shape (N=8192, K=2048) at
    M = 8 .. 512, int8 per-channel and int4 with group 64 / 128 / 256 / 512,
    weights rotating over more than the MALL.  Reports each point's time and
    path, the row count where the library switches from the skinny to the
    dense kernel, and per group size the smallest M from which int8 is at
    least as fast as int4 (the FGM_WEIGHTS=auto:M threshold this GPU
    suggests; forward.rs:26-89 ships auto:16 for the CPU)."""
    from fastgemma_amd import kernels
    N, K = 8192, 2048
    Ms = (8, 16, 32, 48, 64, 65, 96, 128, 256, 512)
    groups = (64, 128, 256, 512)
    n8 = -(-COLD // (N * K))
    n4 = -(-COLD // (N * K // 2))
    w8 = [gpu.w8(N, K) for _ in range(n8)]
    w4 = [gpu.t.randint(0, 256, (N * K // 2,), dtype=gpu.t.uint8, device=gpu.dev) for _ in range(n4)]
    s4 = {g: [(gpu.t.rand((K // g) * N, device=gpu.dev) * 0.045 + 0.005).half().view(gpu.t.int16)
              for _ in range(n4)] for g in groups}
    pts = {}
    for M in Ms:
        x, qs, pa = gpu.act(M, K)
        gpu.prep(x, qs, pa, M, K)
        c = gpu.t.empty(M, N, device=gpu.dev)
        row = {}
        dt = kernel_time(gpu, lambda i: gpu.q8c(M, N, K, pa, qs, w8[i % n8][0], w8[i % n8][1], c),
                         max(16, n8), 3)[0]
        row["q8c"] = {"us": dt * 1e6, "path": kernels.gemm_path(8, M, K)}
        for g in groups:
            dt = kernel_time(gpu, lambda i: gpu.q4g(M, N, K, pa, qs, w4[i % n4], s4[g][i % n4], c, g),
                             max(16, n4), 3)[0]
            row[f"q4g{g}"] = {"us": dt * 1e6, "path": kernels.gemm_path(4, M, K, g)}
        for v in row.values():
            v["TOPS"] = 2.0 * M * N * K / (v["us"] * 1e-6) / 1e12
        pts[M] = row
    switch = {k: next((M for M in Ms if pts[M][k]["path"] == "dense"), None) for k in pts[Ms[0]]}
    int8_from = {}
    for g in groups:
        key = f"q4g{g}"
        int8_from[key] = next((M for M in Ms if all(pts[m]["q8c"]["us"] <= pts[m][key]["us"]
                                                    for m in Ms if m >= M)), None)
    return {"workload": "M sweep on N=8192 K=2048: q8c and q4g g64..512, cold weights",
            "points": {str(M): {k: {"us": round(v["us"], 2), "TOPS": round(v["TOPS"], 1), "path": v["path"]}
                                for k, v in r.items()} for M, r in pts.items()},
            "dense_from_M": switch, "int8_not_slower_from_M": int8_from}


def ceil_gridbar(gpu, L, ok):
    """Cost of one device-wide barrier inside a cooperative launch (what a
    persistent kernel spanning a layer's dependent GEMMs would pay instead of
    a kernel boundary, ~1.66 us here): per variant (fgm_ceil.hip) and grid,
    (time of 250 barriers - time of 50) / 200, every workgroup handing 2 KB
    across each barrier; stale reads and spin-limit exits are counted."""
    import ctypes as C
    L.fgm_ceil_gridbar.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
    L.fgm_ceil_gridbar_bytes.restype = C.c_size_t
    t = gpu.t
    names = {0: "agent fences, acquire polls", 1: "agent fences, relaxed polls",
             2: "agent fences, relaxed polls, non-temporal outputs", 3: "no fences (atomics only)",
             4: "8 group counters, one release fence per group, relaxed polls",
             5: "8 group counters, no fences (atomics only)"}
    out = {}
    for v in (0, 1, 2, 3, 4, 5):
        for nwg in (256, 512):
            bar = t.zeros(L.fgm_ceil_gridbar_bytes() // 4, dtype=t.int32, device=gpu.dev)
            buf = t.zeros(2 * nwg * 512, dtype=t.float32, device=gpu.dev)
            stale = t.zeros(1, dtype=t.int32, device=gpu.dev)

            def run(iters):
                bar.zero_()
                e0, e1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
                e0.record()
                ok(L.fgm_ceil_gridbar(v, nwg, iters, bar.data_ptr(), buf.data_ptr(), stale.data_ptr(),
                                      gpu.stream()))
                e1.record()
                t.cuda.synchronize()
                return e0.elapsed_time(e1) / 1e3, int(bar[2].item())
            run(50)
            t_lo, e_lo = run(50)
            t_hi, e_hi = run(250)
            out[f"v{v} {nwg}wg"] = {"variant": names[v], "us_per_barrier": (t_hi - t_lo) / 200 * 1e6,
                                    "stale_reads": int(stale.item()), "spin_limit_hit": bool(e_lo or e_hi)}
    return out


def extra_vendor(gpu):
    """The vendor int8 GEMM (torch._int_mm, served by hipBLASLt / rocBLAS on
    ROCm) on the prefill shapes, int32 output, no scales: a reference point
    for the dense kernel (which also runs the fp32 epilogue), not part of the
    path."""
    t = gpu.t
    res = {}
    for name, M, N, K in (("q", 256, 2048, 2048), ("k", 256, 512, 2048), ("gate", 256, 8192, 2048),
                          ("down", 256, 2048, 8192), ("cfg5_down", 2048, 2048, 8192)):
        A = t.randint(-127, 128, (M, K), dtype=t.int8, device=gpu.dev)
        Bs = [t.randint(-127, 128, (N, K), dtype=t.int8, device=gpu.dev) for _ in range(8)]
        dt = kernel_avg(gpu, lambda i: t._int_mm(A, Bs[i % 8].t()), 16, 3)
        res[name] = {"us": dt * 1e6, "TOPS": 2.0 * M * N * K / dt / 1e12}
    return {"workload": "torch._int_mm (vendor int8 GEMM), int32 out, graphs of 16", "per_shape": res}


def extra_elem(gpu):
    """The elementwise primitives between the GEMMs (rmsnorm, gelu_mul, rope,
    add, softcap), at the model's decode (M=8) and prefill (M=256, 2048)
    shapes, hidden 2048, FFN 8192, 8 heads x 256, logits 262144.  HBM-bound;
    bytes = reads + writes of f32 operands."""
    import numpy as np
    from fastgemma_amd import kernels
    t = gpu.t
    L, F = gpu.L, gpu.F
    res = {}

    def rec(name, fn, nbytes, n=24):
        dt = kernel_avg(gpu, fn, n, 3)
        res[name] = {"us": dt * 1e6, "GB_s": nbytes / dt / 1e9, "frac_hbm": nbytes / dt / HBM_PEAK,
                     "bytes": nbytes}

    for M in (8, 256, 2048):
        x = t.randn(M, 2048, device=gpu.dev)
        w = t.randn(2048, device=gpu.dev)
        o = t.empty_like(x)
        rec(f"rmsnorm M={M} n=2048",
            lambda i: F.check(L.fgm_hip_rmsnorm_dev(o.data_ptr(), x.data_ptr(), w.data_ptr(), M, 2048,
                                                    1e-6, gpu.stream())),
            8 * M * 2048 + 4 * 2048)
        g = t.randn(M * 8192, device=gpu.dev)
        u = t.randn(M * 8192, device=gpu.dev)
        go = t.empty_like(g)
        rec(f"gelu_mul M={M} n=8192",
            lambda i: F.check(L.fgm_hip_gelu_mul_dev(go.data_ptr(), g.data_ptr(), u.data_ptr(),
                                                     M * 8192, gpu.stream())),
            12 * M * 8192)
        a = t.randn(M * 2048, device=gpu.dev)
        b = t.randn(M * 2048, device=gpu.dev)
        rec(f"add M={M} n=2048",
            lambda i: F.check(L.fgm_hip_add_dev(a.data_ptr(), b.data_ptr(), M * 2048, gpu.stream())),
            12 * M * 2048)
        q = t.randn(M, 8 * 256, device=gpu.dev)
        inv = (1e6 ** (-np.arange(0, 256, 2, dtype=np.float64) / 256)).astype(np.float32)
        cs = t.from_numpy(np.stack([kernels.rope_table(inv, 256, 100 + r) for r in range(M)])).to(gpu.dev)
        rec(f"rope M={M} 8x256",
            lambda i: F.check(L.fgm_hip_rope_dev(q.data_ptr(), M, 8, 256, cs.data_ptr(), gpu.stream())),
            8 * M * 2048 + cs.numel() * 4)
    lg = t.randn(8 * 262144, device=gpu.dev)
    rec("softcap logits M=8 n=262144",
        lambda i: F.check(L.fgm_hip_softcap_dev(lg.data_ptr(), 8 * 262144, 30.0, gpu.stream())),
        8 * 8 * 262144)
    return {"workload": "elementwise primitives, one launch each, graphs of 24 back-to-back "
                        "launches (a launch costs >= 1.8 us on this box)", "per_op": res}


def extra_prep_fused(gpu):
    """The GEMM inputs' producers fused into the prep kernel: rmsnorm + prep
    (before q/k/v and gate/up, hidden 2048) and gelu_mul + prep (before down,
    FFN 8192), with and without the rotation, one launch, against the two separate launches,
    at decode (M=8) and prefill (M=256) row counts.  Bytes of the fused form =
    f32 input(s) + weight + int8 packed output + row scales."""
    t = gpu.t
    L, F = gpu.L, gpu.F
    res = {}
    for M in (8, 256):
        # hsz 128: the converter's rotation for every linear (convert_gemma4.py:37)
        for kind, k, hsz in (("rmsnorm", 2048, 0), ("rmsnorm", 2048, 128), ("gelu_mul", 8192, 128),
                             ("gelu_mul", 8192, 512)):
            x = t.randn(M, k, device=gpu.dev)
            aux = t.randn(k if kind == "rmsnorm" else M * k, device=gpu.dev)
            mid = t.empty(M, k, device=gpu.dev)
            qs = t.empty(M, device=gpu.dev)
            pa = t.empty((M + 15) // 16 * 16 * k, dtype=t.int8, device=gpu.dev)
            if kind == "rmsnorm":
                def sep(i):
                    F.check(L.fgm_hip_rmsnorm_dev(mid.data_ptr(), x.data_ptr(), aux.data_ptr(), M, k,
                                                  1e-6, gpu.stream()))
                    F.check(L.fgm_hip_prep_rows_dev(mid.data_ptr(), k, None, None, qs.data_ptr(),
                                                    pa.data_ptr(), M, k, hsz, 0, M, gpu.stream()))

                def fused(i):
                    F.check(L.fgm_hip_prep_rmsnorm_dev(x.data_ptr(), k, aux.data_ptr(), 1e-6, None,
                                                       None, None, qs.data_ptr(), pa.data_ptr(), M,
                                                       k, hsz, gpu.stream()))
                nbytes = 4 * M * k + 4 * k + pa.numel() + 4 * M
            else:
                def sep(i):
                    F.check(L.fgm_hip_gelu_mul_dev(mid.data_ptr(), x.data_ptr(), aux.data_ptr(), M * k,
                                                   gpu.stream()))
                    F.check(L.fgm_hip_prep_rows_dev(mid.data_ptr(), k, None, None, qs.data_ptr(),
                                                    pa.data_ptr(), M, k, hsz, 0, M, gpu.stream()))

                def fused(i):
                    F.check(L.fgm_hip_prep_gelu_mul_dev(x.data_ptr(), aux.data_ptr(), k, None, None,
                                                        None, qs.data_ptr(), pa.data_ptr(), M, k, hsz,
                                                        gpu.stream()))
                nbytes = 8 * M * k + pa.numel() + 4 * M
            ts = kernel_avg(gpu, sep, 24, 3)
            tf = kernel_avg(gpu, fused, 24, 3)
            res[f"{kind}+prep M={M} k={k} hsz={hsz}"] = {
                "separate_us": ts * 1e6, "fused_us": tf * 1e6, "speedup": ts / tf,
                "fused_GB_s": nbytes / tf / 1e9, "bytes": nbytes}
    return {"workload": "producer + prep_rows: two launches vs the fused launch, graphs of 24",
            "per_op": res}


def extra_attn(gpu):
    """int8-KV attention (the forward pass's other hot loop, ops.c:353-877),
    one fgm_hip_attend_dev call (three launches) per layer: batched decode of
    8 sequences and a 256-row prefill chunk, full attention (head_dim 512,
    8192 positions) and sliding (head_dim 256, window 512, ring 520); 8 query
    heads on one kv head.  Bytes = K and V bytes (+ scales) each row reads."""
    import numpy as np
    from fastgemma_amd import kernels
    t = gpu.t
    res = {}
    nh = 8

    def cache(cap, hd, copies):
        out = []
        for _ in range(copies):
            kc = t.randint(-127, 128, (cap * hd,), dtype=t.int8, device=gpu.dev)
            vt = t.randint(-127, 128, ((cap + 3) // 4 * 4 * hd,), dtype=t.int8, device=gpu.dev)
            ks = t.rand(cap, device=gpu.dev) * 0.01 + 0.001
            vs = t.rand(cap, device=gpu.dev) * 0.01 + 0.001
            out.append((kc, ks, vt, vs))
        return out

    for name, hd, cap, ring, window, nseq, rows, pos in (
            ("decode full M=8 ctx 8192 hd 512", 512, 8192, 0, 0, 8, 1, 8191),
            ("decode sliding M=8 win 512 hd 256", 256, 520, 520, 512, 8, 1, 20000),
            ("prefill full 256 rows ctx 8192 hd 512", 512, 8192, 0, 0, 1, 256, 7936),
            ("prefill sliding 256 rows win 512 hd 256", 256, 768, 768, 512, 1, 256, 20000)):
        copies = 2 if nseq == 1 else 1
        caches = [cache(cap, hd, copies) for _ in range(nseq)]
        m = nseq * rows
        q = t.randn(m * nh * hd, device=gpu.dev)
        out = t.empty(m * nh * hd, device=gpu.dev)
        span = max(ring, window if window else pos + rows)
        nb = kernels.attend_scratch_bytes(m, nh, 1, hd, span)
        scratch = t.empty(nb + 256, dtype=t.uint8, device=gpu.dev)
        nbytes = 0
        for r in range(rows):
            en = pos + r + 1
            n = min(en, window) if window else en
            nbytes += n * (2 * hd + 8)
        nbytes *= nseq

        def call(i):
            seqs = [(c[i % copies][0], c[i % copies][1], c[i % copies][2], c[i % copies][3], cap,
                     ring, pos, rows) for c in caches]
            kernels.attend(out, q, seqs, nh, 1, hd, window, scratch=scratch)
        dt = kernel_avg(gpu, call, 8, 3)
        res[name] = {"us": dt * 1e6, "GB_s": nbytes / dt / 1e9, "frac_hbm": nbytes / dt / HBM_PEAK,
                     "kv_bytes": nbytes}
    return {"workload": "attention per layer call, graphs of 8 calls", "per_case": res}


def extra_model(gpu):
    """A .fgm file on the GPU (model.rs, forward.rs:26-158): a synthetic file
    with the cfg2 up / down shapes (int4 g64, Hadamard 128) and an int8 twin
    of up, opened resident (one upload), Gemm::run (FWHT + quantise + pack,
    then the GEMM) through the DualW rule FGM_WEIGHTS=auto:16 at M=8 (int4)
    and M=256 (the int8 twin), against the host-pointer drop-ins on the same
    bytes (per call: activation up, result down; weights cached)."""
    import tempfile
    import numpy as np
    from fastgemma_amd import kernels
    from fastgemma_amd.fgm_format import write_fgm
    from fastgemma_amd.model import Model, Selection, linear_run
    t = gpu.t
    rng = np.random.default_rng(7)
    tensors = []
    for name, n, k, twin in (("up", 8192, 2048, True), ("down", 2048, 8192, False)):
        tensors.append((name, rng.integers(0, 256, n * k // 2, dtype=np.uint8), "q4g", (n, k),
                        {"hadamard": 128, "group": 64}))
        tensors.append((name + ".scale", (rng.random((k // 64) * n) * 0.045 + 0.005).astype(np.float16),
                        "f16", (k // 64, n), None))
        if twin:
            tensors.append((name + ".i8", rng.integers(-127, 128, n * k, dtype=np.int8), "q8c", (n, k),
                            {"hadamard": 128, "group": 0}))
            tensors.append((name + ".i8.scale", (rng.random(n) * 0.009 + 0.001).astype(np.float32), "f32",
                            (n,), None))
    res = {}
    with tempfile.TemporaryDirectory() as d:
        path = d + "/bench.fgm"
        write_fgm(path, {"hidden_size": 2048}, tensors)
        # the first resident open of a process includes one-time runtime set-up
        # (upload stream, pinned staging); the second is the steady upload rate
        opens = []
        for _ in range(2):
            t0 = time.perf_counter()
            m = Model(path, resident=True)
            t.cuda.synchronize()
            opens.append(time.perf_counter() - t0)
            if len(opens) < 2:
                m.close()
        res["open_resident"] = {"s": opens[1], "first_open_s": opens[0], "bytes": m.total_bytes(),
                                "GB_s": m.total_bytes() / opens[1] / 1e9}
        sel = Selection.parse("auto:16")
        for rows in (8, 256):
            w = m.dual("up").pick(rows, sel)
            a = t.randn(rows, w.k, device=gpu.dev)
            out = t.empty(rows, w.n, device=gpu.dev)
            scratch = t.empty(max(kernels.lib().fgm_hip_linear_scratch_bytes(rows, w.k), 1),
                              dtype=t.uint8, device=gpu.dev)
            dt = kernel_avg(gpu, lambda i: linear_run(w, a, rows, w.k, out, scratch), 16, 3)
            wb = w.n * w.k // 2 if w.bits == 4 else w.n * w.k
            res[f"linear_run up M={rows}"] = {"bits": w.bits, "us": dt * 1e6,
                                              "GB_s_weights": wb / dt / 1e9,
                                              "TOPS": 2.0 * rows * w.n * w.k / dt / 1e12}
            # the drop-in path on the same bytes (host activation and result)
            ah = a.cpu().numpy()
            qs = np.empty(rows, np.float32)
            pa = np.empty(kernels.packed_a_len(rows, w.k), np.int8)
            rot = np.empty(rows * w.k, np.float32)
            qa = np.empty(rows * w.k, np.int8)
            c = np.empty(rows * w.n, np.float32)
            blob, scl = np.ascontiguousarray(w.blob()), np.ascontiguousarray(w.scales())

            def dropin():
                kernels.prep_rows(ah.ravel(), w.k, rot, qa, qs, pa, rows, w.k, w.hadamard, 0, rows)
                if w.bits == 4:
                    kernels.gemm_q4g(rows, w.n, w.k, pa, qs, blob, scl, w.group, c, w.n, 0, w.n // 16)
                else:
                    kernels.gemm_q8c(rows, w.n, w.k, pa, qs, blob, scl, c, w.n, 0, w.n // 16)
            dropin()
            reps = 20
            t0 = time.perf_counter()
            for _ in range(reps):
                dropin()
            res[f"dropin up M={rows}"] = {"bits": w.bits, "us": (time.perf_counter() - t0) / reps * 1e6}
        m.close()
    return {"workload": "synthetic .fgm (cfg2 up/down int4 + int8 twin of up), resident vs drop-in",
            "per_case": res}


# ------------------------------------------------------------ CPU baseline
def bench_siblings():
    """PIDs of other bench.py processes (a Python interpreter running this
    script), matched on the executable name and the script argument, not on
    the whole command line (a shell that mentions bench.py is no sibling;
    fgm-bench main.rs:20-43 does the same on /proc/<pid>/comm)."""
    me, out = os.getpid(), []
    try:
        pids = [int(d) for d in os.listdir("/proc") if d.isdigit()]
    except OSError:
        return out
    for pid in pids:
        if pid == me:
            continue
        try:
            comm = open(f"/proc/{pid}/comm").read().strip()
            argv = open(f"/proc/{pid}/cmdline", "rb").read().split(b"\0")
        except OSError:
            continue
        if comm.startswith("python") and any(x.endswith(b"bench.py") for x in argv[1:3]):
            out.append(pid)
    return out


def load_check(nt):
    """The reference's guard against timing on a loaded host (fgm-bench
    main.rs:45-113): another bench running refuses the CPU leg (unless
    FGM_IGNORE_LOAD is set); a one-minute load average above 0.35 x threads
    is reported with the numbers (this host is shared, so it warns rather
    than refuses)."""
    sibs = bench_siblings()
    try:
        la = float(open("/proc/loadavg").read().split()[0])
    except (OSError, ValueError, IndexError):
        la = None
    return {"siblings": sibs, "loadavg_1m": la, "loaded": la is not None and la > 0.35 * nt,
            "refuse": bool(sibs) and not os.environ.get("FGM_IGNORE_LOAD")}


class CpuPath:
    """The reference's own fgm_prep_rows + fgm_gemm_q8c_vnni / _q4g_vnni
    (oracle/_ref, compiled from the reference's C) or, where that is not
    built, the oracle's restatement, driven by the reference's thread split
    (oracle/cpu_pool.c: pool.rs:110-145 for GEMMs, 16-row blocks for prep)."""

    def __init__(self):
        import oracle
        self.o = oracle
        self.L = oracle.lib()
        R = oracle.ref()
        self.kind = "reference" if R is not None else "port"
        self.amx = bool(R is not None and R.fgm_cpu_has_amx())
        self.nt = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
        self.nt = max(1, min(self.nt, 64))
        src = R if R is not None else None
        self.fq4 = C.cast(src.fgm_gemm_q4g_vnni if src else self.L.orc_gemm_q4g, C.c_void_p).value
        self.fq8 = C.cast(src.fgm_gemm_q8c_vnni if src else self.L.orc_gemm_q8c, C.c_void_p).value
        self.fprep = C.cast(src.fgm_prep_rows if src else self.L.orc_prep_rows, C.c_void_p).value
        self.t1 = __import__("numpy").empty(1, "float64")
        self.L.orc_pool_start(self.nt)

    def close(self):
        self.L.orc_pool_stop()

    def act(self, M, K, seed):
        import numpy as np
        x = self.o.gen_normal(seed, M * K).reshape(M, K)
        return dict(x=x, M=M, K=K, rot=np.empty((M, K), np.float32), qa=np.empty((M, K), np.int8),
                    qs=np.empty(M, np.float32), pa=np.empty((M + 15) // 16 * 16 * K, np.int8))

    def prep(self, a):
        P = self.o._ptr
        self.L.orc_pool_prep(self.fprep, P(a["x"]), a["K"], P(a["rot"]), P(a["qa"]), P(a["qs"]), P(a["pa"]),
                             a["M"], a["K"], 0, 1, P(self.t1))

    def gemm(self, bits, a, N, w, s, c, group=64):
        P = self.o._ptr
        if bits == 8:
            self.L.orc_pool_q8c(self.fq8, a["M"], N, a["K"], P(a["pa"]), P(a["qs"]), P(w), P(s), P(c), N, 1,
                                P(self.t1))
        else:
            self.L.orc_pool_q4g(self.fq4, a["M"], N, a["K"], P(a["pa"]), P(a["qs"]), P(w), P(s), group, P(c),
                                N, 1, P(self.t1))


def time_cpu(fn, min_reps=10, min_s=0.3):
    """fn timed after one warm-up call: at least min_reps calls and min_s
    seconds; (median, min, max, reps) in seconds, as fgm-bench main.rs:190-199
    reports them."""
    fn()
    ts, t_end = [], time.perf_counter() + min_s
    while len(ts) < min_reps or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    m, lo, hi = med_range(ts)
    return m, lo, hi, len(ts)


def _rec(t, work, unit):
    """A CPU row: median / min / max in ms and the median's throughput in the
    GPU row's unit (work = bytes for GB/s, ops for TOPS)."""
    m, lo, hi, n = t
    scale = 1e9 if unit == "GB/s" else 1e12
    return {"median_ms": m * 1e3, "min_ms": lo * 1e3, "max_ms": hi * 1e3, "reps": n,
            "value": work / m / scale, "unit": unit}


def cpu_configs(cp):
    """Every BASELINE config on the CPU path, GEMM-only and prep + GEMM (as
    the reference's own kernel bench times them apart), on host-generated
    operands of the GPU rows' shapes; the units and algorithmic work are the
    GPU rows'."""
    import numpy as np
    rng = np.random.default_rng(99)

    def w8(N, K):
        return (np.frombuffer(rng.bytes(N * K), np.int8).copy(),
                (rng.random(N, dtype=np.float32) * 0.009 + 0.001).astype(np.float32))

    def w4(N, K):
        return (np.frombuffer(rng.bytes(N * K // 2), np.uint8).copy(),
                (rng.random((K // 64) * N, dtype=np.float32) * 0.045 + 0.005).astype(np.float16).view(np.uint16))

    out = {}
    # cfg1: int8 GEMV M=1
    a = cp.act(1, 2048, 31)
    W = w8(8192, 2048)
    c = np.empty((1, 8192), np.float32)
    b = gemm_bytes(8, 1, 8192, 2048)
    out["cfg1"] = {"gemm": _rec(time_cpu(lambda: cp.gemm(8, a, 8192, *W, c)), b, "GB/s"),
                   "prep_gemm": _rec(time_cpu(lambda: (cp.prep(a), cp.gemm(8, a, 8192, *W, c))),
                                     b + prep_bytes(1, 2048), "GB/s")}
    # cfg3: the seven M=256 int8 projections, and the layer
    acts = {K: cp.act(256, K, 40 + K) for K in (2048, 8192)}
    r3, lay_g, lay_pg = {}, [], []
    ws = {name: w8(N, K) for name, N, K in LAYER}
    cs = {name: np.empty((256, N), np.float32) for name, N, K in LAYER}
    for name, N, K in LAYER:
        ops = 2.0 * 256 * N * K
        g = _rec(time_cpu(lambda: cp.gemm(8, acts[K], N, *ws[name], cs[name]), 5), ops, "TOPS")
        pg = _rec(time_cpu(lambda: (cp.prep(acts[K]), cp.gemm(8, acts[K], N, *ws[name], cs[name])), 5), ops,
                  "TOPS")
        r3[name] = {"gemm": g, "prep_gemm": pg}

    def layer(with_prep):
        for name, N, K in LAYER:
            if with_prep and name in ("q", "o", "gate", "down"):
                cp.prep(acts[K])
            cp.gemm(8, acts[K], N, *ws[name], cs[name])
    lops = sum(2.0 * 256 * N * K for _, N, K in LAYER)
    r3["layer"] = {"gemm": _rec(time_cpu(lambda: layer(False), 5), lops, "TOPS"),
                   "prep_gemm": _rec(time_cpu(lambda: layer(True), 5), lops, "TOPS")}
    out["cfg3"] = r3
    del ws, cs
    # cfg4: 30 layers (q,k,v,o,gate,up int4 g64, down int8) + int8 LM head,
    # distinct buffers, M=8, the forward pass's GEMM sequence
    layers = [{name: (w8(N, K) if name == "down" else w4(N, K)) for name, N, K in LAYER} for _ in range(30)]
    head = w8(262144, 2048)
    a2, a8 = cp.act(8, 2048, 51), cp.act(8, 8192, 52)
    outs = {name: np.empty((8, N), np.float32) for name, N, K in LAYER}
    logits = np.empty((8, 262144), np.float32)
    shp = {name: (N, K) for name, N, K in LAYER}

    def step(with_prep):
        for L in layers:
            for grp in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",)):
                a = a8 if grp[0] == "down" else a2
                if with_prep:
                    cp.prep(a)
                for name in grp:
                    cp.gemm(8 if name == "down" else 4, a, shp[name][0], *L[name], outs[name])
        if with_prep:
            cp.prep(a2)
        cp.gemm(8, a2, 262144, *head, logits)
    allb = sum(gemm_bytes(8 if name == "down" else 4, 8, N, K) for name, N, K in LAYER) * 30 \
        + gemm_bytes(8, 8, 262144, 2048)
    preps = 30 * (3 * prep_bytes(8, 2048) + prep_bytes(8, 8192)) + prep_bytes(8, 2048)
    out["cfg4"] = {"gemm": _rec(time_cpu(lambda: step(False), 5, 0.2), allb, "GB/s"),
                   "prep_gemm": _rec(time_cpu(lambda: step(True), 5, 0.2), allb + preps, "GB/s")}
    del layers, head
    # cfg5: M=2048 heavy-tailed (gate/up int4 g64, down int8)
    r5 = {}
    x5 = {K: cp.act(2048, K, 60 + K) for K in (2048, 8192)}
    for K, a in x5.items():
        a["x"][:] = (cp.o.gen_student_t(61 + K, 2048 * K, 3)).reshape(2048, K)
    for name, bits, N, K in (("gate", 4, 8192, 2048), ("up", 4, 8192, 2048), ("down", 8, 2048, 8192)):
        W = w4(N, K) if bits == 4 else w8(N, K)
        c = np.empty((2048, N), np.float32)
        ops = 2.0 * 2048 * N * K
        r5[name] = {"bits": bits,
                    "gemm": _rec(time_cpu(lambda: cp.gemm(bits, x5[K], N, *W, c), 5, 0.2), ops, "TOPS"),
                    "prep_gemm": _rec(time_cpu(lambda: (cp.prep(x5[K]), cp.gemm(bits, x5[K], N, *W, c)), 5, 0.2),
                                      ops, "TOPS")}
    out["cfg5"] = r5
    return out


def cpu_baseline(host, budget_s=10.0):
    """The headline's CPU leg (cfg2: prep + q4g up, prep + q4g down, M=8) for
    about budget_s seconds, and every other config (cpu_configs)."""
    import numpy as np
    cp = CpuPath()
    chk = load_check(cp.nt)
    if chk["refuse"]:
        cp.close()
        return {"refused": f"other bench.py processes running: {chk['siblings']} (set FGM_IGNORE_LOAD=1 "
                           "to time anyway)", "load": chk}
    P = cp.o._ptr
    shapes = (("up", 8192, 2048), ("down", 2048, 8192))
    bufs = {}
    for name, N, K in shapes:
        w, s = host[name]
        bufs[name] = dict(a=cp.act(8, K, 5), w=np.ascontiguousarray(w), s=np.ascontiguousarray(s),
                          c=np.empty((8, N), np.float32), N=N)

    def one_step(with_prep=True):
        for name, N, K in shapes:
            b = bufs[name]
            if with_prep:
                cp.prep(b["a"])
            cp.gemm(4, b["a"], N, b["w"], b["s"], b["c"])

    step_bytes = (gemm_bytes(4, 8, 8192, 2048) + gemm_bytes(4, 8, 2048, 8192)
                  + prep_bytes(8, 2048) + prep_bytes(8, 8192))
    t = time_cpu(one_step, 10, budget_s)
    tg = time_cpu(lambda: one_step(False), 10, budget_s / 4)
    per = cpu_configs(cp)
    cp.close()
    after = bench_siblings()
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    phys, smt = cpu_topology()
    gemm_b = gemm_bytes(4, 8, 8192, 2048) + gemm_bytes(4, 8, 2048, 8192)
    return {"value": step_bytes / t[0] / 1e9, "unit": "GB/s", "cores": cp.nt, "kind": cp.kind,
            "physical_cores": phys, "smt_used": smt, "amx": cp.amx,
            "sample": f"{t[3]} cfg2 steps (prep+q4g up, prep+q4g down, M=8) in ~{budget_s:.0f} s: median "
                      f"{t[0] * 1e3:.3f} ms, range {t[1] * 1e3:.3f}-{t[2] * 1e3:.3f} ms; {cp.kind} VNNI kernels, "
                      f"pool.rs N-split over {cp.nt} threads ({phys} cores); '{cpu}'",
            "cfg2": {"prep_gemm": _rec(t, step_bytes, "GB/s"), "gemm": _rec(tg, gemm_b, "GB/s")},
            "per_config": per,
            "load": {**chk, "siblings_after": after, "suspect": bool(after) or chk["loaded"]}}


def cpu_topology():
    """(physical cores, SMT used) among the CPUs this process may run on."""
    cpus = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else []
    cores = set()
    for c in cpus:
        try:
            pkg = open(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id").read().strip()
            core = open(f"/sys/devices/system/cpu/cpu{c}/topology/core_id").read().strip()
            cores.add((pkg, core))
        except OSError:
            cores.add(("?", c))
    return len(cores), len(cores) < len(cpus)


# ------------------------------------------------------------------ main
def read_traffic():
    """HBM bytes per launch of the dominant kernel from the committed PMC
    summary (profiles/decode_q4g_m8_pair_traffic.txt), or None."""
    p = os.path.join(ROOT, "profiles", "decode_q4g_m8_pair_traffic.txt")
    try:
        for line in open(p):
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def host_cfg2_weights():
    """cfg2's up / down int4 weights generated on the host (for --only cpu)."""
    import numpy as np
    rng = np.random.default_rng(5)
    out = {}
    for name, N, K in (("up", 8192, 2048), ("down", 2048, 8192)):
        out[name] = (np.frombuffer(rng.bytes(N * K // 2), np.uint8).copy(),
                     (rng.random((K // 64) * N, dtype=np.float32) * 0.045 + 0.005).astype(np.float16).view(np.uint16))
    return out


def _r(x, nd=3):
    """x to nd significant digits (compact summary)."""
    if x is None:
        return None
    if isinstance(x, (list, tuple)):
        return [_r(v, nd) for v in x]
    return float(f"{x:.{nd}g}")


def summary(out):
    """The figures a reader needs, compact, printed last in the JSON line:
    GPU time (median, and range where measured), the roofline fraction, and
    the CPU row beside it (GPU / CPU speed-up on the same algorithmic work)."""
    ex, cpu = out.get("extra", {}), out.get("cpu_baseline") or {}
    per = cpu.get("per_config", {})
    sm = {"cfg2_step_us": _r(out["ms_per_step"] * 1e3), "cfg2_step_range_us": _r(out.get("step_range_us")),
          "cfg2_frac_hbm": _r(out["config"]["frac_hbm_step"]),
          "pair_launch_us": _r(out["roofline"]["us_per_launch"]), "pair_frac_hbm": _r(out["roofline"]["frac"])}
    if cpu.get("cfg2"):
        sm["cfg2_cpu_ms"] = _r(cpu["cfg2"]["prep_gemm"]["median_ms"])
    c1 = ex.get("cfg1", {})
    if "us_per_launch" in c1:
        sm["cfg1"] = {"us": _r(c1["us_per_launch"]), "frac_hbm": _r(c1["frac_hbm"])}
        if "cfg1" in per:
            sm["cfg1"]["cpu_ms"] = _r(per["cfg1"]["gemm"]["median_ms"])
    s4 = ex.get("int4_stream", {})
    if "us_per_launch" in s4:
        sm["int4_134MB"] = {"us": _r(s4["us_per_launch"]), "frac_hbm": _r(s4["frac_hbm"])}
    c3 = ex.get("cfg3", {})
    if "per_shape" in c3:
        sm["cfg3_us"] = {k: _r(v["us"]) for k, v in c3["per_shape"].items()}
        lb = c3["layer_batched"]
        sm["cfg3_layer"] = {"us": _r(lb["us"]), "range": _r(lb.get("us_range")), "frac_mfma": _r(lb["frac_mfma"]),
                            "us_one_copy": _r(lb.get("us_one_copy"))}
        if "cfg3" in per:
            sm["cfg3_layer"]["cpu_ms"] = _r(per["cfg3"]["layer"]["gemm"]["median_ms"])
    c4 = ex.get("cfg4", {})
    if "us_per_step" in c4:
        sm["cfg4"] = {"us": _r(c4["us_per_step"]), "frac_hbm": _r(c4["frac_hbm"]), "tok_s": _r(c4["tokens_per_s"])}
        if "gemm_only" in c4:
            sm["cfg4"]["gemm_only_us"] = _r(c4["gemm_only"]["us_per_step"])
        if "cfg4" in per:
            sm["cfg4"]["cpu_ms"] = _r(per["cfg4"]["prep_gemm"]["median_ms"])
            sm["cfg4"]["cpu_gemm_only_ms"] = _r(per["cfg4"]["gemm"]["median_ms"])
    c5 = ex.get("cfg5", {})
    if "per_shape" in c5:
        sm["cfg5"] = {k: {"us": _r(v["us"]), "frac_mfma": _r(v["frac_mfma"])} for k, v in c5["per_shape"].items()}
        for k in sm["cfg5"]:
            if k in per.get("cfg5", {}):
                sm["cfg5"][k]["cpu_ms"] = _r(per["cfg5"][k]["gemm"]["median_ms"])
    sw = ex.get("sweep", {})
    if "dense_from_M" in sw:
        sm["sweep"] = {"dense_from_M": sw["dense_from_M"].get("q8c"), "int8_not_slower_from_M": sw["int8_not_slower_from_M"]}
    if cpu:
        sm["cpu"] = {"kind": cpu.get("kind"), "cores": cpu.get("cores"), "suspect": cpu.get("load", {}).get("suspect")}
    return sm


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=480)
    ap.add_argument("--warmup", type=int, default=48)
    ap.add_argument("--reps", type=int, default=7, help="timed replays of the K-step graph (median reported)")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only", default=None,
                    help="run one extra measurement (ceilings, cfg1, int4_stream, cfg3, vendor, sweep, cfg5, cfg4, "
                         "elem, prep_fused, attn, model, cpu) and print its JSON instead of the headline line")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the weight stream would shard along N, one slice per GPU); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    if args.only == "cpu":
        print(json.dumps({"cpu": cpu_baseline(host_cfg2_weights(), args.cpu_seconds)}))
        return
    gpu = Gpu()
    gpu.t.manual_seed(1234)
    # the ceilings go last: their large rotating buffers must not disturb the
    # other measurements' allocations
    extras = {"cfg1": extra_cfg1, "int4_stream": extra_int4_stream,
              "cfg3": extra_cfg3, "vendor": extra_vendor, "sweep": extra_sweep,
              "cfg5": extra_cfg5, "cfg4": extra_cfg4, "elem": extra_elem,
              "prep_fused": extra_prep_fused, "attn": extra_attn,
              "model": extra_model, "ceilings": extra_ceilings}
    if args.only is not None:
        if args.only not in extras:
            print(f"--only: unknown measurement {args.only!r} (one of {', '.join(extras)}, cpu)",
                  file=sys.stderr)
            sys.exit(2)
        print(json.dumps({args.only: extras[args.only](gpu)}))
        return
    log("setting up cfg2 (48 weight copies)")
    step, gemv_pair, gemv_up, gemv_down, step_bytes, host = cfg2_setup(gpu)

    warm = gpu.graphs(step, max(16, args.warmup), 16)
    gpu.time_graphs(warm)
    # all `steps` steps in one graph; each timed replay is exactly `steps`
    # steps, synchronized on both sides; the median replay is reported
    gs = gpu.graphs(step, args.steps, args.steps)
    log(f"timing {args.steps} steps in one graph, {args.reps} replays")
    dt, dlo, dhi = med_range(gpu.time_each(gs, max(5, args.reps)))
    ms_per_step = dt / args.steps * 1e3
    value = step_bytes * args.steps / dt / 1e9
    del gs, warm

    log("dominant kernel timing")
    pair_s, pair_lo, pair_hi = kernel_time(gpu, gemv_pair)
    up_s = kernel_avg(gpu, gemv_up)
    down_s = kernel_avg(gpu, gemv_down)
    up_b = gemm_bytes(4, 8, 8192, 2048)
    down_b = gemm_bytes(4, 8, 2048, 8192)
    pair_b = up_b + down_b
    roof = {"bound": "hbm", "achieved": pair_b / pair_s / 1e9, "peak": HBM_PEAK / 1e9,
            "unit": "GB/s", "frac": pair_b / pair_s / HBM_PEAK, "traffic": read_traffic(),
            "kernel": "decode_kernel (int4, M <= 8 variant): the step's GEMM launch, "
                      "up N=8192 K=2048 and down N=2048 K=8192 in one launch, M=8",
            "algorithmic_bytes_per_launch": pair_b, "us_per_launch": pair_s * 1e6,
            "us_range": [pair_lo * 1e6, pair_hi * 1e6],
            "timing": "HIP events around a graph of 48 back-to-back launches / 48, median of 5 replays",
            "single_shape_launches": {
                "up": {"us": up_s * 1e6, "GB_s": up_b / up_s / 1e9, "frac": up_b / up_s / HBM_PEAK},
                "down": {"us": down_s * 1e6, "GB_s": down_b / down_s / 1e9,
                         "frac": down_b / down_s / HBM_PEAK}}}

    extra = {}
    if not args.no_extra:
        for name, fn in extras.items():
            log("extra", name)
            try:
                extra[name] = fn(gpu)
            except Exception as e:  # report, keep the headline line
                extra[name] = {"error": repr(e)}
            gpu.t.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        try:
            cpu = cpu_baseline(host, args.cpu_seconds)
        except Exception as e:
            cpu = {"error": repr(e)}

    out = {
        "metric": "decode GEMV HBM GB/s (M=8 int4 g64, up+down, incl. quantise+pack)",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (device-generated: N(0,1) activations, uniform int4/int8 weights, "
                "uniform scales; 48 rotating weight copies)",
        "config": {"workload": "BASELINE configs[1]: batched decode skinny GEMM M=8, int4 g64, "
                               "up N=8192 K=2048 + down N=2048 K=8192",
                   "global_batch": 8, "algorithmic_bytes_per_step": step_bytes,
                   "frac_hbm_step": value * 1e9 / HBM_PEAK},
        "timing": f"one graph of {args.steps} steps, median of {max(5, args.reps)} timed replays",
        "step_range_us": [dlo / args.steps * 1e6, dhi / args.steps * 1e6],
        "roofline": roof,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    out["summary"] = summary(out)
    log("done")
    print(json.dumps(out))


if __name__ == "__main__":
    main()
