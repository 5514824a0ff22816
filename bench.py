"""Benchmark of the MI355X linear hot path of MingTTS.

Headline step: one decode step of the backbone linears -- 24 Qwen2-0.5B layers x {qkv
1152x896 + bias, o 896x896 (+= residual), gate|up 2 x 4864x896 with SiLU*mul, down
896x4864 (+= residual)} at M = 2 rows (the CFG cond/uncond pair), fp16 weights ~
N(0, 0.02^2), fp32 activations ~ N(0, 1), run as ONE persistent launch of the linear
sequence (96 dependent linears).  ``value`` is the step's achieved HBM rate in GB/s
(algorithmic bytes / step time), inputs resident in HBM.

Also measured in the same run (extra keys of the JSON line), every figure a HIP-graph
replay timed with HIP events on its stream (host launch cost excluded): the empty-dispatch
floor, the single GEMV (4864 x 896, fp16, from a rotated >= 1 GiB weight pool), the same
decode step as 96 separate launches, the prefill GEMM stack at M = 64 / 256 / 512 (MFMA
TFLOPS), batch-2 decode attention over fp16 caches, the DiT head MLP warm and cold, the flow
stage and the VAE latent; and the CPU baseline (the oracle's vectorised restatement of the
reference CPU loop over the whole step, on every host thread and on one).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--only decode]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ming-tts_amd"))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
H, QKV, INTER, LAYERS = 896, 1152, 4864, 24
METRIC = "decode-step linear µs + achieved HBM GB/s (% of 8 TB/s); prefill MFMA TFLOPS"


PROFILE = os.path.join(ROOT, "profiles", "layer_kernel_decode_24L_M2.md")


def measured_traffic(path: str = PROFILE):
    """HBM bytes per launch of the decode kernel from its committed rocprofv3 counter summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled against a 1 GiB copy): the line
    ``traffic_per_launch_bytes: N``.  None when the summary is absent."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_per_launch_bytes:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def ensure_built() -> None:
    import mingtts
    if not os.path.exists(mingtts.LIB_PATH):
        log("library not built; building")
        import __graft_entry__
        __graft_entry__.build()


class Events:
    """HIP events on torch's current stream (the stream every launch below uses), or on
    `stream`."""

    def __init__(self, torch, stream=None):
        self.torch = torch
        self.stream = stream
        self.a = torch.cuda.Event(enable_timing=True)
        self.b = torch.cuda.Event(enable_timing=True)

    def start(self):
        self.a.record(self.stream)

    def stop_ms(self) -> float:
        self.b.record(self.stream)
        self.b.synchronize()
        return self.a.elapsed_time(self.b)


def graph_us(torch, fn, stream, rounds=5) -> float:
    """Median time (us) of one replay of a HIP graph holding fn()'s launches, each replay
    bracketed by HIP events on the replay stream (the stream the launches were captured on),
    so host launch cost is outside every figure.  fn runs once eagerly first: the split-K
    workspace may not grow under capture."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        fn()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=stream):
            fn()
    torch.cuda.synchronize()
    times = []
    with torch.cuda.stream(stream):
        g.replay()
        torch.cuda.synchronize()
        for _ in range(rounds):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            g.replay()
            b.record()
            b.synchronize()
            times.append(a.elapsed_time(b))
    del g
    return 1e3 * sorted(times)[len(times) // 2]


def bench_launch_floor(torch, dev, n=200):
    """The empty-dispatch floor, as the reference's GemvBench measures it (one-element copies
    back to back, GemvBench.swift:117-123): n one-element device kernels in one graph."""
    a = torch.zeros(1, device=dev)
    b = torch.zeros(1, device=dev)
    cs = torch.cuda.Stream(device=dev)

    def run():
        for _ in range(n):
            b.add_(a)

    return dict(us_per_dispatch=graph_us(torch, run, cs) / n, dispatches=n,
                kernel="one-element elementwise add (torch), graph replay")


def make_layers(torch, dev, layers=LAYERS, seed=0):
    """Distinct per-layer fp16 weights ~ N(0, 0.02^2): 715.6 MB for 24 layers (> the 256 MB
    Infinity Cache, so every step streams from HBM).  Synthetic, generated on the device."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def w(*shape):
        return (torch.randn(*shape, generator=g, device=dev, dtype=torch.float32) * 0.02).half()

    def gain(n):
        return (1.0 + 0.1 * torch.randn(n, generator=g, device=dev, dtype=torch.float32)).half()

    return [dict(qkv=w(QKV, H), qkv_b=w(QKV), o=w(H, H), gate=w(INTER, H), up=w(INTER, H), down=w(H, INTER),
                 norm1=gain(H), norm2=gain(H)) for _ in range(layers)]


def decode_ops(mt, ws, M, resid, qkv, mlp):
    """One layer's linears (Qwen.swift:84-91) with the two RMSNorms fused into qkv and gate|up;
    the attention output is stood in for by the q part of qkv (attention is timed apart)."""
    ops = []
    for p in ws:
        ops.append(mt.op(resid, p["qkv"], qkv, M, bias=p["qkv_b"], norm=p["norm1"]))
        ops.append(mt.op(qkv, p["o"], resid, M, flags=mt.GemvFlags.accumulate, ldx=QKV))
        ops.append(mt.op(resid, p["gate"], mlp, M, flags=mt.GemvFlags.siluGate, w2=p["up"], norm=p["norm2"]))
        ops.append(mt.op(mlp, p["down"], resid, M, flags=mt.GemvFlags.accumulate))
    return ops


def shape_bytes(M, N, K, f, xsize=4) -> int:
    """Algorithmic bytes of one linear: 16-bit weights (x2 gated) + bias + x read + fp32 y
    write (+ y read when accumulating)."""
    wb = 2 * N * K * (2 if f & 8 else 1) + (2 * N if f & 1 else 0)
    return wb + xsize * M * K + 4 * M * N * (2 if f & 2 else 1)


def op_bytes(o, xsize=4) -> int:
    """shape_bytes plus the RMSNorm gain ([K] fp16) when the op has one."""
    return shape_bytes(o.p.M, o.p.N, o.p.K, o.p.flags, xsize) + (2 * o.p.K if o.norm else 0)


def op_flops(o) -> int:
    return 2 * o.p.M * o.p.N * o.p.K * (2 if o.p.flags & 8 else 1)


def bench_decode_seq(torch, mt, dev, ws, steps, warmup, M=2):
    """Each step resets the residual (a device copy outside the timed bracket), then runs the
    sequence between two HIP events on the launch stream.  All steps are queued without host
    synchronisation, so each bracket holds the kernel and its dispatch only."""
    resid = torch.randn(M, H, device=dev)
    qkv = torch.zeros(M, QKV, device=dev)
    mlp = torch.zeros(M, INTER, device=dev)
    x0 = resid.clone()
    ops = decode_ops(mt, ws, M, resid, qkv, mlp)
    seq = mt.Seq(ops)
    for _ in range(warmup):
        resid.copy_(x0)
        seq.run()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in ev:
        resid.copy_(x0)
        a.record()
        seq.run()
        b.record()
    torch.cuda.synchronize()
    times = [a.elapsed_time(b) for a, b in ev]
    seq.check()
    nbytes = sum(op_bytes(o) for o in ops)
    flops = sum(op_flops(o) for o in ops)
    res = dict(groups=seq.groups, bytes=nbytes, flops=flops, times_ms=times, ops=len(ops),
               kernel=("mt::layer_kernel<1, 2, false> (fp16 weights, M = 2, the Qwen2-0.5B decode-layer kernel)"
                       if seq.kernel == mt.SEQ_DECODE_LAYER else
                       "mt::seq_kernel<1, 2, false> (fp16 weights, M = 2, linears only)")
               + "; one launch per decode step")
    seq.close()
    return res


def bench_decode_layers(torch, mt, dev, ws, steps, warmup, M=2, cap=512):
    """The whole decode layer (Qwen.swift:84-91) in one persistent launch: per layer the four
    linears plus a decode attention item (RoPE, K/V append at the row's position, GQA over
    the row's fp16 cache of 512 slots, 14 q / 2 kv heads), 120 items per step.  Positions are
    the batch-2 attention workload's (lengths ~ U[32, 512], seed 0).  Timed as the linear
    step is (HIP events around each launch)."""
    import numpy as np
    HQ, HKV = 14, 2
    lens = np.random.default_rng(0).integers(32, 513, M).astype(np.int32)
    pos = torch.from_numpy(lens - 1).to(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    caches = [(torch.randn(M, HKV, cap, 64, generator=g, device=dev).half(),
               torch.randn(M, HKV, cap, 64, generator=g, device=dev).half()) for _ in ws]
    i = torch.arange(32, device=dev, dtype=torch.float32)
    inv_freq = (1.0 / torch.pow(torch.tensor(1e6, device=dev), 2.0 * i / 64.0)).float()
    resid = torch.randn(M, H, device=dev)
    qkv = torch.zeros(M, QKV, device=dev)
    att = torch.zeros(M, HQ * 64, device=dev)
    mlp = torch.zeros(M, INTER, device=dev)
    x0 = resid.clone()
    items = []
    for p, (kc, vc) in zip(ws, caches):
        items.append(mt.op(resid, p["qkv"], qkv, M, bias=p["qkv_b"], norm=p["norm1"]))
        items.append(mt.attn_op(qkv, M, HQ, HKV, pos, kc, vc, cap, HKV * cap * 64, inv_freq, att))
        items.append(mt.op(att, p["o"], resid, M, flags=mt.GemvFlags.accumulate))
        items.append(mt.op(resid, p["gate"], mlp, M, flags=mt.GemvFlags.siluGate, w2=p["up"], norm=p["norm2"]))
        items.append(mt.op(mlp, p["down"], resid, M, flags=mt.GemvFlags.accumulate))
    seq = mt.Seq(items)
    for _ in range(warmup):
        resid.copy_(x0)
        seq.run()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in ev:
        resid.copy_(x0)
        a.record()
        seq.run()
        b.record()
    torch.cuda.synchronize()
    t = sorted(a.elapsed_time(b) for a, b in ev)
    seq.check()
    seq.close()
    kv_bytes = len(ws) * sum(2 * HKV * int(n) * 64 * 2 for n in lens)
    return dict(us=1e3 * sum(t) / len(t), us_median=1e3 * t[len(t) // 2], items=len(items),
                positions=[int(n) - 1 for n in lens], kv_cache_bytes_read=kv_bytes)


def bench_decode_per_op(torch, mt, dev, ws, rounds=5, M=2):
    """The same decode step as 96 separate mt_linear / mt_linear_rmsnorm launches, captured in
    a HIP graph and replayed (the reference encodes them serially into one command buffer)."""
    resid = torch.randn(M, H, device=dev)
    qkv = torch.zeros(M, QKV, device=dev)
    mlp = torch.zeros(M, INTER, device=dev)
    ops = decode_ops(mt, ws, M, resid, qkv, mlp)
    L = mt.load()
    cs = torch.cuda.Stream(device=dev)
    s = cs.cuda_stream

    def step():
        for o in ops:
            if o.norm:
                rc = L.mt_linear_rmsnorm(o.x, o.xt, o.norm, o.w, o.w2, o.wt, o.bias, o.y, o.p, s)
            else:
                rc = L.mt_linear(o.x, o.xt, o.w, o.w2, o.wt, o.bias, o.y, o.p, s)
            if rc:
                raise RuntimeError(mt.last_error())

    return dict(us=graph_us(torch, step, cs, rounds), launches=len(ops))


def bench_gemv_single(torch, mt, dev, M=1, rounds=5):
    """4864 x 896 fp16 GEMV, x fp16: one graph of back-to-back dispatches, each reading the
    next slice of a >= 1 GiB weight pool (so no dispatch finds its weights in the 256 MB
    Infinity Cache), the reference's rotating-pool method (GemvBench.swift:96-98, 126-131)."""
    N, K = 4864, 896
    per = N * K
    copies = (1 << 30) // (per * 2) + 1
    pool = (torch.randn(copies, N, K, device=dev) * 0.02).half()
    x = torch.randn(M, K, device=dev).half()
    y = torch.zeros(M, N, device=dev)
    L = mt.load()
    cs = torch.cuda.Stream(device=dev)
    p = mt.GemvParams(M, N, K, K, N, 0, 0.0)

    def run():
        for i in range(copies):
            rc = L.mt_linear(x.data_ptr(), mt.F16, pool[i].data_ptr(), None, mt.F16, None, y.data_ptr(), p,
                             cs.cuda_stream)
            if rc:
                raise RuntimeError(mt.last_error())

    us = graph_us(torch, run, cs, rounds) / copies
    nbytes = 2 * N * K + 2 * M * K + 4 * M * N
    del pool
    gbs = nbytes / (us * 1e-6) / 1e9
    return dict(M=M, us_per_dispatch=us, gbs=gbs, pct_of_hbm_peak=100 * gbs / HBM_PEAK_GBS, bytes=nbytes,
                pool_copies=copies, timing="graph replay of one dispatch per pool slice")


# The decode-time linear shapes the reference's GEMV bench times (GemvBench.swift:18-36):
# (label, M, N, K, flags, gated).
GEMV_BENCH_SHAPES = [
    ("llm qkv", 1, 1152, 896, 0, False), ("llm o", 1, 896, 896, 2, False), ("llm gate|up", 1, 4864, 896, 8, True),
    ("llm down", 1, 896, 4864, 2, False), ("agg qkv", 2, 3072, 1024, 0, False), ("agg out", 2, 1024, 1024, 2, False),
    ("agg ff1", 2, 4096, 1024, 4, False), ("agg ff2", 2, 1024, 4096, 2, False), ("vae qkv", 4, 1152, 896, 0, False),
    ("vae o", 4, 896, 896, 2, False), ("vae gate|up", 4, 4864, 896, 8, True), ("vae down", 4, 896, 4864, 2, False),
    ("vae head", 4, 3530, 896, 0, False), ("flow qkv", 6, 3072, 1024, 0, False), ("flow out", 6, 1024, 1024, 2, False),
    ("flow ff1", 6, 4096, 1024, 4, False), ("flow ff2", 6, 1024, 4096, 2, False),
]


def bench_gemv_shapes(torch, mt, dev, rounds=3):
    """The reference's GEMV bench (GemvBench.swift:18-36, 96-157) on MI355X: each decode-time
    linear shape as a graph of back-to-back dispatches, each reading the next slice of a
    >= 1 GiB fp16 weight pool (no cache level serves a weight twice), fp32 x and y as the
    reference's activations; per shape the median replay / dispatches."""
    L = mt.load()
    cs = torch.cuda.Stream(device=dev)
    out = []
    for label, M, N, K, flags, gated in GEMV_BENCH_SHAPES:
        per = N * K * (2 if gated else 1)
        copies = (1 << 30) // (per * 2) + 1
        pool = torch.empty(copies, per, device=dev, dtype=torch.float16)
        pool.normal_(0.0, 0.02)
        x = torch.randn(M, K, device=dev)
        y = torch.zeros(M, N, device=dev)
        p = mt.GemvParams(M, N, K, K, N, flags, 0.0)

        def run():
            for i in range(copies):
                w = pool[i].data_ptr()
                rc = L.mt_linear(x.data_ptr(), mt.F32, w, w + N * K * 2 if gated else None, mt.F16, None,
                                 y.data_ptr(), p, cs.cuda_stream)
                if rc:
                    raise RuntimeError(mt.last_error())

        us = graph_us(torch, run, cs, rounds) / copies
        nbytes = shape_bytes(M, N, K, flags)
        gbs = nbytes / (us * 1e-6) / 1e9
        out.append(dict(shape=label, M=M, N=N, K=K, us_per_dispatch=us, gbs=gbs,
                        pct_of_hbm_peak=100 * gbs / HBM_PEAK_GBS, family=int(mt.linear_kernel(M, N, K, mt.F32, mt.F16))))
        del pool
    torch.cuda.synchronize()
    return out


def bench_prefill_parts(torch, mt, dev, ws, M=174, cap=512, reps=3):
    """The reference's prefill bench (QwenBench.swift:114-129): the prompt's M = 174 rows through
    the 24 layers with the reference's types (fp32 activations, fp16 weights), as the whole
    layer sequence (rmsnorm + qkv, rope_cache, causal attention from position 0, o +=,
    rmsnorm + gate|up, down +=: 144 launches) and each part alone over the 24 layers' weights,
    every figure a HIP-graph replay."""
    HQ, HKV = 14, 2
    resid = torch.randn(M, H, device=dev)
    qkv = torch.zeros(M, QKV, device=dev)
    att = torch.zeros(M, HQ * 64, device=dev)
    mlp = torch.zeros(M, INTER, device=dev)
    caches = [(torch.zeros(HKV, cap, 64, device=dev).half(), torch.zeros(HKV, cap, 64, device=dev).half()) for _ in ws]
    i = torch.arange(32, device=dev, dtype=torch.float32)
    invf = (1.0 / torch.pow(torch.tensor(1e6, device=dev), 2.0 * i / 64.0)).float()
    cs = torch.cuda.Stream(device=dev)
    F = mt.GemvFlags

    def qkv_part(p, s):
        mt.linear(resid, p["qkv"], qkv, M, bias=p["qkv_b"], norm=p["norm1"], stream=s)

    def rope_part(c, s):
        mt.rope_cache(qkv, QKV, M, HQ, HKV, 0, c[0], c[1], cap, invf, stream=s)

    def attn_part(c, s):
        mt.attention(qkv, QKV, M, HQ, HKV, 0, 0, c[0], c[1], cap, att, HQ * 64, stream=s)

    def o_part(p, s):
        mt.linear(att, p["o"], resid, M, flags=F.accumulate, stream=s)

    def gu_part(p, s):
        mt.linear(resid, p["gate"], mlp, M, flags=F.siluGate, w2=p["up"], norm=p["norm2"], stream=s)

    def down_part(p, s):
        mt.linear(mlp, p["down"], resid, M, flags=F.accumulate, stream=s)

    def layers(parts):
        def run():
            s = cs.cuda_stream
            for p, c in zip(ws, caches):
                for name, fn in parts:
                    fn(c if name in ("rope_cache", "attention") else p, s)
        return run

    seq_parts = [("rmsnorm+qkv", qkv_part), ("rope_cache", rope_part), ("attention", attn_part), ("o+res", o_part),
                 ("rmsnorm+gate|up", gu_part), ("down+res", down_part)]
    whole = graph_us(torch, layers(seq_parts), cs, rounds=reps)
    parts = {}
    for name, fn in seq_parts:
        us = graph_us(torch, layers([(name, fn)]), cs, rounds=reps)
        parts[name] = dict(us_per_dispatch=us / len(ws), us_per_step=us)
    lin = {"rmsnorm+qkv": (QKV, H, 1), "o+res": (H, H, 1), "rmsnorm+gate|up": (INTER, H, 2), "down+res": (H, INTER, 1)}
    flops = sum(2 * M * n * k * g for n, k, g in lin.values()) * len(ws)
    return dict(M=M, layer_sequence_us=whole, launches=6 * len(ws), parts=parts,
                linear_tflops=flops / (sum(parts[k]["us_per_step"] for k in lin) * 1e-6) / 1e12,
                activations="fp32 (the reference's), fp16 weights, fp16 K/V cache")


def bench_prefill(torch, mt, dev, ws, M, reps=3):
    """The 24-layer backbone GEMMs at M rows, fp16 activations, fp32 outputs: 96 launches,
    captured in a HIP graph and replayed, as the reference encodes them into one command
    buffer (so host launch cost is excluded)."""
    x = torch.randn(M, H, device=dev).half()
    xi = torch.randn(M, INTER, device=dev).half()
    yq = torch.zeros(M, QKV, device=dev)
    yh = torch.zeros(M, H, device=dev)
    ym = torch.zeros(M, INTER, device=dev)
    ops = []
    for p in ws:
        ops.append(mt.op(x, p["qkv"], yq, M, bias=p["qkv_b"]))
        ops.append(mt.op(x, p["o"], yh, M, flags=mt.GemvFlags.accumulate))
        ops.append(mt.op(x, p["gate"], ym, M, flags=mt.GemvFlags.siluGate, w2=p["up"]))
        ops.append(mt.op(xi, p["down"], yh, M, flags=mt.GemvFlags.accumulate))
    L = mt.load()
    cs = torch.cuda.Stream(device=dev)

    def stack():
        for o in ops:
            rc = L.mt_linear(o.x, o.xt, o.w, o.w2, o.wt, o.bias, o.y, o.p, cs.cuda_stream)
            if rc:
                raise RuntimeError(mt.last_error())

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cs):
        stack()  # eager run first: split-K workspace growth is refused under capture
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=cs):
            stack()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    ev = Events(torch)
    best = None
    for _ in range(reps):
        ev.start()
        graph.replay()
        ms = ev.stop_ms()
        best = ms if best is None else min(best, ms)
    del graph
    flops = sum(op_flops(o) for o in ops)
    nbytes = sum(op_bytes(o, xsize=2) for o in ops)
    tflops = flops / (best * 1e-3) / 1e12
    attainable = min(MFMA_F16_PEAK_TFLOPS, flops / nbytes * HBM_PEAK_GBS / 1e3)
    return dict(M=M, us=best * 1e3, tflops=tflops, pct_mfma_peak=100 * tflops / MFMA_F16_PEAK_TFLOPS,
                pct_attainable=100 * tflops / attainable, gflop=flops / 1e9, mbytes=nbytes / 1e6)


def bench_prefill_chain(torch, mt, dev, ws, M, reps=3):
    """The prefill chain with the reference's activation types (QwenForward.dispatches at M
    prompt rows, Qwen.swift:84-91, its linears): fp32 residual and activations, RMSNorm fused
    into qkv and gate|up, o reading the q part of qkv in place of the attention output, each
    op consuming the previous op's fp32 output (x split into hi + lo halves of the weights'
    type on the MFMA GEMM): 96 dependent launches captured in a HIP graph and replayed."""
    resid = torch.randn(M, H, device=dev)
    qkv = torch.zeros(M, QKV, device=dev)
    mlp = torch.zeros(M, INTER, device=dev)
    ops = decode_ops(mt, ws, M, resid, qkv, mlp)
    L = mt.load()
    cs = torch.cuda.Stream(device=dev)

    def stack():
        s = cs.cuda_stream
        for o in ops:
            if o.norm:
                rc = L.mt_linear_rmsnorm(o.x, o.xt, o.norm, o.w, o.w2, o.wt, o.bias, o.y, o.p, s)
            else:
                rc = L.mt_linear(o.x, o.xt, o.w, o.w2, o.wt, o.bias, o.y, o.p, s)
            if rc:
                raise RuntimeError(mt.last_error())

    us = graph_us(torch, stack, cs, rounds=reps)
    flops = sum(op_flops(o) for o in ops)
    tflops = flops / (us * 1e-6) / 1e12
    return dict(M=M, us=us, tflops=tflops, pct_mfma_peak=100 * tflops / MFMA_F16_PEAK_TFLOPS, gflop=flops / 1e9,
                activations="fp32 (hi + lo halves on the MFMA: 2 MFMAs per product)", norms="fused")


def bench_attention(torch, mt, dev, reps=200):
    """Batch-2 decode attention, 14 q / 2 kv heads, d 64, fp16 caches of 512, lengths ~ U[32, 512]:
    reps dispatches in one graph (the caches stay cache-resident, as the reference's layer loop
    finds them after the RoPE append)."""
    import numpy as np
    B, HQ, HKV, CAP = 2, 14, 2, 512
    lens = np.random.default_rng(0).integers(32, 513, B).astype(np.int32)
    kc = torch.randn(B, HKV, CAP, 64, device=dev).half()
    vc = torch.randn(B, HKV, CAP, 64, device=dev).half()
    q = torch.randn(B, HQ * 64, device=dev)
    out = torch.zeros(B, HQ * 64, device=dev)
    lens_d = torch.from_numpy(lens).to(dev)
    stride = HKV * CAP * 64
    cs = torch.cuda.Stream(device=dev)

    def run():
        for _ in range(reps):
            mt.attention_decode(q, HQ * 64, B, HQ, HKV, lens_d, 0, kc, vc, CAP, stride, out, HQ * 64,
                                stream=cs.cuda_stream)

    us = graph_us(torch, run, cs) / reps
    nbytes = int(sum(2 * HKV * int(l) * 64 * 2 for l in lens)) + 2 * B * HQ * 64 * 4
    return dict(us_per_dispatch=us, gbs=nbytes / (us * 1e-6) / 1e9, lens=lens.tolist(), bytes=nbytes)


def bench_dit(torch, mt, dev, cold=False, rounds=5):
    """DiT head MLP (896 -> 3584 GELU -> 896, += residual) at M = 64 and adaLN 896 -> 5376 at
    M = 2, 8 blocks x 10 ODE steps = 240 launches in one graph.  Warm: the 8 blocks' weights
    repeat across the steps (Infinity-Cache resident after the first).  Cold: every step has
    its own copy of the 8 blocks (1.8 GB in all, well past the 256 MB Infinity Cache), so
    each launch streams its weights from HBM, as the rotating pool does."""
    g = torch.Generator(device=dev)
    g.manual_seed(5)

    def blockset():
        return [dict(ff1=(torch.randn(3584, H, generator=g, device=dev) * 0.02).half(),
                     ff1_b=(torch.randn(3584, generator=g, device=dev) * 0.02).half(),
                     ff2=(torch.randn(H, 3584, generator=g, device=dev) * 0.02).half(),
                     ff2_b=(torch.randn(H, generator=g, device=dev) * 0.02).half(),
                     ada=(torch.randn(6 * H, H, generator=g, device=dev) * 0.02).half(),
                     ada_b=(torch.randn(6 * H, generator=g, device=dev) * 0.02).half()) for _ in range(8)]

    sets = [blockset() for _ in range(10 if cold else 1)]
    x = torch.randn(64, H, device=dev).half()
    hmid = torch.randn(64, 3584, device=dev).half()
    t = torch.randn(2, H, device=dev).half()
    y1 = torch.zeros(64, 3584, device=dev)
    y2 = torch.zeros(64, H, device=dev)
    ya = torch.zeros(2, 6 * H, device=dev)
    ops = []
    for k in range(10):
        for b in sets[k % len(sets)]:
            ops.append(mt.op(t, b["ada"], ya, 2, bias=b["ada_b"]))
            ops.append(mt.op(x, b["ff1"], y1, 64, flags=mt.GemvFlags.gelu, bias=b["ff1_b"]))
            ops.append(mt.op(hmid, b["ff2"], y2, 64, flags=mt.GemvFlags.accumulate, bias=b["ff2_b"]))
    L = mt.load()
    cs = torch.cuda.Stream(device=dev)

    def run():
        for o in ops:
            rc = L.mt_linear(o.x, o.xt, o.w, o.w2, o.wt, o.bias, o.y, o.p, cs.cuda_stream)
            if rc:
                raise RuntimeError(mt.last_error())

    us = graph_us(torch, run, cs, rounds)
    flops = sum(op_flops(o) for o in ops)
    nbytes = sum(op_bytes(o, xsize=2) for o in ops)
    res = dict(us_10_steps=us, us_per_launch=us / len(ops), tflops=flops / (us * 1e-6) / 1e12,
               gbs_algorithmic=nbytes / (us * 1e-6) / 1e9, launches=len(ops),
               weights="cold (10 distinct block sets)" if cold else "warm (one block set, cache resident)")
    del sets
    return res


def bench_gemm_ops(torch, mt, dev, ws, reps=5):
    """Each prefill linear alone, 24 launches over the 24 layers' distinct weights, captured in
    a HIP graph and replayed (so host launch cost is excluded): this library's mt_linear next to
    hipBLASLt (torch.matmul, fp16 out, gate and up concatenated into one 9728-row weight) on the
    same shapes.  Returns µs per launch."""
    L = mt.load()
    gu = [torch.cat([p["gate"], p["up"]], 0).contiguous() for p in ws]
    rows = []
    for M in (64, 256, 512):
        x = torch.randn(M, H, device=dev).half()
        xi = torch.randn(M, INTER, device=dev).half()
        kinds = [("qkv", x, [p["qkv"] for p in ws], None, QKV, 0, [p["qkv"] for p in ws]),
                 ("o", x, [p["o"] for p in ws], None, H, mt.GemvFlags.accumulate, [p["o"] for p in ws]),
                 ("gate|up", x, [p["gate"] for p in ws], [p["up"] for p in ws], INTER, mt.GemvFlags.siluGate, gu),
                 ("down", xi, [p["down"] for p in ws], None, H, mt.GemvFlags.accumulate, [p["down"] for p in ws])]
        for name, xx, wl, w2l, N, fl, blas_w in kinds:
            y = torch.zeros(M, N, device=dev)
            ops = [mt.op(xx, wl[i], y, M, flags=fl, w2=(w2l[i] if w2l else None)) for i in range(len(ws))]
            cs = torch.cuda.Stream(device=dev)

            def ours():
                for o in ops:
                    rc = L.mt_linear(o.x, o.xt, o.w, o.w2, o.wt, o.bias, o.y, o.p, cs.cuda_stream)
                    if rc:
                        raise RuntimeError(mt.last_error())

            def blas():
                for w in blas_w:
                    torch.matmul(xx, w.t())

            row = dict(M=M, op=name)
            for tag, fn in (("mt_linear_us", ours), ("hipblaslt_us", blas)):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.stream(cs):
                    fn()  # eager run first: split-K workspace growth is refused under capture
                    torch.cuda.synchronize()
                    with torch.cuda.graph(g, stream=cs):
                        fn()
                torch.cuda.synchronize()
                g.replay()
                torch.cuda.synchronize()
                ev = Events(torch)
                best = None
                for _ in range(reps):
                    ev.start()
                    g.replay()
                    ms = ev.stop_ms()
                    best = ms if best is None else min(best, ms)
                row[tag] = round(best * 1e3 / len(ops), 2)
                del g
            rows.append(row)
    return rows


def flow_step_graph(torch, mt, dev, fused=True, persistent=False):
    """The flow stage of one generation step at the reference's flow-head shape
    (MingEngine.encodeStep, Engine.swift:387-402; DiTForward.encode, DiT.swift:35-52): the
    cond embedder (896 -> 1024, M = 1), then 10 ODE steps of the EPSS schedule with sway
    (FlowSchedule, DiT.swift:55-65) of flow_assemble with that step's time embedding
    (precomputed once by the time MLP, Engine.swift:186-198, outside the timed region), 8 DiT
    blocks (hidden 1024, 16 heads, batch 2 x seq 3 = 6 rows: rmsnorm+qkv 3072x1024,
    dit_attention, out 1024x1024 +=, rmsnorm+ff1 4096x1024 GELU, ff2 1024x4096 +=), the final
    rmsnorm + 64x1024 linear and flow_euler with dt = t[k+1] - t[k], each step's Euler update
    fused with the next step's flow_assemble (mt_flow_euler_assemble): 422 launches, bf16
    weights ~ N(0, 0.02^2), captured in a HIP graph on its own stream.  With ``fused`` each
    block's attention runs inside its out projection (mt_dit_attention_linear): 342 launches.
    With ``persistent`` each ODE step's 8 blocks are one launch of the DiT-block kernel
    (mt_seq_create_items with DiT attention items): 32 launches, run on the stream (with
    --seq-launch coop the sequence launch is cooperative, which a graph does not capture; an
    ordinary one times the same either way), so `graph` is then the stage's function.
    Returns (graph, stream, launches, weight bytes per ODE step, the tensors to keep alive)."""
    HID, HEADS, LAT, BLOCKS, STEPS = 1024, 16, 64, 8, 10
    g = torch.Generator(device=dev)
    g.manual_seed(5)

    def w(*shape, scale=0.02):
        return (torch.randn(*shape, generator=g, device=dev) * scale).bfloat16()

    def gain(n):
        return (1.0 + 0.1 * torch.randn(n, generator=g, device=dev)).bfloat16()

    blocks = [dict(n1=gain(HID), qkv=w(3 * HID, HID), qkv_b=w(3 * HID), out=w(HID, HID), out_b=w(HID), n2=gain(HID),
                   ff1=w(4 * HID, HID), ff1_b=w(4 * HID), ff2=w(HID, 4 * HID), ff2_b=w(HID)) for _ in range(BLOCKS)]
    fin_n, fin_w, fin_b = gain(HID), w(LAT, HID), w(LAT)
    xw, xb, cb = w(HID, LAT, scale=0.05), w(HID, scale=0.05), w(HID, scale=1.0)
    i = torch.arange(32, device=dev, dtype=torch.float32)
    invf = (1.0 / torch.pow(torch.tensor(1e4, device=dev), 2.0 * i / 64.0)).float()
    y = torch.randn(LAT, device=dev)
    hist, cemb = torch.randn(LAT, device=dev), torch.zeros(1, HID, device=dev)
    z = torch.randn(1, H, device=dev)
    cond_w, cond_b = w(HID, H), w(HID)
    sched = mt.FlowSchedule.timesteps(STEPS)
    temb = mt.time_embeddings((w(HID, 256), w(HID)), (w(HID, HID), w(HID)), sched)
    x = torch.zeros(6, HID, device=dev)
    qkv = torch.zeros(6, 3 * HID, device=dev)
    att = torch.zeros(6, HID, device=dev)
    ff = torch.zeros(6, 4 * HID, device=dev)
    pred = torch.zeros(6, LAT, device=dev)
    cs = torch.cuda.Stream(device=dev)
    dts = [float(sched[k + 1] - sched[k]) for k in range(STEPS)]
    seq = None
    if persistent:
        items = []
        for p in blocks:
            items += [mt.op(x, p["qkv"], qkv, 6, bias=p["qkv_b"], norm=p["n1"]),
                      mt.dit_attn_op(qkv, 2, 3, HEADS, invf, att),
                      mt.op(att, p["out"], x, 6, flags=mt.GemvFlags.accumulate, bias=p["out_b"]),
                      mt.op(x, p["ff1"], ff, 6, flags=mt.GemvFlags.gelu, bias=p["ff1_b"], norm=p["n2"]),
                      mt.op(ff, p["ff2"], x, 6, flags=mt.GemvFlags.accumulate, bias=p["ff2_b"])]
        seq = mt.Seq(items)
    torch.cuda.synchronize()

    def step():
        mt.linear(z, cond_w, cemb, 1, bias=cond_b, stream=cs.cuda_stream)
        mt.flow_assemble(y, hist, cemb[0], cb, temb[0], xw, xb, x, stream=cs.cuda_stream)
        for k in range(STEPS):
            for p in ([] if persistent else blocks):
                mt.linear(x, p["qkv"], qkv, 6, bias=p["qkv_b"], norm=p["n1"], stream=cs.cuda_stream)
                if fused:
                    mt.dit_attention_linear(qkv, 2, 3, HEADS, invf, p["out"], x, flags=mt.GemvFlags.accumulate,
                                            bias=p["out_b"], stream=cs.cuda_stream)
                else:
                    mt.dit_attention(qkv, 2, 3, HEADS, invf, att, stream=cs.cuda_stream)
                    mt.linear(att, p["out"], x, 6, flags=mt.GemvFlags.accumulate, bias=p["out_b"],
                              stream=cs.cuda_stream)
                mt.linear(x, p["ff1"], ff, 6, flags=mt.GemvFlags.gelu, bias=p["ff1_b"], norm=p["n2"],
                          stream=cs.cuda_stream)
                mt.linear(ff, p["ff2"], x, 6, flags=mt.GemvFlags.accumulate, bias=p["ff2_b"], stream=cs.cuda_stream)
            if persistent:
                seq.run(stream=cs.cuda_stream)
            mt.linear(x, fin_w, pred, 6, bias=fin_b, norm=fin_n, stream=cs.cuda_stream)
            if k + 1 < STEPS:  # this step's Euler update and the next step's flow input, one launch
                mt.flow_euler_assemble(y, pred, 2, 5, 2.0, dts[k], hist, cemb[0], cb, temb[k + 1], xw, xb, x,
                                       stream=cs.cuda_stream)
            else:
                mt.flow_euler(y, pred, 2, 5, 2.0, dts[k], stream=cs.cuda_stream)

    wbytes = sum(sum(t.numel() * 2 for t in p.values()) for p in blocks) + (fin_w.numel() + xw.numel()) * 2
    keep = (blocks, fin_n, fin_w, fin_b, xw, xb, cb, invf, y, hist, cemb, z, cond_w, cond_b, temb, x, qkv, att, ff, pred,
            seq)
    if persistent:
        step()
        torch.cuda.synchronize()
        seq.check()
        return step, cs, 2 + STEPS * 3, wbytes, keep
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cs):
        step()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=cs):
            step()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    return graph, cs, 2 + STEPS * (2 + (4 if fused else 5) * BLOCKS), wbytes, keep


def bench_flow_step(torch, mt, dev, reps=5, fused=True, persistent=False):
    """The flow stage of flow_step_graph, replayed (or, persistent, run on its stream): the best
    of `reps` runs, each bracketed by HIP events on that stream."""
    graph, cs, launches, wbytes, keep = flow_step_graph(torch, mt, dev, fused, persistent)
    ev = Events(torch, cs) if persistent else Events(torch)
    best = None
    for _ in range(reps):
        ev.start()
        if persistent:
            graph()
        else:
            graph.replay()
        ms = ev.stop_ms()
        best = ms if best is None else min(best, ms)
    if persistent:
        torch.cuda.synchronize()
        keep[-1].check()
    del graph
    return dict(us_per_generation_step=best * 1e3, us_per_ode_step=best * 1e3 / 10,
                launches=launches, weight_mb_per_ode_step=wbytes / 1e6,
                schedule="EPSS 10 steps, sway -1",
                blocks="one DiT-block kernel launch per ODE step" if persistent else "a launch per linear",
                attention="inside the out projection" if fused or persistent else "separate launch")


def aggregator_stage(torch, mt, dev, persistent=False):
    """The aggregator stage of one generation step (MingEngine.encodeStep, Engine.swift:405-410):
    the cls row and x_embedder (1024 x 64) of the new latent, the 8-block DiT (hidden 1024, 16
    heads) at batch 1 x seq 2 (M = 2, attention inside the out projection), the final norm +
    896 x 1024 linear of row 0: 35 launches, bf16 weights ~ N(0, 0.02^2).  With ``persistent``
    the 8 blocks are one launch of the DiT-block kernel (DiT attention items): 4 launches.
    Returns (stage(stream handle), plan or None, launches, weight bytes)."""
    HID, HEADS, LAT, BLOCKS = 1024, 16, 64, 8
    g = torch.Generator(device=dev)
    g.manual_seed(7)

    def w(*shape, scale=0.02):
        return (torch.randn(*shape, generator=g, device=dev) * scale).bfloat16()

    def gain(n):
        return (1.0 + 0.1 * torch.randn(n, generator=g, device=dev)).bfloat16()

    blocks = [dict(n1=gain(HID), qkv=w(3 * HID, HID), qkv_b=w(3 * HID), out=w(HID, HID), out_b=w(HID), n2=gain(HID),
                   ff1=w(4 * HID, HID), ff1_b=w(4 * HID), ff2=w(HID, 4 * HID), ff2_b=w(HID)) for _ in range(BLOCKS)]
    fin_n, fin_w, fin_b = gain(HID), w(H, HID), w(H)
    xw, xb = w(HID, LAT, scale=0.05), w(HID, scale=0.05)
    i = torch.arange(32, device=dev, dtype=torch.float32)
    invf = (1.0 / torch.pow(torch.tensor(1e4, device=dev), 2.0 * i / 64.0)).float()
    cls = torch.randn(HID, device=dev)
    latent = torch.randn(1, LAT, device=dev)
    x = torch.zeros(2, HID, device=dev)
    qkv = torch.zeros(2, 3 * HID, device=dev)
    ff = torch.zeros(2, 4 * HID, device=dev)
    att = torch.zeros(2, HID, device=dev)
    out = torch.zeros(1, H, device=dev)
    seq = None
    if persistent:
        items = []
        for p in blocks:
            items += [mt.op(x, p["qkv"], qkv, 2, bias=p["qkv_b"], norm=p["n1"]),
                      mt.dit_attn_op(qkv, 1, 2, HEADS, invf, att),
                      mt.op(att, p["out"], x, 2, flags=mt.GemvFlags.accumulate, bias=p["out_b"]),
                      mt.op(x, p["ff1"], ff, 2, flags=mt.GemvFlags.gelu, bias=p["ff1_b"], norm=p["n2"]),
                      mt.op(ff, p["ff2"], x, 2, flags=mt.GemvFlags.accumulate, bias=p["ff2_b"])]
        seq = mt.Seq(items)

    def stage(s):
        x[0].copy_(cls)
        mt.linear(latent, xw, x[1:], 1, bias=xb, stream=s)
        if persistent:
            seq.run(stream=s)
        for p in ([] if persistent else blocks):
            mt.linear(x, p["qkv"], qkv, 2, bias=p["qkv_b"], norm=p["n1"], stream=s)
            mt.dit_attention_linear(qkv, 1, 2, HEADS, invf, p["out"], x, flags=mt.GemvFlags.accumulate, bias=p["out_b"],
                                    stream=s)
            mt.linear(x, p["ff1"], ff, 2, flags=mt.GemvFlags.gelu, bias=p["ff1_b"], norm=p["n2"], stream=s)
            mt.linear(ff, p["ff2"], x, 2, flags=mt.GemvFlags.accumulate, bias=p["ff2_b"], stream=s)
        mt.linear(x, fin_w, out, 1, bias=fin_b, norm=fin_n, stream=s)

    stage.keep = (blocks, fin_n, fin_w, fin_b, xw, xb, invf, cls, latent, x, qkv, ff, att, out)
    wbytes = sum(sum(t.numel() * 2 for t in p.values()) for p in blocks) + (fin_w.numel() + xw.numel()) * 2
    return stage, seq, 1 + 1 + (1 if persistent else 4 * BLOCKS) + 1, wbytes


def bench_aggregator(torch, mt, dev, reps=5, persistent=False):
    """The aggregator stage (aggregator_stage): as a HIP graph of 35 launches replayed, or, with
    ``persistent``, 4 launches run on the stream (as flow_step_graph runs its persistent
    stage), the median of `reps` runs between HIP events."""
    stage_fn, seq, launches, wbytes = aggregator_stage(torch, mt, dev, persistent)
    cs = torch.cuda.Stream(device=dev)

    def stage():
        stage_fn(cs.cuda_stream)

    if persistent:
        with torch.cuda.stream(cs):
            stage()
            torch.cuda.synchronize()
            ev = Events(torch, cs)
            times = []
            for _ in range(reps):
                ev.start()
                stage()
                times.append(ev.stop_ms() * 1e3)
        seq.check()
        us = sorted(times)[len(times) // 2]
        seq.close()
    else:
        us = graph_us(torch, stage, cs, rounds=reps)
    return dict(us_per_generation_step=us, launches=launches,
                weight_mb=wbytes / 1e6, gbs_algorithmic=wbytes / (us * 1e-6) / 1e9,
                blocks="one DiT-block kernel launch" if persistent else "a launch per linear")


def vae_latent_graph(torch, mt, dev, ws, fused=True):
    """The VAE latent of bench_vae_latent captured in a HIP graph on its own stream; returns
    (graph, stream, launches, the tensors the graph reads and writes, to be kept alive while
    it is replayed)."""
    HQ, HKV, CAP, NFFT, HOP, RING = 14, 2, 512, 3528, 882, 8
    pos0 = 4 * 50
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    h = [torch.randn(H, generator=g, device=dev) for _ in range(3)]
    frames = torch.zeros(4, H, device=dev)
    qkv = torch.zeros(4, QKV, device=dev)
    att = torch.zeros(4, HQ * 64, device=dev)
    mlp = torch.zeros(4, INTER, device=dev)
    spec = torch.zeros(4, NFFT + 2, device=dev)
    head_w = (torch.randn(NFFT + 2, H, generator=g, device=dev) * 0.02).half()
    head_b = (torch.randn(NFFT + 2, generator=g, device=dev) * 0.02).half()
    caches = [(torch.randn(HKV, CAP, 64, generator=g, device=dev).half(),
               torch.randn(HKV, CAP, 64, generator=g, device=dev).half()) for _ in ws]
    i = torch.arange(32, device=dev, dtype=torch.float32)
    invf = (1.0 / torch.pow(torch.tensor(1e6, device=dev), 2.0 * i / 64.0)).float()
    t = torch.arange(NFFT, device=dev, dtype=torch.float64)
    window = (0.5 - 0.5 * torch.cos(2 * torch.pi * t / NFFT)).float()
    cos_table = torch.cos(2 * torch.pi * t / NFFT).float()
    ring = torch.zeros(RING, NFFT, device=dev)
    pcm = torch.zeros(4 * HOP, device=dev)
    cs = torch.cuda.Stream(device=dev)
    s = cs.cuda_stream

    def step():
        mt.upsample4(h[0], h[1], h[2], frames, stream=s)
        for p, (kc, vc) in zip(ws, caches):
            mt.linear(frames, p["qkv"], qkv, 4, bias=p["qkv_b"], norm=p["norm1"], stream=s)
            if fused:
                mt.rope_attention(qkv, QKV, 4, HQ, HKV, pos0, 65, kc, vc, CAP, invf, att, HQ * 64, stream=s)
            else:
                mt.rope_cache(qkv, QKV, 4, HQ, HKV, pos0, kc, vc, CAP, invf, stream=s)
                mt.attention(qkv, QKV, 4, HQ, HKV, pos0, 65, kc, vc, CAP, att, HQ * 64, stream=s)
            mt.linear(att, p["o"], frames, 4, flags=mt.GemvFlags.accumulate, stream=s)
            mt.linear(frames, p["gate"], mlp, 4, flags=mt.GemvFlags.siluGate, w2=p["up"], norm=p["norm2"], stream=s)
            mt.linear(mlp, p["down"], frames, 4, flags=mt.GemvFlags.accumulate, stream=s)
        mt.linear(frames, head_w, spec, 4, bias=head_b, stream=s)
        mt.istft_frames(spec, 4, NFFT, cos_table, window, ring, 4 * 50, RING, stream=s)
        mt.istft_emit(ring, window, NFFT, HOP, 4 * 50 * HOP, 4 * HOP, 4 * 50 + 3, RING, pcm, stream=s)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cs):
        step()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=cs):
            step()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    keep = (h, frames, qkv, att, mlp, spec, head_w, head_b, caches, invf, window, cos_table, ring, pcm)
    return graph, cs, 1 + (5 if fused else 6) * len(ws) + 3, keep


def bench_vae_latent(torch, mt, dev, ws, reps=5, fused=True):
    """One latent of the streaming VAE decoder (VAEDecoder.decodeDispatches, VAEDecoder.swift:
    81-107) after fc1: upsample4, the 24-layer sliding-window Qwen stack at M = 4 rows (rmsnorm
    + qkv, rope_cache, attention over the last 65 keys, o +=, rmsnorm + gate|up, down +=; the
    backbone's synthetic fp16 weights stand in for the VAE stack's, same shapes), the 3530 x
    896 spectrum head, istft_frames (nfft 3528) and istft_emit (4 hops): 148 launches,
    captured in a HIP graph and replayed.  With ``fused`` each layer's rope_cache and
    attention run as one mt_rope_attention launch: 124 launches."""
    graph, cs, launches, keep = vae_latent_graph(torch, mt, dev, ws, fused)
    us = graph_us_replay(torch, graph, cs, reps)
    del graph
    return dict(us_per_latent=us, launches=launches, audio_ms_per_latent=4 * 882 / 44100 * 1e3)


def vae_latent_seq_stage(torch, mt, dev, ws):
    """The VAE latent with its 24-layer stack as one persistent launch: upsample4, the stack at
    M = 4 rows of one sequence (rmsnorm + qkv, RoPE + cache append + attention over the last
    65 keys as an attention item, o +=, rmsnorm + gate|up, down +=: 120 items), the spectrum
    head, istft_frames and istft_emit: 5 launches.  Returns (step(stream handle), plan)."""
    HQ, HKV, CAP, NFFT, HOP, RING = 14, 2, 512, 3528, 882, 8
    pos0 = 4 * 50
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    h = [torch.randn(H, generator=g, device=dev) for _ in range(3)]
    frames = torch.zeros(4, H, device=dev)
    qkv = torch.zeros(4, QKV, device=dev)
    att = torch.zeros(4, HQ * 64, device=dev)
    mlp = torch.zeros(4, INTER, device=dev)
    spec = torch.zeros(4, NFFT + 2, device=dev)
    head_w = (torch.randn(NFFT + 2, H, generator=g, device=dev) * 0.02).half()
    head_b = (torch.randn(NFFT + 2, generator=g, device=dev) * 0.02).half()
    caches = [(torch.randn(HKV, CAP, 64, generator=g, device=dev).half(),
               torch.randn(HKV, CAP, 64, generator=g, device=dev).half()) for _ in ws]
    i = torch.arange(32, device=dev, dtype=torch.float32)
    invf = (1.0 / torch.pow(torch.tensor(1e6, device=dev), 2.0 * i / 64.0)).float()
    t = torch.arange(NFFT, device=dev, dtype=torch.float64)
    window = (0.5 - 0.5 * torch.cos(2 * torch.pi * t / NFFT)).float()
    cos_table = torch.cos(2 * torch.pi * t / NFFT).float()
    ring = torch.zeros(RING, NFFT, device=dev)
    pcm = torch.zeros(4 * HOP, device=dev)
    pos_d = torch.arange(pos0, pos0 + 4, device=dev, dtype=torch.int32)
    items = []
    for p, (kc, vc) in zip(ws, caches):
        items.append(mt.op(frames, p["qkv"], qkv, 4, bias=p["qkv_b"], norm=p["norm1"]))
        items.append(mt.attn_op(qkv, 4, HQ, HKV, pos_d, kc, vc, CAP, 0, invf, att, window=65))
        items.append(mt.op(att, p["o"], frames, 4, flags=mt.GemvFlags.accumulate))
        items.append(mt.op(frames, p["gate"], mlp, 4, flags=mt.GemvFlags.siluGate, w2=p["up"], norm=p["norm2"]))
        items.append(mt.op(mlp, p["down"], frames, 4, flags=mt.GemvFlags.accumulate))
    seq = mt.Seq(items)
    keep = (h, frames, qkv, att, mlp, spec, head_w, head_b, caches, invf, window, cos_table, ring, pcm, pos_d, items)

    def step(s):
        mt.upsample4(h[0], h[1], h[2], frames, stream=s)
        seq.run(s)
        mt.linear(frames, head_w, spec, 4, bias=head_b, stream=s)
        mt.istft_frames(spec, 4, NFFT, cos_table, window, ring, 4 * 50, RING, stream=s)
        mt.istft_emit(ring, window, NFFT, HOP, 4 * 50 * HOP, 4 * HOP, 4 * 50 + 3, RING, pcm, stream=s)

    step.keep = keep
    return step, seq


def bench_vae_latent_seq(torch, mt, dev, ws, reps=7):
    """The VAE latent of bench_vae_latent with its 24-layer stack as one persistent launch
    (vae_latent_seq_stage): 5 launches on one stream (as flow_step_graph runs its persistent
    stage), timed with HIP events on it."""
    HOP = 882
    run, seq = vae_latent_seq_stage(torch, mt, dev, ws)
    cs = torch.cuda.Stream(device=dev)
    s = cs.cuda_stream

    def step():
        run(s)

    times = []
    with torch.cuda.stream(cs):
        step()
        torch.cuda.synchronize()
        for _ in range(reps):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            step()
            b.record()
            b.synchronize()
            times.append(a.elapsed_time(b))
    seq.check()
    kern = seq.kernel
    seq.close()
    return dict(us_per_latent=1e3 * sorted(times)[len(times) // 2], launches=5, items=120,
                kernel="decode-layer kernel" if kern == mt.SEQ_DECODE_LAYER else "general sequence kernel",
                audio_ms_per_latent=4 * HOP / 44100 * 1e3)


def llm_token_stage(torch, mt, dev, ws, M=1, cap=512):
    """The llm stage's token (MingEngine.encodeStep, Engine.swift:381-385): the 24 decode layers
    with attention at the reference's single row (QwenForward.dispatches with rows 1,
    Qwen.swift:72-97) as one persistent launch of 120 items, the final RMSNorm of that row
    (Qwen.swift:94) and the stop head (2 x 896 + bias, Engine.swift:385).  Returns
    (stage(stream handle), plan)."""
    import numpy as np
    HQ, HKV = 14, 2
    lens = np.random.default_rng(1).integers(32, cap + 1, M).astype(np.int32)
    pos = torch.from_numpy(lens - 1).to(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    caches = [(torch.randn(M, HKV, cap, 64, generator=g, device=dev).half(),
               torch.randn(M, HKV, cap, 64, generator=g, device=dev).half()) for _ in ws]
    i = torch.arange(32, device=dev, dtype=torch.float32)
    inv_freq = (1.0 / torch.pow(torch.tensor(1e6, device=dev), 2.0 * i / 64.0)).float()
    resid = torch.randn(M, H, generator=g, device=dev)
    qkv = torch.zeros(M, QKV, device=dev)
    att = torch.zeros(M, HQ * 64, device=dev)
    mlp = torch.zeros(M, INTER, device=dev)
    z = torch.zeros(M, H, device=dev)
    final_norm = (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).half()
    stop_w = (0.02 * torch.randn(2, H, generator=g, device=dev)).half()
    stop_b = (0.02 * torch.randn(2, generator=g, device=dev)).half()
    logits = torch.zeros(M, 2, device=dev)
    items = []
    for p, (kc, vc) in zip(ws, caches):
        items.append(mt.op(resid, p["qkv"], qkv, M, bias=p["qkv_b"], norm=p["norm1"]))
        items.append(mt.attn_op(qkv, M, HQ, HKV, pos, kc, vc, cap, HKV * cap * 64, inv_freq, att))
        items.append(mt.op(att, p["o"], resid, M, flags=mt.GemvFlags.accumulate))
        items.append(mt.op(resid, p["gate"], mlp, M, flags=mt.GemvFlags.siluGate, w2=p["up"], norm=p["norm2"]))
        items.append(mt.op(mlp, p["down"], resid, M, flags=mt.GemvFlags.accumulate))
    seq = mt.Seq(items)

    def stage(s):
        seq.run(s)
        mt.rmsnorm(resid, final_norm, z, rows=M, stream=s)
        mt.linear(z, stop_w, logits, M, bias=stop_b, stream=s)

    stage.keep = (caches, pos, inv_freq, resid, qkv, att, mlp, z, final_norm, stop_w, stop_b, logits, items)
    return stage, seq


# The reference's per-stage GPU times of one generation step on its Apple GPU (bf16 weights,
# fp32 activations), .claude/skills/verify/features/bench.md:25, in us.
REF_STEP_US = {"llm": 5240.0, "flow": 8930.0, "agg": 840.0, "total": 15010.0}


def bench_generation_step(torch, mt, dev, ws, reps=5):
    """One whole generation step after the prefill (MingEngine.encodeStep, Engine.swift:377-415),
    stage by stage as the reference's StepRecorder times it (Engine.swift:30-85), on one stream
    with HIP events between the stages:
      llm:  llm_token_stage (24 decode layers with attention at M = 1 in one launch, final
            norm, stop head);
      vae:  the VAE frames of an older latent (vae_latent_seq_stage).  The reference encodes
            them beside the llm token on a concurrent encoder (Engine.swift:383-384), so its
            "llm" figure covers both; here they run one after the other;
      flow: the cond embedder and 10 EPSS ODE steps of the 8-block DiT at M = 6
            (flow_step_graph, persistent: each ODE step's 8 blocks one DiT-block kernel launch,
            32 launches);
      agg:  the aggregator with its 8 DiT blocks as one launch (aggregator_stage).
    The median of `reps` runs per stage, after one untimed run."""
    llm, llm_seq = llm_token_stage(torch, mt, dev, ws)
    vae, vae_seq = vae_latent_seq_stage(torch, mt, dev, ws)
    flow, cs, flow_launches, _, flow_keep = flow_step_graph(torch, mt, dev, fused=True, persistent=True)
    agg, agg_seq, agg_launches, _ = aggregator_stage(torch, mt, dev, persistent=True)
    s = cs.cuda_stream
    names = ("llm", "vae", "flow", "agg")
    times = {n: [] for n in names}
    with torch.cuda.stream(cs):
        for r in range(reps + 1):
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
            ev[0].record(cs)
            llm(s)
            ev[1].record(cs)
            vae(s)
            ev[2].record(cs)
            flow()
            ev[3].record(cs)
            agg(s)
            ev[4].record(cs)
            ev[4].synchronize()
            if r:
                for j, n in enumerate(names):
                    times[n].append(1e3 * ev[j].elapsed_time(ev[j + 1]))
    for q in (llm_seq, vae_seq, agg_seq, flow_keep[-1]):
        q.check()
        q.close()
    med = {n: sorted(t)[len(t) // 2] for n, t in times.items()}
    out = {f"{n}_us": med[n] for n in names}
    out["llm_with_vae_us"] = med["llm"] + med["vae"]
    out["total_us"] = sum(med.values())
    out["launches"] = {"llm": 3, "vae": 5, "flow": flow_launches, "agg": agg_launches}
    out["reference_us"] = {"llm_with_vae": REF_STEP_US["llm"], "flow": REF_STEP_US["flow"], "agg": REF_STEP_US["agg"],
                           "total": REF_STEP_US["total"],
                           "source": "Apple M-series GPU, .claude/skills/verify/features/bench.md:25"}
    out["llm_rows"] = 1
    del flow, flow_keep
    return out


def graph_us_replay(torch, graph, stream, rounds=5) -> float:
    """Median replay time (us) of an already captured graph on `stream`, HIP events on it."""
    times = []
    with torch.cuda.stream(stream):
        for _ in range(rounds):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            graph.replay()
            b.record()
            b.synchronize()
            times.append(a.elapsed_time(b))
    return 1e3 * sorted(times)[len(times) // 2]


def bench_paired(torch, mt, dev, ws, rounds=7, M=2):
    """The paired step of the reference (MingEngine.encodeStep, Engine.swift:377-385;
    QwenForward.encodePaired, Qwen.swift:103-115; timed paired against serial by QwenBench,
    QwenBench.swift:135-154): the LLM token's decode step and the VAE frames of an earlier
    latent issued together.  Here: the decode step (one persistent launch of the 24 layers'
    96 linears at M = 2) on one stream and the VAE latent (the graph of bench_vae_latent) on
    a second stream that starts with it; serial: the same two back to back on one stream.
    Medians over `rounds`, each bracketed by HIP events on the first stream."""
    graph, _, _, keep = vae_latent_graph(torch, mt, dev, ws)
    resid = torch.randn(M, H, device=dev)
    qkv = torch.zeros(M, QKV, device=dev)
    mlp = torch.zeros(M, INTER, device=dev)
    x0 = resid.clone()
    seq = mt.Seq(decode_ops(mt, ws, M, resid, qkv, mlp))
    sa = torch.cuda.Stream(device=dev)
    sb = torch.cuda.Stream(device=dev)

    def timed(paired: bool) -> float:
        with torch.cuda.stream(sa):
            resid.copy_(x0)
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            if paired:
                sb.wait_event(a)
            seq.run(sa)
            if paired:
                with torch.cuda.stream(sb):
                    graph.replay()
                    done = torch.cuda.Event()
                    done.record()
                sa.wait_event(done)
            else:
                graph.replay()
            b.record()
        b.synchronize()
        return a.elapsed_time(b)

    timed(False)
    timed(True)
    serial, paired = [], []
    for _ in range(rounds):
        serial.append(timed(False))
        paired.append(timed(True))
    seq.check()
    seq.close()
    del graph
    med = lambda v: 1e3 * sorted(v)[len(v) // 2]
    return dict(serial_us=med(serial), paired_us=med(paired), saved_us=med(serial) - med(paired),
                decode="persistent decode step, 24 layers, M = 2", vae="VAE latent graph, 124 launches")


def bench_copy(torch, dev, mib=1024, reps=5):
    """A plain device-to-device copy of a known size: the calibration run for the HBM byte
    counters (FETCH_SIZE / WRITE_SIZE per dispatch against exactly mib MiB each way)."""
    a = torch.empty(mib << 18, device=dev, dtype=torch.float32).fill_(1.0)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    ev = Events(torch)
    ev.start()
    for _ in range(reps):
        b.copy_(a)
    ms = ev.stop_ms()
    return dict(copy_mib=mib, reps=reps, us_per_copy=round(ms * 1e3 / reps, 2),
                gbs_read_plus_write=round(2 * (mib << 20) * reps / (ms * 1e-3) / 1e9, 1))


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), as lscpu prints it."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(torch, ws, target_s=8.0, M=2):
    """The oracle's vectorised restatement of the reference CPU loop (KernelTests.swift:86-101,
    K sum split 16 ways, OpenMP over output rows) on the host cores, over the whole decode step
    (all 24 layers, same shapes, same weights): steps repeated for about target_s seconds on
    every OpenMP thread, then again on one thread."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as O
    host = [{k: v.cpu().numpy().view(np.uint16) for k, v in p.items()} for p in ws]
    rng = np.random.default_rng(1)
    resid0 = rng.standard_normal((M, H)).astype(np.float32)
    gains = [(O.decode16(p["norm1"], O.F16), O.decode16(p["norm2"], O.F16)) for p in host]

    def norm(x, g):
        return (x * (np.float32(1.0) / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + np.float32(1e-6))) * g
                ).astype(np.float32)

    def step(threads):
        resid = resid0.copy()
        for p, (g1, g2) in zip(host, gains):
            qkv = O.linear_fast(norm(resid, g1), p["qkv"], None, O.F16, p["qkv_b"], None, M, QKV, H, 0, threads)
            resid = O.linear_fast(np.ascontiguousarray(qkv[:, :H]), p["o"], None, O.F16, None, resid, M, H, H,
                                  O.ACCUM, threads)
            mlp = O.linear_fast(norm(resid, g2), p["gate"], p["up"], O.F16, None, None, M, INTER, H, O.SILU_GATE,
                                threads)
            resid = O.linear_fast(mlp, p["down"], None, O.F16, None, resid, M, H, INTER, O.ACCUM, threads)
        return resid

    def timed(threads):
        step(threads)
        n = 0
        t0 = time.perf_counter()
        while True:
            step(threads)
            n += 1
            dt = time.perf_counter() - t0
            if dt >= target_s:
                return n, dt

    threads = O.max_threads()
    n, dt = timed(threads)
    n1, dt1 = timed(1)
    per_layer = (shape_bytes(M, QKV, H, 1) + shape_bytes(M, H, H, 2) + shape_bytes(M, INTER, H, 8)
                 + shape_bytes(M, H, INTER, 2))
    nbytes = per_layer * len(host)
    return dict(value=nbytes * n / dt / 1e9, unit="GB/s", cores=threads, kind="port",
                sample=f"the whole decode step (24 layers, 96 linears, M=2, fp16 W) x {n} steps in {dt:.1f} s on "
                       f"{threads} OpenMP threads, then x {n1} steps in {dt1:.1f} s on 1 thread; oracle linear_fast "
                       f"(K sum split 16 ways)",
                step_ms=1e3 * dt / n, value_1thread=nbytes * n1 / dt1 / 1e9, step_ms_1thread=1e3 * dt1 / n1,
                cpu_model=cpu_model(), nproc=os.cpu_count())


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--seq-launch", choices=["coop", "plain"], default="plain",
                    help="launch of the persistent sequence kernels: ordinary (the library's default) "
                         "or cooperative (co-residency guaranteed, about 17 us later per launch)")
    ap.add_argument("--only", choices=["decode", "layer", "all", "copy", "gemm", "prefill", "chain", "vae", "attention", "flow",
                                       "step", "refshapes", "prefill174"],
                    default="all",
                    help="decode: only the linear decode step; layer: it and the decode step with attention; "
                         "copy: only the 1 GiB device copy that calibrates the HBM byte counters; "
                         "gemm: only the prefill and DiT GEMM stacks; prefill: only the prefill stack at --rows; "
                         "chain: only the fp32-activation prefill chain at --rows; vae: only the VAE latent "
                         "(graph of launches, then with the persistent stack); attention: only the decode attention; "
                         "step: only one whole generation step, stage by stage; refshapes: only the reference "
                         "benches' shapes (the 17 GEMV bench shapes, the 174-row prefill per part); prefill174: "
                         "only the 174-row prefill per part")
    ap.add_argument("--rows", type=int, default=512, help="with --only prefill or chain: the prompt rows M")
    ap.add_argument("--vs-blas", action="store_true",
                    help="with --only gemm: also time each prefill linear alone (graph replay) "
                         "next to hipBLASLt on the same shapes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: there is no multi-GPU path (the linear hot path would "
              "shard by output features across GPUs); run with --gpus 1", file=sys.stderr)
        return 2
    ensure_built()
    import torch
    import mingtts as mt
    mt.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.only == "copy":
        print(json.dumps(bench_copy(torch, dev)), flush=True)
        return 0
    mt.set_tuning(mt.TUNE_SEQ_LAUNCH, 1 if args.seq_launch == "plain" else 0)
    log("generating 24 layers of fp16 weights")
    ws = make_layers(torch, dev)
    torch.cuda.synchronize()
    if args.only == "prefill":
        log(f"prefill stack M={args.rows}")
        print(json.dumps({k: (round(v, 3) if isinstance(v, float) else v)
                          for k, v in bench_prefill(torch, mt, dev, ws, args.rows).items()}), flush=True)
        return 0
    if args.only == "vae":
        log("VAE latent: graph of launches, then with the layer stack as one persistent launch")
        out = {"vae_latent": bench_vae_latent(torch, mt, dev, ws), "vae_latent_persistent": bench_vae_latent_seq(torch, mt, dev, ws)}
        print(json.dumps({k: {kk: (round(vv, 3) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                          for k, v in out.items()}), flush=True)
        return 0
    if args.only == "flow":
        log("flow stage of one generation step (10 ODE steps, 8 DiT blocks, graph replay)")
        out = {"aggregator": bench_aggregator(torch, mt, dev),
               "aggregator_persistent": bench_aggregator(torch, mt, dev, persistent=True)}
        for name, kw in (("flow_step_persistent", dict(persistent=True)), ("flow_step", dict(fused=True)),
                         ("flow_step_separate_attention", dict(fused=False))):
            out[name] = {k: (round(v, 3) if isinstance(v, float) else v)
                         for k, v in bench_flow_step(torch, mt, dev, **kw).items()}
        print(json.dumps(out), flush=True)
        return 0
    if args.only == "refshapes":
        log("the reference GEMV bench's 17 decode shapes, rotated 1 GiB pools")
        out = {"gemv_bench_shapes": bench_gemv_shapes(torch, mt, dev)}
        log("prefill at the reference bench's 174 prompt rows, whole layers and per part")
        out["prefill_174"] = bench_prefill_parts(torch, mt, dev, ws)
        print(json.dumps(out), flush=True)
        return 0
    if args.only == "prefill174":
        log("prefill at the reference bench's 174 prompt rows, whole layers and per part")
        print(json.dumps({"prefill_174": bench_prefill_parts(torch, mt, dev, ws)}), flush=True)
        return 0
    if args.only == "step":
        log("one generation step: llm token, VAE latent, flow stage, aggregator")
        print(json.dumps({k: (round(v, 3) if isinstance(v, float) else v)
                          for k, v in bench_generation_step(torch, mt, dev, ws).items()}), flush=True)
        return 0
    if args.only == "attention":
        log("decode attention, batch 2")
        print(json.dumps({k: (round(v, 3) if isinstance(v, float) else v) for k, v in bench_attention(torch, mt, dev).items()}),
              flush=True)
        return 0
    if args.only == "chain":
        log(f"prefill chain (fp32 activations, fused norms) M={args.rows}")
        print(json.dumps({k: (round(v, 3) if isinstance(v, float) else v)
                          for k, v in bench_prefill_chain(torch, mt, dev, ws, args.rows).items()}), flush=True)
        return 0
    if args.only == "gemm":
        out = {"prefill": [], "dit_head": None}
        for M in (64, 256, 512):
            log(f"prefill stack M={M}")
            out["prefill"].append({k: (round(v, 3) if isinstance(v, float) else v)
                                   for k, v in bench_prefill(torch, mt, dev, ws, M).items()})
        out["prefill_chain"] = []
        for M in (64, 256, 512):
            log(f"prefill chain (fp32 activations, fused norms) M={M}")
            out["prefill_chain"].append({k: (round(v, 3) if isinstance(v, float) else v)
                                         for k, v in bench_prefill_chain(torch, mt, dev, ws, M).items()})
        log("DiT head")
        out["dit_head"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in bench_dit(torch, mt, dev).items()}
        log("flow stage of one generation step (10 ODE steps, 8 DiT blocks, graph replay)")
        out["flow_step"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in bench_flow_step(torch, mt, dev).items()}
        log("aggregator stage of one generation step (8 DiT blocks at M = 2, graph replay)")
        out["aggregator"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in bench_aggregator(torch, mt, dev).items()}
        log("prefill at the reference bench's 174 prompt rows, whole layers and per part")
        out["prefill_174"] = bench_prefill_parts(torch, mt, dev, ws)
        if args.vs_blas:
            log("per-op graph replay: mt_linear vs hipBLASLt")
            out["per_op_graph_replay"] = bench_gemm_ops(torch, mt, dev, ws)
        print(json.dumps(out), flush=True)
        return 0

    log(f"decode step (persistent sequence, {args.seq_launch} launch): {args.warmup} warmup + {args.steps} timed")
    d = bench_decode_seq(torch, mt, dev, ws, args.steps, args.warmup)
    t = sorted(d["times_ms"])
    mean_ms = sum(t) / len(t)
    median_ms = t[len(t) // 2]
    gbs = d["bytes"] / (mean_ms * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(mean_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0, 0.02^2) fp16 weights, N(0, 1) fp32 activations, generated on the device)",
        "config": {
            "workload": "decode step of the Qwen2-0.5B backbone linears: 24 layers x {rmsnorm+qkv 1152x896+bias, "
                        "o 896x896 +=, rmsnorm+gate|up 2x4864x896 SiLU*mul, down 896x4864 +=}, M=2 (CFG pair), "
                        "fp16 W, fp32 activations and outputs, one persistent launch of 96 dependent linears "
                        "(RMSNorm fused into the qkv and gate|up prologues)",
            "layers": LAYERS, "rows": 2, "hidden": H, "intermediate": INTER, "qkv": QKV,
            "parallelism": "single GPU",
        },
        "decode_step_us": round(mean_ms * 1e3, 2),
        "decode_step_us_median": round(median_ms * 1e3, 2),
        "decode_step_us_min": round(t[0] * 1e3, 2),
        "hbm_pct_of_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "algorithmic_bytes_per_step": d["bytes"],
        "seq_workgroups": d["groups"],
        "seq_launch": args.seq_launch,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "traffic_source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, profiles/layer_kernel_decode_24L_M2.md",
                     "kernel": d["kernel"]},
    }
    if args.only in ("all", "layer"):
        log("decode layers with attention (persistent sequence, 120 items)")
        line["decode_layer_step"] = {k: (round(v, 3) if isinstance(v, float) else v)
                                     for k, v in bench_decode_layers(torch, mt, dev, ws, args.steps, args.warmup).items()}
    if args.only == "all":
        log("empty-dispatch floor (graph of one-element kernels)")
        line["launch_floor"] = {k: (round(v, 3) if isinstance(v, float) else v)
                                for k, v in bench_launch_floor(torch, dev).items()}
        log("decode step as 96 separate launches (graph replay)")
        line["decode_step_us_per_op_launches"] = round(bench_decode_per_op(torch, mt, dev, ws)["us"], 2)
        log("single GEMV 4864x896 from a rotated 1 GiB pool")
        line["gemv_single"] = {k: (round(v, 3) if isinstance(v, float) else v)
                               for k, v in bench_gemv_single(torch, mt, dev).items()}
        line["gemv_single_m2"] = {k: (round(v, 3) if isinstance(v, float) else v)
                                  for k, v in bench_gemv_single(torch, mt, dev, M=2).items()}
        line["prefill"] = []
        for M in (64, 256, 512):
            log(f"prefill stack M={M}")
            line["prefill"].append({k: (round(v, 3) if isinstance(v, float) else v)
                                    for k, v in bench_prefill(torch, mt, dev, ws, M).items()})
        line["prefill_chain"] = []
        for M in (64, 256, 512):
            log(f"prefill chain (fp32 activations, fused norms) M={M}")
            line["prefill_chain"].append({k: (round(v, 3) if isinstance(v, float) else v)
                                          for k, v in bench_prefill_chain(torch, mt, dev, ws, M).items()})
        log("prefill at the reference bench's 174 prompt rows, whole layers and per part")
        line["prefill_174"] = bench_prefill_parts(torch, mt, dev, ws)
        log("the reference GEMV bench's 17 decode shapes, rotated 1 GiB pools")
        line["gemv_bench_shapes"] = bench_gemv_shapes(torch, mt, dev)
        log("decode attention batch 2")
        line["attention_decode"] = {k: (round(v, 3) if isinstance(v, float) else v)
                                    for k, v in bench_attention(torch, mt, dev).items()}
        log("DiT head")
        line["dit_head"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in bench_dit(torch, mt, dev).items()}
        log("DiT head, cold weights")
        line["dit_head_cold"] = {k: (round(v, 3) if isinstance(v, float) else v)
                                 for k, v in bench_dit(torch, mt, dev, cold=True).items()}
        log("flow stage of one generation step (10 ODE steps, 8 DiT blocks, graph replay)")
        line["flow_step"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in bench_flow_step(torch, mt, dev).items()}
        log("flow stage as one DiT-block kernel launch per ODE step")
        line["flow_step_persistent"] = {k: (round(v, 3) if isinstance(v, float) else v)
                                        for k, v in bench_flow_step(torch, mt, dev, persistent=True).items()}
        line["flow_step_separate_attention"] = {k: (round(v, 3) if isinstance(v, float) else v)
                                                for k, v in bench_flow_step(torch, mt, dev, fused=False).items()}
        log("aggregator stage of one generation step (8 DiT blocks at M = 2, graph replay)")
        line["aggregator"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in bench_aggregator(torch, mt, dev).items()}
        log("aggregator stage with the 8 DiT blocks as one persistent launch")
        line["aggregator_persistent"] = {k: (round(v, 3) if isinstance(v, float) else v)
                                         for k, v in bench_aggregator(torch, mt, dev, persistent=True).items()}
        log("VAE decode of one latent (24-layer stack at M = 4, head, ISTFT; graph replay)")
        line["vae_latent"] = {k: (round(v, 3) if isinstance(v, float) else v)
                              for k, v in bench_vae_latent(torch, mt, dev, ws).items()}
        log("VAE decode of one latent with the layer stack as one persistent launch")
        line["vae_latent_persistent"] = {k: (round(v, 3) if isinstance(v, float) else v)
                                         for k, v in bench_vae_latent_seq(torch, mt, dev, ws).items()}
        log("one generation step, stage by stage (llm token, VAE latent, flow, aggregator)")
        line["generation_step"] = {k: (round(v, 3) if isinstance(v, float) else v)
                                   for k, v in bench_generation_step(torch, mt, dev, ws).items()}
        log("LLM decode step paired with a VAE latent on two streams, and serial")
        line["llm_vae_paired"] = {k: (round(v, 3) if isinstance(v, float) else v)
                                  for k, v in bench_paired(torch, mt, dev, ws).items()}
    if not args.no_cpu:
        log("CPU baseline (oracle, host cores)")
        cb = cpu_baseline(torch, ws)
        line["cpu_baseline"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in cb.items()}
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
