#!/usr/bin/env python3
"""Benchmark of the gfx950 PQ2_0 matmul path (one MI355X).

Headline metric: decode GEMV GB/s at 17408x5120 (config 1's gate/up shape),
batch 1.  A "step" is one bonsai_p40_gemv over one
17408x5120 PQ2_0 matrix with an already-quantised activation resident in HBM.
The weights rotate through enough distinct copies (>= 1.1 GB) that every step
streams its matrix from HBM rather than from the 256 MB Infinity Cache.

`value` = algorithmic bytes per GEMV (W + Q8_1 activation + fp32 output =
23,750,272 B) / measured time per GEMV.  Timing uses HIP events on the stream
the kernels run on (torch's current stream, whose handle is passed to the C
ABI).  The same JSON line carries the roofline of that kernel, secondary
measurements (configs 0-4: FWHT+Q8_1 pre-pass, FFN chain, per-token sweep,
small batch, prefill GEMM TOPS) and the CPU baseline: the reference's own host
GEMV (compiled from the reference sources into oracle/_ref) timed on this
host's cores on a bounded sample of the same workload.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--quick] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "p40-kernel_amd"))

import torch  # noqa: E402

import bonsai_p40 as B  # noqa: E402

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA
N_EMBD, N_FF, Q_DIM, KV_DIM, N_LAYER = 5120, 17408, 6144, 1024, 64


def gemv_bytes(n_out: int, n_in: int, n_tok: int = 1) -> int:
    return B.pq2_bytes(n_out, n_in) + n_tok * (B.q8_bytes(n_in) + 4 * n_out)


# ------------------------------------------------------ synthetic inputs
def synth_weights(n_out: int, n_in: int, gen: torch.Generator) -> torch.Tensor:
    """PQ2_0 blocks on the GPU: codes {0,1,2} w.p. (1-0.001)/3 each, code 3
    w.p. 0.001; d = fp16(|N(0, 0.02)| + 1e-4)."""
    nb = n_in // B.QK_PQ2
    nblk = n_out * nb
    u = torch.rand((nblk, 32, 4), generator=gen, device="cuda")
    codes = torch.where(u <= 0.001, torch.full_like(u, 3.0),
                        torch.clamp(torch.floor((u - 0.001) / (0.999 / 3)), max=2.0)).to(torch.int32)
    packed = (codes[..., 0] | (codes[..., 1] << 2) | (codes[..., 2] << 4) | (codes[..., 3] << 6)).to(torch.uint8)
    d = (torch.randn((nblk,), generator=gen, device="cuda").abs() * 0.02 + 1e-4).to(torch.float16)
    blocks = torch.empty((nblk, B.PQ2_BYTES), dtype=torch.uint8, device="cuda")
    blocks[:, 0:2] = d.view(torch.uint8).view(nblk, 2)
    blocks[:, 2:] = packed
    return blocks.view(-1)


def synth_activation_q8(n_in: int, gen: torch.Generator, n_tok: int = 1) -> torch.Tensor:
    """N(0,1) token rows -> FWHT-1024 -> Q8_1, through the product pre-pass."""
    x = torch.randn((n_tok, n_in), generator=gen, device="cuda")
    q = torch.empty(B.q8_bytes(n_in, n_tok), dtype=torch.uint8, device="cuda")
    if n_tok == 1:
        B.fwht_quant(x, None, q, n_in)
    else:
        B.quant_tokens(x, None, q, n_in, n_tok, True)
    return q


# --------------------------------------------------------------- timing
def time_loop_eager(fn, steps: int, warmup: int) -> float:
    """ms per call of fn(i) launched one by one from Python (HIP events on
    the current stream): includes the host launch cost of each call."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        fn(warmup + i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


GRAPH = True


def gpu_busy_while_host_enqueues(cycles: int = 2_000_000) -> None:
    """Queue a GPU spin ahead of the start event, outside the timed region:
    the host then enqueues the graph replays while the GPU spins, so the
    interval between the two events is the replays' GPU execution only, not
    the host's graph-launch latency (at 20 launches per graph that latency
    alone adds ~0.6 us per launch).  No-op where torch has no spin kernel."""
    try:
        torch.cuda._sleep(cycles)
    except (AttributeError, RuntimeError):
        pass


def time_loop(fn, steps: int, warmup: int, per_graph: int = 0) -> float:
    """ms per call of fn(i), measured on the GPU: `per_graph` consecutive
    calls are captured once into a HIP graph, the graph is replayed until
    `steps` calls ran, bracketed by HIP events on the stream the kernels run
    on.  The graph only removes the host's per-call launch cost; every call is
    still one full kernel launch (or more) on the stream.  A GPU spin queued
    before the start event keeps the host's graph-launch latency out of the
    interval; each replay's own GPU-side start-up stays in it (measured ~5 us
    per replay at 17408x5120: 20 launches per graph read ~0.2 us per launch
    more than 100 per graph)."""
    if not GRAPH:
        return time_loop_eager(fn, steps, warmup)
    k = per_graph or min(steps, 100)
    reps = max(1, (steps + k - 1) // k)
    for i in range(min(warmup, 3)):
        fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(k):
            fn(i)
    for _ in range(max(1, warmup // k)):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    gpu_busy_while_host_enqueues()
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    del g
    return e0.elapsed_time(e1) / (reps * k)


def copies_for(nbytes: int, target: float = 1.1e9) -> int:
    return max(2, math.ceil(target / nbytes))


def bench_gemv(n_out, n_in, steps, warmup, gen, n_tok=1, copies=0, ws=False):
    """us per launch over `copies` weight copies (0: enough to leave every
    cache cold; 1: one copy reused, cache-warm).  ws: the GEMM with its
    workspace (bonsai_p40_gemm_ws; the workspace's conversion pass is inside
    every timed call)."""
    W0 = synth_weights(n_out, n_in, gen)
    R = copies or copies_for(W0.numel())
    Ws = [W0] + [W0.clone() for _ in range(R - 1)]
    xq = synth_activation_q8(n_in, gen, n_tok)
    y = torch.empty(n_out * n_tok, dtype=torch.float32, device="cuda")
    if n_tok == 1:
        fn = lambda i: B.gemv(Ws[i % R], xq, y, n_out, n_in)  # noqa: E731
    elif ws:
        wsb = torch.empty(max(16, B.gemm_workspace_bytes(n_in, n_tok)), dtype=torch.uint8, device="cuda")
        fn = lambda i: B.gemm_ws(Ws[i % R], xq, y, n_out, n_in, n_tok, wsb)  # noqa: E731
    else:
        fn = lambda i: B.gemm(Ws[i % R], xq, y, n_out, n_in, n_tok)  # noqa: E731
    ms = time_loop(fn, steps, warmup)
    del Ws
    return ms


def bench_stream_read(nbytes, steps, warmup, blocks=8192):
    """Achievable-read ceiling at the GEMV's byte count: bonsai_p40_stream_read
    over rotating buffers of the same size (the analog of tools/bwtest.cu)."""
    nbytes = (nbytes + 255) // 256 * 256
    R = copies_for(nbytes)
    buf = torch.empty(R * nbytes, dtype=torch.uint8, device="cuda")
    out = torch.zeros(blocks, dtype=torch.int32, device="cuda")
    base = buf.data_ptr()
    ms = time_loop(lambda i: B.stream_read(base + (i % R) * nbytes, nbytes, out, blocks), steps, warmup)
    del buf
    return ms


def bench_unit_dma(n_out, n_in, steps, warmup, gen):
    """bonsai_p40_unit_dma_probe: the decode GEMV's unit DMA schedule alone (no
    activation, no arithmetic) over the same rotating weight copies as
    bench_gemv -- the floor the GEMV's own addressing sets."""
    W0 = synth_weights(n_out, n_in, gen)
    R = copies_for(W0.numel())
    Ws = [W0] + [W0.clone() for _ in range(R - 1)]
    sink = torch.zeros(4096, dtype=torch.int32, device="cuda")
    ms = time_loop(lambda i: B.unit_dma_probe(Ws[i % R], n_out, n_in, sink), steps, warmup)
    del Ws
    return ms


def bench_fwht_gemv(n_out, n_in, steps, warmup, gen):
    """bonsai_p40_fwht_gemv: FWHT + Q8_1 of an fp32 activation and the GEMV in
    one launch, over rotating weight copies."""
    W0 = synth_weights(n_out, n_in, gen)
    R = copies_for(W0.numel())
    Ws = [W0] + [W0.clone() for _ in range(R - 1)]
    x = torch.randn(n_in, generator=gen, device="cuda")
    y = torch.empty(n_out, dtype=torch.float32, device="cuda")
    ms = time_loop(lambda i: B.fwht_gemv(Ws[i % R], x, None, y, n_out, n_in), steps, warmup)
    del Ws
    return ms


def bench_gemv_repack(n_out, n_in, steps, warmup, gen):
    """bonsai_p40_gemv_repack (fp32 activation, quantised inside) on weights
    repacked once with bonsai_p40_repack, over rotating copies."""
    W0 = synth_weights(n_out, n_in, gen)
    Wr = torch.empty_like(W0)
    B.repack(W0, Wr, n_out, n_in)
    R = copies_for(Wr.numel())
    Ws = [Wr] + [Wr.clone() for _ in range(R - 1)]
    del W0
    x = torch.randn(n_in, generator=gen, device="cuda")
    y = torch.empty(n_out, dtype=torch.float32, device="cuda")
    ms = time_loop(lambda i: B.gemv_repack(Ws[i % R], x, y, n_out, n_in), steps, warmup)
    del Ws
    return ms


def bench_prepass(n, steps, warmup, gen):
    x = torch.randn(n, generator=gen, device="cuda")
    q = torch.empty(B.q8_bytes(n), dtype=torch.uint8, device="cuda")
    return time_loop(lambda i: B.fwht_quant(x, None, q, n), steps, warmup)


def bench_rms_prepass(n, steps, warmup, gen):
    """Layer-input pre-pass: bonsai_p40_rmsnorm_fwht_quant (one launch) and
    the unfused bonsai_p40_rmsnorm + bonsai_p40_fwht_quant (two launches)."""
    x = torch.randn(n, generator=gen, device="cuda")
    w = torch.randn(n, generator=gen, device="cuda") * 0.1 + 1
    h = torch.empty(n, dtype=torch.float32, device="cuda")
    q = torch.empty(B.q8_bytes(n), dtype=torch.uint8, device="cuda")
    fused = time_loop(lambda i: B.rmsnorm_fwht_quant(x, w, None, q, n, 1, 1e-6), steps, warmup)

    def two(i):
        B.rmsnorm(x, w, h, 1, n, 1e-6)
        B.fwht_quant(h, None, q, n)
    return fused, time_loop(two, steps, warmup)


def bench_ffn_chain(steps, warmup, gen):
    """Config 1: pre-pass, gate + up GEMVs, SwiGLU+FWHT+Q8_1, down GEMV."""
    sets = []
    per = 3 * B.pq2_bytes(N_FF, N_EMBD)
    R = copies_for(per)
    base = [synth_weights(N_FF, N_EMBD, gen), synth_weights(N_FF, N_EMBD, gen),
            synth_weights(N_EMBD, N_FF, gen)]
    for r in range(R):
        sets.append(base if r == 0 else [w.clone() for w in base])
    x = torch.randn(N_EMBD, generator=gen, device="cuda")
    xq = torch.empty(B.q8_bytes(N_EMBD), dtype=torch.uint8, device="cuda")
    hq = torch.empty(B.q8_bytes(N_FF), dtype=torch.uint8, device="cuda")
    g = torch.empty(N_FF, device="cuda")
    u = torch.empty(N_FF, device="cuda")
    y = torch.empty(N_EMBD, device="cuda")

    def step(i):
        Wg, Wu, Wd = sets[i % R]
        B.fwht_quant(x, None, xq, N_EMBD)
        B.gemv(Wg, xq, g, N_FF, N_EMBD)
        B.gemv(Wu, xq, u, N_FF, N_EMBD)
        B.swiglu_fwht_quant(g, u, None, hq, N_FF)
        B.gemv(Wd, hq, y, N_EMBD, N_FF)

    def step_grouped(i):
        Wg, Wu, Wd = sets[i % R]
        B.fwht_gemv_group([Wg, Wu], x, None, [g, u], [N_FF, N_FF], N_EMBD)
        B.swiglu_fwht_quant(g, u, None, hq, N_FF)
        B.gemv(Wd, hq, y, N_EMBD, N_FF)

    def gate_up(i):
        Wg, Wu, _ = sets[i % R]
        B.gemv_group([Wg, Wu], xq, [g, u], [N_FF, N_FF], N_EMBD)

    ms = time_loop(step, steps, warmup)
    ms_grouped = time_loop(step_grouped, steps, warmup)
    ms_gu = time_loop(gate_up, steps, warmup)
    del sets, base
    return ms, per, ms_grouped, ms_gu  # weight bytes per chain


def bench_token_sweep(steps, warmup, gen, mode="separate"):
    """Config 2: 64 layers x (q, k, v, o, gate, up, down) over 5.79 GB of
    distinct weights per token, each GEMV fed by an FWHT+Q8_1 of its input.
    mode "separate": a pre-pass launch before every GEMV (7 + 7 launches per
    layer).  "fused": the rotation inside each GEMV launch
    (bonsai_p40_fwht_gemv), except the 17408-wide down projection, whose
    separate pre-pass is faster.  "grouped": as a model runs it -- q/k/v and
    gate/up share their input, one grouped fused launch each
    (bonsai_p40_fwht_gemv_group), o fused, down with its pre-pass (4 GEMV
    launches + 1 pre-pass per layer).  "layer": as "grouped", with both layer
    inputs RMS-normalised inside the grouped launches
    (bonsai_p40_rmsnorm_fwht_gemv_group) and the down projection fed by the
    SwiGLU + FWHT + Q8_1 pre-pass of the gate/up outputs."""
    shapes = [(Q_DIM, N_EMBD), (KV_DIM, N_EMBD), (KV_DIM, N_EMBD), (N_EMBD, Q_DIM),
              (N_FF, N_EMBD), (N_FF, N_EMBD), (N_EMBD, N_FF)]
    proto = {s: synth_weights(s[0], s[1], gen) for s in set(shapes)}
    layers = [[proto[s].clone() for s in shapes] for _ in range(N_LAYER)]
    xs = {n: torch.randn(n, generator=gen, device="cuda") for n in (N_EMBD, Q_DIM, N_FF)}
    qs = {n: torch.empty(B.q8_bytes(n), dtype=torch.uint8, device="cuda") for n in xs}
    ys = {n: torch.empty(n, device="cuda") for n in (Q_DIM, KV_DIM, N_EMBD, N_FF)}
    wbytes = sum(B.pq2_bytes(*s) for s in shapes) * N_LAYER

    yk, yv, yg, yu = (torch.empty(n, device="cuda") for n in (KV_DIM, KV_DIM, N_FF, N_FF))

    nw = torch.randn(N_EMBD, generator=gen, device="cuda") * 0.1 + 1
    ws = torch.zeros(B.ffn_workspace_bytes(N_FF), dtype=torch.uint8, device="cuda")
    chain = None
    if mode == "chain":
        # the whole token as one persistent launch: per layer q/k/v from the
        # RMS-normalised layer input, o from q, gate/up from the normalised o,
        # the SwiGLU glue, down; the next layer's input is this layer's down
        # output (every step depends on the one before it)
        yd = torch.empty(N_EMBD, device="cuda")
        csteps = []
        x_in = xs[N_EMBD]
        for Wq, Wk, Wv, Wo, Wg, Wu, Wd in layers:
            csteps += [
                B.chain_step(B.CHAIN_RMSNORM_FWHT, [Wq, Wk, Wv], [ys[Q_DIM], yk, yv], [Q_DIM, KV_DIM, KV_DIM],
                             N_EMBD, x=x_in, norm_w=nw, eps=1e-6),
                B.chain_step(B.CHAIN_FWHT, [Wo], [ys[N_EMBD]], [N_EMBD], Q_DIM, x=ys[Q_DIM]),
                B.chain_step(B.CHAIN_RMSNORM_FWHT, [Wg, Wu], [yg, yu], [N_FF, N_FF], N_EMBD, x=ys[N_EMBD],
                             norm_w=nw, eps=1e-6),
                B.chain_step(B.CHAIN_SWIGLU, n_in=N_FF, x=yg, x2=yu, q_out=qs[N_FF]),
                B.chain_step(B.CHAIN_Q8, [Wd], [yd], [N_EMBD], N_FF, x=qs[N_FF]),
            ]
            x_in = yd
        chain = B.Chain(csteps)

    def token(i):
        if chain is not None:
            chain.run()
            return
        for L in layers:
            if mode == "layer_ffn":
                Wq, Wk, Wv, Wo, Wg, Wu, Wd = L
                B.rmsnorm_fwht_gemv_group([Wq, Wk, Wv], xs[N_EMBD], nw, None, [ys[Q_DIM], yk, yv],
                                          [Q_DIM, KV_DIM, KV_DIM], N_EMBD, 1e-6)
                B.fwht_gemv(Wo, xs[Q_DIM], None, ys[N_EMBD], N_EMBD, Q_DIM)
                B.ffn_gate_up_swiglu(Wg, Wu, xs[N_EMBD], nw, None, None, qs[N_FF], N_FF, N_EMBD, 1e-6, ws)
                B.gemv(Wd, qs[N_FF], ys[N_EMBD], N_EMBD, N_FF)
                continue
            if mode == "layer":
                Wq, Wk, Wv, Wo, Wg, Wu, Wd = L
                B.rmsnorm_fwht_gemv_group([Wq, Wk, Wv], xs[N_EMBD], nw, None, [ys[Q_DIM], yk, yv],
                                          [Q_DIM, KV_DIM, KV_DIM], N_EMBD, 1e-6)
                B.fwht_gemv(Wo, xs[Q_DIM], None, ys[N_EMBD], N_EMBD, Q_DIM)
                B.rmsnorm_fwht_gemv_group([Wg, Wu], xs[N_EMBD], nw, None, [yg, yu], [N_FF, N_FF], N_EMBD, 1e-6)
                B.swiglu_fwht_quant(yg, yu, None, qs[N_FF], N_FF)
                B.gemv(Wd, qs[N_FF], ys[N_EMBD], N_EMBD, N_FF)
                continue
            if mode == "grouped":
                Wq, Wk, Wv, Wo, Wg, Wu, Wd = L
                B.fwht_gemv_group([Wq, Wk, Wv], xs[N_EMBD], None, [ys[Q_DIM], yk, yv],
                                  [Q_DIM, KV_DIM, KV_DIM], N_EMBD)
                B.fwht_gemv(Wo, xs[Q_DIM], None, ys[N_EMBD], N_EMBD, Q_DIM)
                B.fwht_gemv_group([Wg, Wu], xs[N_EMBD], None, [yg, yu], [N_FF, N_FF], N_EMBD)
                B.fwht_quant(xs[N_FF], None, qs[N_FF], N_FF)
                B.gemv(Wd, qs[N_FF], ys[N_EMBD], N_EMBD, N_FF)
                continue
            for (n_out, n_in), W in zip(shapes, L):
                if mode == "fused" and n_in != N_FF:
                    B.fwht_gemv(W, xs[n_in], None, ys[n_out], n_out, n_in)
                else:
                    B.fwht_quant(xs[n_in], None, qs[n_in], n_in)
                    B.gemv(W, qs[n_in], ys[n_out], n_out, n_in)

    ms = time_loop(token, steps, warmup, per_graph=1)
    if chain is not None:
        torch.cuda.synchronize()
        if int(chain.status.item()) != 0:
            raise RuntimeError("decode chain: a barrier wait gave up")
    del layers, proto
    return ms, wbytes


def host_cpu():
    """Model and core count of this host, and the threads the baseline uses
    (the job's OMP_NUM_THREADS share where set, else every core)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    nproc = os.cpu_count() or 1
    try:
        nproc = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        pass
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or nproc
    return model, nproc, max(1, min(threads, nproc))


def _timed(fn, seconds):
    t0 = time.perf_counter()
    n = 0
    while True:
        fn()
        n += 1
        if time.perf_counter() - t0 >= seconds:
            break
    return (time.perf_counter() - t0) / n, n


def cpu_baseline(sample_s: float):
    """CPU baseline on this host's cores (a reported baseline, not a target):
    * the reference's own host GEMV (pq2_0_row_dot_perm per row, compiled from
      the reference sources into oracle/_ref; the restatement where _ref is
      absent), single-threaded as the reference runs it;
    * the oracle restatement (bit-identical output) with OpenMP over output
      rows on all of the job's cores: `value`;
    * the GEMM loop of tests/test_p40.cpp:449-470 on a row sample of the
      17408x5120 prefill shape at M = 512, single-threaded and on all cores.
    Same input distribution as the GPU runs; ~sample_s seconds in total."""
    sys.path.insert(0, ROOT)
    import numpy as np
    from oracle import oracle as O
    R = O.ref()
    model, nproc, threads = host_cpu()
    n_out, n_in = N_FF, N_EMBD
    W = O.gen_weights(77, n_out, n_in)
    xq = O.quantize_q8_1(O.fwht(O.gen_normal(78, n_in)), True)
    y = np.empty(n_out, np.float32)
    P = lambda a, t: O._p(a, t)  # noqa: E731
    if R is not None:
        kind1 = "reference"
        one = lambda: R.ref_gemv(P(W, O._u8p), P(xq, O._u8p), P(y, O._f32p), n_out, n_in)  # noqa: E731
    else:
        kind1 = "port"
        one = lambda: O.lib().orc_gemv(P(W, O._u8p), P(xq, O._u8p), P(y, O._f32p), n_out, n_in, 1)  # noqa: E731
    many = lambda: O.lib().orc_gemv(P(W, O._u8p), P(xq, O._u8p), P(y, O._f32p), n_out, n_in, threads)  # noqa: E731
    share = sample_s / 4
    dt1, n1 = _timed(one, share)
    dtn, nn = _timed(many, share)
    gb = gemv_bytes(n_out, n_in)

    # GEMM: 256 rows x 5120 x 512 tokens (the per-(row, token, chunk) loop)
    M, rows = 512, 256
    Xq = O.quantize_chunk_major(np.stack([O.fwht(O.gen_normal(90 + t, n_in)) for t in range(M)]))
    Ws = W[:rows * (n_in // 128) * 34]
    Y = np.empty((rows, M), np.float32)
    if R is not None:
        g1 = lambda: R.ref_gemm(P(Ws, O._u8p), P(Xq, O._u8p), P(Y, O._f32p), rows, n_in, M)  # noqa: E731
    else:
        g1 = lambda: O.lib().orc_gemm(P(Ws, O._u8p), P(Xq, O._u8p), P(Y, O._f32p), rows, n_in, M, 1)  # noqa: E731
    gn = lambda: O.lib().orc_gemm(P(Ws, O._u8p), P(Xq, O._u8p), P(Y, O._f32p), rows, n_in, M, threads)  # noqa: E731
    tg1, _ = _timed(g1, share)
    tgn, _ = _timed(gn, share)
    ops = 2.0 * rows * n_in * M
    return {"value": round(gb / dtn / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "ms_per_gemv": round(dtn * 1e3, 3),
            "sample": f"{nn} host GEMVs of 17408x5120 by the oracle restatement (bit-identical to the "
                      f"reference's pq2_0_row_dot_perm), OpenMP over rows on {threads} threads, "
                      f"{nn * dtn:.1f} s",
            "host": {"cpu_model": model, "nproc": nproc, "threads_used": threads},
            "single_thread": {"value": round(gb / dt1 / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": kind1,
                              "ms_per_gemv": round(dt1 * 1e3, 3),
                              "sample": f"{n1} single-thread host GEMVs of 17408x5120, {n1 * dt1:.1f} s"},
            "gemm_prefill_row_sample": {
                "shape": f"{rows} of 17408 rows x 5120, M = {M} tokens (tests/test_p40.cpp:449-470 loop)",
                "single_thread": {"TOPS": round(ops / tg1 / 1e12, 5), "kind": kind1,
                                  "ms": round(tg1 * 1e3, 2)},
                "all_cores": {"TOPS": round(ops / tgn / 1e12, 5), "kind": "port", "threads": threads,
                              "ms": round(tgn * 1e3, 2)},
                "full_shape_ms_all_cores": round(tgn * 1e3 * n_out / rows, 1)}}


def bench_sustained_read(gb: float = 2.0, reps: int = 5):
    """Sustained HBM read: one launch over a gb-GB buffer with 8 workgroups of
    256 lanes per CU (tools/bwtest.cu:37-47,133), HIP events around each
    launch on the current stream; the best of reps."""
    nbytes = int(gb * (1 << 30)) // 256 * 256
    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    blocks = 8 * cus
    out = torch.zeros(blocks, dtype=torch.int32, device="cuda")
    B.stream_read(buf, nbytes, out, blocks)
    torch.cuda.synchronize()
    best = None
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        B.stream_read(buf, nbytes, out, blocks)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1)
        best = ms if best is None else min(best, ms)
    del buf
    return nbytes, best


def mfma_peak(kind: int, iters: int = 4096, per_cu: int = 4):
    """MFMA peak probe (bonsai_p40_mfma_probe): per_cu 4-wave workgroups per
    CU, each wave iters * 4 independent back-to-back MFMAs.  Returns (TOPS by
    HIP events around the launch, the clock that rate implies at the MFMA's
    documented throughput: 1024 int8 or 512 f16 MACs per SIMD per cycle)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    blocks = per_cu * cus
    clk = torch.zeros(2 * blocks, dtype=torch.int64, device="cuda")
    sink = torch.zeros(blocks, dtype=torch.int32, device="cuda")
    B.mfma_probe(kind, blocks, 64, clk, sink)
    torch.cuda.synchronize()
    best = None
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        B.mfma_probe(kind, blocks, iters, clk, sink)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1)
        if best is None or ms < best[0]:
            best = (ms, clk.cpu())
    ms, _ = best
    ops_per = 32768 if kind == 0 else 16384
    ops = float(blocks) * 4 * iters * 4 * ops_per
    tops = ops / (ms * 1e-3) / 1e12
    ops_per_clk = cus * 4 * (1024 if kind == 0 else 512) * 2
    return tops, tops * 1e12 / ops_per_clk / 1e6


def valu_mfma_overlap(iters: int = 4096, per_cu: int = 4,
                      modes=(("mfma_only", 0), ("fma_only", 1), ("both", 2), ("gemm_core", 3))):
    """bonsai_p40_overlap_probe at per_cu waves per SIMD (per_cu 4-wave
    workgroups per CU): ms for 4 f16 MFMAs per iteration alone, 16 fp32 FMAs
    alone (4 per MFMA: the prefill GEMM's rescale ratio), both in one wave
    stream, and the GEMM's chunk step."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    blocks = per_cu * cus
    sink = torch.zeros(blocks, dtype=torch.int32, device="cuda")
    out = {}
    for name, mode in modes:
        B.overlap_probe(mode, 1, blocks, 64, sink)
        torch.cuda.synchronize()
        best = None
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            B.overlap_probe(mode, 1, blocks, iters, sink)
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1)
            best = ms if best is None else min(best, ms)
        out[name + "_us"] = round(best * 1e3, 2)
    if "both_us" in out:
        out["both_over_sum"] = round(out["both_us"] / (out["mfma_only_us"] + out["fma_only_us"]), 3)
        out["both_over_max"] = round(out["both_us"] / max(out["mfma_only_us"], out["fma_only_us"]), 3)
    # the GEMM's chunk step alone: iters steps per wave, 4 waves per SIMD, each
    # step a 32 x 32 x 32 piece of the product; scaled to the M = 2048
    # 17408x5120 prefill (5,570,560 such pieces over the CUs' SIMDs)
    per_piece_ns = out["gemm_core_us"] * 1e3 / (iters * per_cu)
    pieces = 2048 * N_FF * N_EMBD / 32768
    out["gemm_core_ns_per_32x32x32_per_simd"] = round(per_piece_ns, 2)
    out["gemm_core_floor_us_m2048_17408x5120"] = round(per_piece_ns * pieces / (4 * cus) / 1e3, 1)
    return out


def launch_floor(steps: int = 200):
    """us per launch of an empty kernel (256 workgroups of 64 threads) in a
    HIP graph of back-to-back launches: what any launch that depends on the
    one before it costs on this GPU, the floor under every decode kernel."""
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    ms = time_loop(lambda i: B.launch_probe(256, 64, sink), steps, 10)
    return ms * 1e3


def kernel_source_hash():
    """sha256 over the device sources that build the decode GEMV kernel: a
    traffic figure measured on another build of them is not reported."""
    import hashlib
    h = hashlib.sha256()
    for f in ("gemv.hip", "gemv_device.h", "pq2_device.h", "fwht_device.h"):
        with open(os.path.join(ROOT, "p40-kernel_amd", "csrc", f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def load_traffic(path):
    """The PMC traffic record of the decode GEMV kernel, if it was measured on
    the current kernel sources (else None and the reason)."""
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None, "no PMC record"
    if t.get("source_sha256") != kernel_source_hash():
        return None, "PMC record measured on other kernel sources"
    return t, None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--quick", action="store_true", help="headline only (no secondary configs)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=16.0)
    ap.add_argument("--only-gemv", action="store_true", help="headline GEMV loop only (profiling)")
    ap.add_argument("--eager", action="store_true",
                    help="time Python launches one by one instead of replaying HIP graphs")
    ap.add_argument("--only-read", action="store_true",
                    help="stream-read probe over 23,750,272-byte buffers only (PMC calibration)")
    ap.add_argument("--shape", default=f"{N_FF}x{N_EMBD}", metavar="ROWSxCOLS",
                    help="matrix of --only-gemm / --only-small (default the headline 17408x5120)")
    ap.add_argument("--ws", action="store_true", help="--only-gemm through bonsai_p40_gemm_ws")
    ap.add_argument("--only-gemm", type=int, default=0, metavar="M",
                    help="prefill GEMM 17408x5120 with M tokens only (profiling)")
    ap.add_argument("--only-small", type=int, default=0, metavar="B",
                    help="small-batch GEMM 17408x5120 with B tokens only (profiling)")
    ap.add_argument("--only-fused", action="store_true",
                    help="fused FWHT+Q8_1+GEMV 17408x5120 from fp32 only (profiling)")
    ap.add_argument("--only-probes", action="store_true",
                    help="MFMA peak and VALU/MFMA overlap probes only (profiling)")
    ap.add_argument("--only-sweep", default="", metavar="MODE", choices=["", "separate", "fused", "grouped", "layer", "layer_ffn", "chain"],
                    help="config-2 token sweep in one mode only (profiling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the PQ2_0 path would shard by weight rows, with the activation "
              "replicated and the outputs all-gathered)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        sys.exit(1)
    B.lib()
    global GRAPH
    GRAPH = not args.eager
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1234)

    if args.only_probes:
        for kind in (0, 1):
            print(f"[bench] mfma peak kind {kind}: {mfma_peak(kind)}", flush=True)
        print(f"[bench] valu/mfma overlap: {valu_mfma_overlap()}", flush=True)
        for per_cu in (1, 2, 3, 4, 8):
            core = valu_mfma_overlap(per_cu=per_cu, modes=(("gemm_core", 3),))
            print(f"[bench] gemm core at {per_cu} waves per SIMD: "
                  f"{core['gemm_core_floor_us_m2048_17408x5120']} us floor (17408x5120, M = 2048)", flush=True)
        print(f"[bench] dependent launch floor: {launch_floor():.3f} us", flush=True)
        return
    if args.only_read:
        ms = bench_stream_read(gemv_bytes(N_FF, N_EMBD), args.steps, args.warmup)
        print(f"[bench] stream_read 23750272 B: {ms * 1e3:.2f} us", file=sys.stderr, flush=True)
        z = torch.empty(23750400 // 4, dtype=torch.float32, device="cuda")
        for _ in range(args.steps):
            z.zero_()              # writes 23,750,400 B: WRITE_SIZE calibration
        torch.cuda.synchronize()
        return

    if args.only_gemm or args.only_small:
        m = args.only_gemm or args.only_small
        no, ni = map(int, args.shape.split("x"))
        ms = bench_gemv(no, ni, args.steps, args.warmup, gen, n_tok=m, ws=args.ws)
        if args.only_gemm:
            tops = 2.0 * m * no * ni / (ms * 1e-3) / 1e12
            print(f"[bench] gemm {no}x{ni} M={m}: {ms * 1e3:.1f} us  {tops:.1f} TOPS", file=sys.stderr, flush=True)
        else:
            gbs = gemv_bytes(no, ni, m) / (ms * 1e-3) / 1e9
            print(f"[bench] small batch {no}x{ni} B={m}: {ms * 1e3:.2f} us  {gbs:.1f} GB/s", file=sys.stderr, flush=True)
        return

    if args.only_sweep:
        ms, wb = bench_token_sweep(max(1, args.steps), min(args.warmup, 2), gen, mode=args.only_sweep)
        print(f"[bench] token sweep {args.only_sweep}: {ms:.3f} ms/token  {wb / (ms * 1e-3) / 1e9:.1f} GB/s",
              file=sys.stderr, flush=True)
        return

    if args.only_fused:
        ms = bench_fwht_gemv(N_FF, N_EMBD, args.steps, args.warmup, gen)
        print(f"[bench] fwht_gemv 17408x5120: {ms * 1e3:.2f} us", file=sys.stderr, flush=True)
        return

    # ---- headline: decode GEMV 17408x5120
    ms = bench_gemv(N_FF, N_EMBD, args.steps, args.warmup, gen)
    nbytes = gemv_bytes(N_FF, N_EMBD)
    gbs = nbytes / (ms * 1e-3) / 1e9
    print(f"[bench] gemv 17408x5120: {ms * 1e3:.2f} us  {gbs:.1f} GB/s", file=sys.stderr, flush=True)
    if args.only_gemv:
        return

    extra = {"timing": "HIP graph replay of back-to-back launches" if GRAPH else "eager Python launches"}
    if GRAPH:
        W0 = synth_weights(N_FF, N_EMBD, gen)
        Rc = copies_for(W0.numel())
        Ws = [W0] + [W0.clone() for _ in range(Rc - 1)]
        xq = synth_activation_q8(N_EMBD, gen)
        yv = torch.empty(N_FF, device="cuda")
        me = time_loop_eager(lambda i: B.gemv(Ws[i % Rc], xq, yv, N_FF, N_EMBD), args.steps, args.warmup)
        extra["gemv_17408x5120_eager_python_launch"] = {"us": round(me * 1e3, 3),
                                                        "GB/s": round(nbytes / (me * 1e-3) / 1e9, 1)}
        del Ws, W0
    mw = bench_gemv(N_FF, N_EMBD, args.steps, args.warmup, gen, copies=1)
    extra["gemv_17408x5120_warm"] = {
        "us": round(mw * 1e3, 3), "GB/s": round(nbytes / (mw * 1e-3) / 1e9, 1),
        "note": "one weight copy reused by every launch: its 23.75 MB stay in the 256 MB MALL, so this "
                "is not HBM bandwidth (value rotates >= 1.1 GB of copies, cold)"}
    print(f"[bench] gemv warm: {extra['gemv_17408x5120_warm']}", file=sys.stderr, flush=True)
    ms_read = bench_stream_read(nbytes, args.steps, args.warmup)
    read_gbs = nbytes / (ms_read * 1e-3) / 1e9
    extra["stream_read_same_bytes"] = {"us": round(ms_read * 1e3, 3), "GB/s": round(read_gbs, 1),
                                       "note": "plain 16-byte streaming read of 23,750,272 B per launch: "
                                               "the achievable ceiling for one launch of this size"}
    print(f"[bench] stream read ceiling: {extra['stream_read_same_bytes']}", file=sys.stderr, flush=True)
    for (no, ni) in ((N_FF, N_EMBD), (N_EMBD, N_FF)):
        ms_dma = bench_unit_dma(no, ni, args.steps, args.warmup, gen)
        nb_ = B.pq2_bytes(no, ni)
        extra[f"gemv_unit_dma_skeleton_{no}x{ni}"] = {
            "us": round(ms_dma * 1e3, 3), "GB/s": round(nb_ / (ms_dma * 1e-3) / 1e9, 1),
            "note": "bonsai_p40_unit_dma_probe: the GEMV's own weight DMA schedule (units, grid, ring, waits) "
                    "with no activation and no arithmetic"}
        print(f"[bench] unit DMA skeleton {no}x{ni}: {extra[f'gemv_unit_dma_skeleton_{no}x{ni}']}",
              file=sys.stderr, flush=True)
    sb, sms = bench_sustained_read()
    sus_gbs = sb / (sms * 1e-3) / 1e9
    extra["stream_read_sustained"] = {"bytes": sb, "us": round(sms * 1e3, 1), "GB/s": round(sus_gbs, 1),
                                      "frac_hbm_peak": round(sus_gbs / HBM_PEAK_GBS, 4),
                                      "note": "one launch over 2 GiB, 8 workgroups per CU: sustained HBM read"}
    print(f"[bench] sustained read: {extra['stream_read_sustained']}", file=sys.stderr, flush=True)
    peaks = {}
    for kind, name in ((0, "int8"), (1, "f16")):
        tops, mhz = mfma_peak(kind)
        peaks[name] = {"TOPS": round(tops, 1), "implied_clock_MHz": round(mhz, 0)}
    extra["mfma_peak_probe"] = {
        **peaks, "published_dense": {"int8": INT8_PEAK_TOPS, "f16": 2500.0},
        "note": "back-to-back independent v_mfma_i32_16x16x64_i8 / v_mfma_f32_16x16x32_f16, "
                "16 waves per CU; implied clock = measured rate / (CUs x 4 SIMDs x the instruction's "
                "documented MACs per cycle x 2)"}
    print(f"[bench] mfma peak: {extra['mfma_peak_probe']}", file=sys.stderr, flush=True)
    extra["valu_mfma_overlap"] = dict(valu_mfma_overlap(), note=(
        "4 independent v_mfma_f32_16x16x32_f16 and 16 independent fp32 FMAs per iteration per wave, "
        "4 waves per SIMD: both_over_sum near 1 means the VALU and the matrix core take turns"))
    print(f"[bench] valu/mfma overlap: {extra['valu_mfma_overlap']}", file=sys.stderr, flush=True)
    extra["dependent_launch_floor_us"] = round(launch_floor(), 3)
    print(f"[bench] dependent launch floor: {extra['dependent_launch_floor_us']} us", file=sys.stderr, flush=True)
    if not args.quick:
        for (n_out, n_in, tag) in ((N_EMBD, N_FF, "gemv_5120x17408"), (N_EMBD, N_EMBD, "gemv_5120x5120")):
            m = bench_gemv(n_out, n_in, args.steps, args.warmup, gen)
            extra[tag] = {"us": round(m * 1e3, 3), "GB/s": round(gemv_bytes(n_out, n_in) / (m * 1e-3) / 1e9, 1)}
            print(f"[bench] {tag}: {extra[tag]}", file=sys.stderr, flush=True)
        for n in (N_EMBD, N_FF):
            m = bench_prepass(n, args.steps, args.warmup, gen)
            extra[f"fwht_quant_{n}_us"] = round(m * 1e3, 3)
            mf, m2 = bench_rms_prepass(n, args.steps, args.warmup, gen)
            extra[f"rmsnorm_fwht_quant_{n}"] = {"us": round(mf * 1e3, 3), "unfused_us": round(m2 * 1e3, 3),
                                                "note": "fused RMSNorm+FWHT+Q8_1 vs rmsnorm then fwht_quant"}
            print(f"[bench] rmsnorm_fwht_quant {n}: {extra[f'rmsnorm_fwht_quant_{n}']}", file=sys.stderr,
                  flush=True)
        for (n_out, n_in) in ((N_FF, N_EMBD), (N_EMBD, N_FF)):
            m = bench_gemv_repack(n_out, n_in, args.steps, args.warmup, gen)
            extra[f"gemv_repack_{n_out}x{n_in}"] = {
                "us": round(m * 1e3, 3), "weight_GB/s": round(gemv_bytes(n_out, n_in) / (m * 1e-3) / 1e9, 1),
                "note": "repacked weights, fp32 activation quantised inside (bonsai_p40_gemv_repack)"}
            print(f"[bench] gemv_repack {n_out}x{n_in}: {extra[f'gemv_repack_{n_out}x{n_in}']}",
                  file=sys.stderr, flush=True)
        for (n_out, n_in) in ((N_FF, N_EMBD), (N_EMBD, N_FF)):
            m = bench_fwht_gemv(n_out, n_in, args.steps, args.warmup, gen)
            extra[f"fwht_gemv_{n_out}x{n_in}"] = {
                "us": round(m * 1e3, 3), "weight_GB/s": round(gemv_bytes(n_out, n_in) / (m * 1e-3) / 1e9, 1),
                "note": "fp32 activation in: FWHT + Q8_1 + GEMV in one launch (bonsai_p40_fwht_gemv)"}
            print(f"[bench] fwht_gemv {n_out}x{n_in}: {extra[f'fwht_gemv_{n_out}x{n_in}']}",
                  file=sys.stderr, flush=True)
        m, wb, mg, mgu = bench_ffn_chain(max(20, args.steps // 4), 5, gen)
        extra["ffn_chain_config1"] = {"us": round(m * 1e3, 2), "weight_GB/s": round(wb / (m * 1e-3) / 1e9, 1),
                                      "note": "pre-pass, gate GEMV, up GEMV, SwiGLU+FWHT+Q8_1, down GEMV"}
        extra["ffn_chain_config1_grouped"] = {
            "us": round(mg * 1e3, 2), "weight_GB/s": round(wb / (mg * 1e-3) / 1e9, 1),
            "note": "gate+up as one fused grouped launch from fp32 x, SwiGLU+FWHT+Q8_1, down GEMV"}
        gu_bytes = 2 * gemv_bytes(N_FF, N_EMBD) - B.q8_bytes(N_EMBD)
        extra["gemv_group_gate_up_2x17408x5120"] = {
            "us": round(mgu * 1e3, 3), "GB/s": round(gu_bytes / (mgu * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round(gu_bytes / (mgu * 1e-3) / 1e9 / 8000.0, 4),
            "note": "config 1's gate and up GEMVs as one grouped launch (bonsai_p40_gemv_group)"}
        print(f"[bench] ffn chain: {extra['ffn_chain_config1']}", file=sys.stderr, flush=True)
        print(f"[bench] ffn chain grouped: {extra['ffn_chain_config1_grouped']}", file=sys.stderr, flush=True)
        print(f"[bench] gate+up grouped: {extra['gemv_group_gate_up_2x17408x5120']}", file=sys.stderr, flush=True)
        m, wb = bench_token_sweep(5, 2, gen)
        extra["token_sweep_config2"] = {"ms_per_token": round(m, 3), "tok/s": round(1e3 / m, 2),
                                        "weight_GB/s": round(wb / (m * 1e-3) / 1e9, 1),
                                        "weight_bytes": wb}
        print(f"[bench] token sweep: {extra['token_sweep_config2']}", file=sys.stderr, flush=True)
        for mode, note in (("fused", "FWHT+Q8_1 inside each GEMV launch (down: separate pre-pass)"),
                           ("grouped", "q/k/v and gate/up as grouped fused launches, o fused, "
                                       "down with its pre-pass: 4 GEMV launches + 1 pre-pass per layer"),
                           ("layer", "as grouped, with both layer RMSNorms inside the grouped launches "
                                     "and SwiGLU+FWHT+Q8_1 of the gate/up outputs feeding down"),
                           ("layer_ffn", "as layer, with the SwiGLU+FWHT+Q8_1 glue inside the gate/up launch "
                                         "(bonsai_p40_ffn_gate_up_swiglu): 4 launches per layer"),
                           ("chain", "as layer, each step fed by the one before it, the whole token as ONE "
                                     "persistent launch (bonsai_p40_chain_run: 320 steps, grid barriers, the next "
                                     "step's weights prefetched through each barrier)")):
            m, wb = bench_token_sweep(5, 2, gen, mode=mode)
            extra[f"token_sweep_config2_{mode}"] = {"ms_per_token": round(m, 3), "tok/s": round(1e3 / m, 2),
                                                    "weight_GB/s": round(wb / (m * 1e-3) / 1e9, 1),
                                                    "note": note}
            print(f"[bench] token sweep {mode}: {extra[f'token_sweep_config2_{mode}']}", file=sys.stderr,
                  flush=True)
        for bt in (2, 4, 8):
            for (n_out, n_in) in ((N_FF, N_EMBD), (N_EMBD, N_FF)):
                m = bench_gemv(n_out, n_in, max(20, args.steps // 2), 10, gen, n_tok=bt)
                extra[f"small_batch_B{bt}_{n_out}x{n_in}"] = {
                    "us": round(m * 1e3, 2), "GB/s": round(gemv_bytes(n_out, n_in, bt) / (m * 1e-3) / 1e9, 1)}
        print(f"[bench] small batch done", file=sys.stderr, flush=True)
        for M in (512, 2048):
            for (n_out, n_in) in ((N_FF, N_EMBD), (N_EMBD, N_FF)):
                m = bench_gemv(n_out, n_in, 10, 3, gen, n_tok=M, ws=True)
                m0 = bench_gemv(n_out, n_in, 10, 3, gen, n_tok=M)
                tops = 2.0 * M * n_out * n_in / (m * 1e-3) / 1e12
                extra[f"prefill_M{M}_{n_out}x{n_in}"] = {
                    "us": round(m * 1e3, 1), "TOPS": round(tops, 1),
                    "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                    "frac_int8_probe": round(tops / peaks["int8"]["TOPS"], 4),
                    "us_without_workspace": round(m0 * 1e3, 1),
                    "note": "bonsai_p40_gemm_ws (its activation conversion pass included); "
                            "us_without_workspace: bonsai_p40_gemm, the reference's signature"}
                print(f"[bench] prefill M={M} {n_out}x{n_in}: {extra[f'prefill_M{M}_{n_out}x{n_in}']}",
                      file=sys.stderr, flush=True)

    traffic, why = load_traffic(os.path.join(ROOT, "profiles", "gemv_17408x5120_traffic.json"))
    roof = {"bound": "hbm", "kernel": "gemv_nb_kernel<40, 2, 8> (bonsai_p40_gemv)",
            "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "frac_of_achievable": round(gbs / sus_gbs, 4),
            "frac_of_single_launch_read": round(gbs / read_gbs, 4),
            "traffic": traffic.get("bytes_per_launch") if traffic else None,
            "traffic_source": (f"profiles/gemv_17408x5120_traffic.json (kernel sources {traffic['source_sha256']})"
                               if traffic else why),
            "algorithmic_bytes": nbytes}
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_seconds)
        print(f"[bench] cpu baseline: {cpu}", file=sys.stderr, flush=True)

    line = {
        "metric": "PQ2_0 decode GEMV GB/s (% HBM peak) at 17408x5120; prefill GEMM int8 TOPS",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded PQ2_0 codes/scales of config 0 distribution; N(0,1) -> FWHT -> Q8_1)",
        "config": {"workload": "decode GEMV 17408x5120 PQ2_0 x Q8_1 (config 1 gate/up), batch 1, "
                               f"weights rotated over {copies_for(B.pq2_bytes(N_FF, N_EMBD))} HBM copies",
                   "n_out": N_FF, "n_in": N_EMBD, "bytes_per_step": nbytes},
        "roofline": roof,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
