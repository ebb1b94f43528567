"""GDN hot-path benchmark on one MI355X (prints ONE JSON line).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

Headline (``value``): config 1, Qwen3-Next GDN chunked prefill (B=1,
T=8192, 16 qk-heads -> 32 v-heads, K=V=128, bf16 q/k/v, fp32 g/beta/state,
initial state, output_final_state=True) in tokens/s.  A step is one
``chunk_gated_delta_rule`` call over the whole 8192-token batch, launched
eagerly K times in a row between two ``torch.cuda.synchronize()`` calls and
timed with events on the stream the kernels run on (the host enqueues a call
in far less time than the GPU runs it, so the kernels run back to back;
``host_enqueue_ms_per_step`` reports it).  Inputs are resident in HBM before
timing starts.  Every timed region follows CLOCK_WARMUP_MS of untimed calls
(the GPU's clocks ramp up over the first ~20 ms of load after idle); the
same K steps measured right after the W warmup steps, without it, are
``ms_per_step_after_idle``.

Secondary (``decode``): config 2, batch-256 fused-recurrent decode with the
fp32 state [256, 32, 128, 128] updated in place, 1000 consecutive steps
cycling a pool of 10 pre-generated q/k/v/g/beta sets; GB/s over
1,080,098,816 algorithmic bytes per step.

``layer_ops``: the layer's neighbours of the core (causal conv1d prefill and
decode update, gating, l2norm, gated RMSNorm, decode over a state-slot pool)
at the Qwen3-Next layer shape, each as GB/s over its algorithmic bytes per
launch (20 launches in one HIP graph, median of 5 replays).

``cpu_baseline``: the C/OpenMP fp32 oracle (oracle/gdn_cpu.c, a port, not the
reference: the reference has no GDN code) timed on this host's cores.
Methodology follows the reference's GEMM benchmark
(benchmark/gemm/bench_amdgpu_gemm.py:36-52: warm up, then events around the
timed launches), the decode and backward lines replaying HIP graphs of
several calls; the headline launches eagerly, because replaying a graph of
one call per step adds ~5 us of graph-launch turnover between steps (0.176
against 0.171 ms per call on one box; a graph of four calls measures 0.172).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "GDN prefill tokens/s at Qwen3-Next shape; decode state-update GB/s vs HBM peak"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
C = 64


def prefill_flops(T, Hv, K=128, V=128):
    """Algorithmic flops of the chunked prefill: (6CK + 4CV + 6KV) per token per v-head."""
    return (6 * C * K + 4 * C * V + 6 * K * V) * T * Hv


def backward_flops(T, Hv, K=128, V=128):
    """Flops of one gdn_chunk_bwd call: (16KV + 12CV + 18CK + 4C^2) per token per v-head.

    Per chunk and v-head: the forward recomputation (K K^T, Q K^T in the prep;
    K S, Tb Y, K^T U in the saving chain: 4CKV + 2C^2V + 4C^2K), the reverse
    chain (K dS', P^T dO, Tb^T dd, K^T Z, Q^T dO: 6CKV + 4C^2V) and the
    gradient kernel (dO S^T, dd S^T, d dS'^T: 6CKV; dO d^T, dd V^T, T^T dd:
    6C^2V; R2 K^T, T^T dW, M K, M^T K, MP K, MP^T Q: 12C^2K; dT T^T and
    T^T M1: 4C^3; K K^T and Q K^T once per qk-head: 2C^2K per v-head at G = 2).
    hi/lo split passes are not counted.
    """
    return (16 * K * V + 12 * C * V + 18 * C * K + 4 * C * C) * T * Hv


def decode_bytes(N, Hqk, Hv, K=128, V=128):
    """State read + write (fp32) plus q, k, v, o (bf16) and g, beta (fp32) per step."""
    return 2 * N * Hv * K * V * 4 + N * (2 * Hqk * K + 2 * Hv * V) * 2 + N * Hv * 2 * 4


TRAFFIC_SOURCE = ("profiles/traffic.json: HBM bytes per launch from two rocprofv3 --pmc runs "
                  "(FETCH_SIZE, WRITE_SIZE) of bench.py --profile-pass, each scaled by a 256 MiB "
                  "copy in the same run (bench.py --pmc-summary); not measured in this run")


def _load_traffic(name):
    """HBM bytes per launch measured by rocprofv3 --pmc (profiles/traffic.json), if present."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(name)
    except (OSError, ValueError):
        return None


# Untimed load before every timed region.  MI355X clocks ramp up over the
# first ~20 ms of load after an idle gap: 40 config-1 prefill calls straight
# after 50 ms of idle averaged 0.166 ms per call, the same 40 calls under
# steady load 0.148 ms, and 200 calls from idle 0.152 ms.  The reference's
# GEMM benchmark warms up "to JIT-compile and stabilize clocks"
# (benchmark/gemm/bench_amdgpu_gemm.py:31-34); this does the same by time
# rather than by count, so that every figure is the steady state of a GPU
# running a model, not its ramp-up.  The headline also reports the K steps
# measured straight after the W warmup steps, before this warm-up.
CLOCK_WARMUP_MS = 150.0


def _clock_warmup(dev, fn, ms=CLOCK_WARMUP_MS):
    """Run ``fn`` back to back, untimed, until ``ms`` of wall time have passed."""
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    n = 0
    while True:
        fn()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize(dev)
            if time.perf_counter() - t0 >= ms * 1e-3:
                break
    torch.cuda.synchronize(dev)


def bench_prefill(dev, steps, warmup, l2norm=False):
    from avelang_amd import chunk_gated_delta_rule, chunk_workspace_bytes
    from avelang_amd import workloads as W

    wl = W.config("cfg1_prefill_qwen3next", seed=1)
    d = wl.dims
    t = wl.torch(dev)
    B, T, Hqk, Hv, K, V, N = (d[x] for x in ("B", "T", "Hqk", "Hv", "K", "V", "N"))
    ws = torch.empty(chunk_workspace_bytes(B, T, Hqk, Hv, K, V, N, False, l2norm),
                     dtype=torch.uint8, device=dev)
    o = torch.empty_like(t["v"])
    ht = torch.empty((N, Hv, K, V), dtype=torch.float32, device=dev)

    def call():
        chunk_gated_delta_rule(t["q"], t["k"], t["v"], t["g"], t["beta"],
                               initial_state=t["initial_state"], output_final_state=True,
                               workspace=ws, out=o, final_state=ht,
                               use_qk_l2norm_in_kernel=l2norm)

    stream = torch.cuda.current_stream(dev)

    def timed():
        # W warmup steps, then exactly K timed steps between synchronizations
        for _ in range(warmup):
            call()
        torch.cuda.synchronize(dev)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        w0 = time.perf_counter()
        e0.record(stream)
        for _ in range(steps):
            call()
        e1.record(stream)
        enq = time.perf_counter() - w0
        torch.cuda.synchronize(dev)
        wall = time.perf_counter() - w0
        return e0.elapsed_time(e1) / steps, wall * 1e3 / steps, enq * 1e3 / steps

    cold, _, _ = timed()
    _clock_warmup(dev, call)
    ms, wall_ms, enq_ms = timed()
    return dict(ms=ms, ms_after_idle=cold, wall_ms=wall_ms, enqueue_ms=enq_ms, T=T, Hv=Hv,
                K=K, V=V, wl=wl)


def bench_backward(dev, steps, warmup):
    """Graph replay of one gdn_chunk_bwd call at config 1 (dO ~ N(0,1) bf16, dht 0.01 N(0,1))."""
    from avelang_amd import chunk_bwd_workspace_bytes, chunk_gated_delta_rule_bwd
    from avelang_amd import workloads as W

    wl = W.config("cfg1_prefill_qwen3next", seed=1)
    d = wl.dims
    t = wl.torch(dev)
    B, T, Hqk, Hv, K, V, N = (d[x] for x in ("B", "T", "Hqk", "Hv", "K", "V", "N"))
    gen = torch.Generator(device=dev).manual_seed(11)
    do = torch.randn((B, T, Hv, V), generator=gen, device=dev).to(torch.bfloat16)
    dht = 0.01 * torch.randn((N, Hv, K, V), generator=gen, device=dev)
    ws = torch.empty(chunk_bwd_workspace_bytes(B, T, Hqk, Hv, K, V, N, False),
                     dtype=torch.uint8, device=dev)

    def call():
        chunk_gated_delta_rule_bwd(t["q"], t["k"], t["v"], t["g"], t["beta"], do, dht,
                                   initial_state=t["initial_state"], workspace=ws)

    launches = max(steps // 5, 1)
    ms = _time_graph(dev, call, launches=launches, reps=5)

    # training step: the forward that keeps the backward's inputs, and the
    # backward from that workspace (no recomputation)
    from avelang_amd import chunk_gated_delta_rule_fwd_save
    o = torch.empty_like(t["v"])

    def fwd_save():
        chunk_gated_delta_rule_fwd_save(t["q"], t["k"], t["v"], t["g"], t["beta"],
                                        initial_state=t["initial_state"],
                                        output_final_state=True, workspace=ws)

    def bwd_saved():
        chunk_gated_delta_rule_bwd(t["q"], t["k"], t["v"], t["g"], t["beta"], do, dht,
                                   initial_state=t["initial_state"], workspace=ws, saved=True)

    ms_fs = _time_graph(dev, fwd_save, launches=launches, reps=5)
    fwd_save()
    ms_bs = _time_graph(dev, bwd_saved, launches=launches, reps=5)
    return dict(ms=ms, ms_fwd_save=ms_fs, ms_bwd_saved=ms_bs, T=T, Hv=Hv, K=K, V=V, wl=wl,
                ws_bytes=ws.numel())


def cpu_backward(wl, runs=3):
    """The fp32 numpy chunked backward oracle on config 1 in full (median of ``runs``)."""
    from threadpoolctl import threadpool_info

    from oracle import gdn_bwd_ref as RB

    a = wl.numpy()
    rng = np.random.Generator(np.random.PCG64(5))
    T, Hv = wl.dims["T"], wl.dims["Hv"]
    do = rng.standard_normal((1, T, Hv, wl.dims["V"]), dtype=np.float32)
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        RB.chunked_bwd(a["q"], a["k"], a["v"], a["g"], a["beta"], do, None,
                       initial_state=a["initial_state"], dtype=np.float32)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    from oracle import cpu as oracle

    threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    host = oracle.host_info(threads)
    host["compiler"], host["cflags"] = "numpy (BLAS)", None
    return dict(value=T / med, unit="tokens/s", cores=threads, kind="port",
                implementation="numpy",
                sample=f"config 1 in full (T={T}, {Hv} v-heads), numpy fp32 chunked backward "
                       f"oracle (oracle/gdn_bwd_ref.py; threads = the BLAS pool's), median of "
                       f"{runs} runs ({med:.2f} s each)",
                host=host)


# Workload seeds of the extra prefill lines.  Config 3's lengths are drawn
# uniform in [128, 4096] from the seed; seed 5 gives 134,847 tokens, the
# draw of seeds 0-11 closest to the ~134k the configuration names (seed 1,
# used before, gave 116,494).
EXTRA_SEEDS = {"cfg3_varlen_64seq": 5, "cfg4_long_context": 1}


def bench_prefill_config(dev, name, reps=3):
    """One eager call per repetition of another prefill config (median ms)."""
    from avelang_amd import chunk_gated_delta_rule
    from avelang_amd import workloads as W

    wl = W.config(name, seed=EXTRA_SEEDS.get(name, 1))
    t = wl.torch(dev)

    def call():
        return chunk_gated_delta_rule(t["q"], t["k"], t["v"], t["g"], t["beta"],
                                      initial_state=t["initial_state"], output_final_state=True,
                                      cu_seqlens=t["cu_seqlens"])
    _clock_warmup(dev, call)
    stream = torch.cuda.current_stream(dev)
    times = []
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        call()
        e1.record(stream)
        torch.cuda.synchronize(dev)
        times.append(e0.elapsed_time(e1))
    ms = float(np.median(times))
    d = wl.dims
    tokens = d["B"] * d["T"]
    flops = prefill_flops(tokens, d["Hv"], d["K"], d["V"])
    return {"workload": name, "tokens": tokens, "sequences": d["N"], "ms": round(ms, 3),
            "value": round(tokens / (ms * 1e-3), 1), "unit": "tokens/s",
            "roofline_frac": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)}


def bench_decode(dev, nsteps=1000, pool=10):
    from avelang_amd import fused_recurrent_gated_delta_rule
    from avelang_amd import workloads as W

    sets = [W.config("cfg2_decode_b256", seed=200 + i) for i in range(pool)]
    d = sets[0].dims
    N, Hqk, Hv, K, V = (d[x] for x in ("N", "Hqk", "Hv", "K", "V"))
    ins = [s.torch(dev) for s in sets]
    state = ins[0]["initial_state"].clone()
    outs = [torch.empty_like(x["v"]) for x in ins]

    def step(i):
        x = ins[i % pool]
        fused_recurrent_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"],
                                         initial_state=state, output_final_state=True,
                                         inplace_final_state=True, out=outs[i % pool])

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for i in range(pool):
            step(i)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(pool):
            step(i)
    reps = nsteps // pool
    _clock_warmup(dev, graph.replay)
    stream = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize(dev)
    ms = e0.elapsed_time(e1) / (reps * pool)
    return dict(ms=ms, bytes=decode_bytes(N, Hqk, Hv, K, V), N=N, Hqk=Hqk, Hv=Hv, K=K, V=V,
                steps=reps * pool)


def _time_graph(dev, fn, launches=20, reps=5):
    """Median per-launch ms of ``fn`` captured ``launches`` times in one HIP graph."""
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(launches):
            fn()
    _clock_warmup(dev, graph.replay)
    stream = torch.cuda.current_stream(dev)
    times = []
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        graph.replay()
        e1.record(stream)
        torch.cuda.synchronize(dev)
        times.append(e0.elapsed_time(e1) / launches)
    return float(np.median(times))


def bench_fusions(dev):
    """The layer's gating fused into the core against the two-step sequence
    (fused_gdn_gating, then the core), per layer call: config 1 prefill and
    config 2 decode (state in place), a / b bf16 [B, T, Hv], A_log / dt_bias
    fp32.  Bytes saved per (token, v-head): the gating kernel's a, b reads
    (4) and g, beta writes (8), and the core's g, beta reads (8), less the
    fused core's a, b reads (4) = 16."""
    from avelang_amd import (chunk_gated_delta_rule, chunk_gated_delta_rule_gated,
                             chunk_workspace_bytes, fused_gdn_gating,
                             fused_recurrent_gated_delta_rule,
                             fused_recurrent_gated_delta_rule_gated)
    from avelang_amd import workloads as W

    def gates(B, T, Hv, seed):
        gen = torch.Generator(device="cpu").manual_seed(seed)
        a = torch.randn((B, T, Hv), generator=gen).to(dev, torch.bfloat16)
        b = torch.randn((B, T, Hv), generator=gen).to(dev, torch.bfloat16)
        A_log = torch.log(torch.empty(Hv).uniform_(0.5, 8.0, generator=gen)).to(dev)
        dt_bias = torch.ones(Hv, device=dev)
        return a, b, A_log, dt_bias

    out = {}
    wl = W.config("cfg1_prefill_qwen3next", seed=1)
    d = wl.dims
    t = wl.torch(dev)
    B, T, Hqk, Hv, K, V, N = (d[x] for x in ("B", "T", "Hqk", "Hv", "K", "V", "N"))
    a, b, A_log, dt_bias = gates(B, T, Hv, 5)
    ws = torch.empty(chunk_workspace_bytes(B, T, Hqk, Hv, K, V, N, False, False),
                     dtype=torch.uint8, device=dev)
    o = torch.empty_like(t["v"])
    kw = dict(initial_state=t["initial_state"], output_final_state=True, workspace=ws, out=o)

    def two_step():
        g, beta = fused_gdn_gating(A_log, a, b, dt_bias)
        chunk_gated_delta_rule(t["q"], t["k"], t["v"], g, beta, **kw)

    def fused():
        chunk_gated_delta_rule_gated(t["q"], t["k"], t["v"], a, b, A_log, dt_bias, **kw)

    ms2, ms1 = _time_graph(dev, two_step, launches=10), _time_graph(dev, fused, launches=10)
    out["prefill_cfg1"] = {"two_step_us": round(ms2 * 1e3, 2), "fused_us": round(ms1 * 1e3, 2),
                           "saved_us": round((ms2 - ms1) * 1e3, 2),
                           "hbm_bytes_saved": 16 * B * T * Hv}
    wl = W.config("cfg2_decode_b256", seed=2)
    d = wl.dims
    t = wl.torch(dev)
    B, T, Hqk, Hv, K, V, N = (d[x] for x in ("B", "T", "Hqk", "Hv", "K", "V", "N"))
    a, b, A_log, dt_bias = gates(B, T, Hv, 6)
    state = t["initial_state"].clone()
    o = torch.empty_like(t["v"])

    def two_step_dec():
        g, beta = fused_gdn_gating(A_log, a, b, dt_bias)
        fused_recurrent_gated_delta_rule(t["q"], t["k"], t["v"], g, beta, initial_state=state,
                                         output_final_state=True, out=o)

    def fused_dec():
        fused_recurrent_gated_delta_rule_gated(t["q"], t["k"], t["v"], a, b, A_log, dt_bias,
                                               initial_state=state, output_final_state=True,
                                               out=o)

    ms2, ms1 = _time_graph(dev, two_step_dec), _time_graph(dev, fused_dec)
    out["decode_cfg2"] = {"two_step_us": round(ms2 * 1e3, 2), "fused_us": round(ms1 * 1e3, 2),
                          "saved_us": round((ms2 - ms1) * 1e3, 2),
                          "hbm_bytes_saved": 16 * B * T * Hv}
    return out


def bench_layer_ops(dev):
    """The layer's neighbours of the core at the Qwen3-Next layer shape
    (T = 8192, conv_dim = 2 * 16 * 128 + 32 * 128 = 8192; decode batch 256),
    each against HBM bandwidth with its algorithmic bytes per launch."""
    from avelang_amd import fused_recurrent_gated_delta_rule, layer_ops as L
    from avelang_amd import workloads as W

    g = torch.Generator(device=dev).manual_seed(7)

    def rnd(*shape, dtype=torch.bfloat16):
        return torch.randn(*shape, generator=g, device=dev, dtype=torch.float32).to(dtype)

    T, D, Hqk, Hv, K = 8192, 8192, 16, 32, 128
    Bd, S, Wk = 256, 3, 4
    res = {}

    def add(name, fn, nbytes, shape):
        ms = _time_graph(dev, fn)
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = {"shape": shape, "us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                     "bytes_per_launch": int(nbytes), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}

    x = rnd(1, T, D).transpose(1, 2)                       # the layer's channel-last memory
    w = rnd(D, Wk)
    add("causal_conv1d_fn", lambda: L.causal_conv1d_fn(x, w, None, activation="silu"),
        2 * 2 * D * T, f"x [1, {D}, {T}] bf16 channel-last, W={Wk}, SiLU")
    xd = rnd(Bd, D)
    cs = rnd(Bd, D, S)
    add("causal_conv1d_update", lambda: L.causal_conv1d_update(xd, cs, w, None, activation="silu"),
        2 * 2 * Bd * D + 2 * 2 * Bd * D * S, f"x [{Bd}, {D}] bf16, state [{Bd}, {D}, {S}] in place")
    a, b = rnd(1, T, Hv), rnd(1, T, Hv)
    A_log, dt_bias = torch.zeros(Hv, device=dev), torch.zeros(Hv, device=dev)
    add("fused_gdn_gating", lambda: L.fused_gdn_gating(A_log, a, b, dt_bias),
        T * Hv * (2 + 2 + 4 + 4), f"a, b [1, {T}, {Hv}] bf16 -> g, beta fp32")
    qk = rnd(1, T, Hqk, K)
    add("l2norm_fwd", lambda: L.l2norm_fwd(qk), 2 * 2 * T * Hqk * K, f"[1, {T}, {Hqk}, {K}] bf16")
    o, z = rnd(1, T, Hv, K), rnd(1, T, Hv, K)
    nw = torch.ones(K, device=dev, dtype=torch.bfloat16)
    add("rms_norm_gated", lambda: L.rms_norm_gated(o, z, nw), 3 * 2 * T * Hv * K,
        f"o, z [1, {T}, {Hv}, {K}] bf16")
    dl = W.config("cfg2_decode_b256", seed=300).torch(dev)
    pool = 0.01 * torch.randn((2 * Bd, Hv, K, K), generator=g, device=dev)
    idx = torch.randperm(2 * Bd, generator=g, device=dev)[:Bd].to(torch.int32)
    out = torch.empty_like(dl["v"])
    add("fused_recurrent_state_pool",
        lambda: fused_recurrent_gated_delta_rule(dl["q"], dl["k"], dl["v"], dl["g"], dl["beta"],
                                                 initial_state=pool, output_final_state=True,
                                                 ssm_state_indices=idx, out=out),
        decode_bytes(Bd, Hqk, Hv), f"{Bd} sequences over a {2 * Bd}-slot fp32 state pool")
    return res


def cpu_prefill(wl, runs=5):
    from oracle import cpu as oracle

    threads = oracle.host_threads()
    a = wl.numpy()
    oracle.run("chunk", **a, threads=threads)          # warm-up
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        oracle.run("chunk", **a, threads=threads)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return dict(value=wl.dims["T"] / med, unit="tokens/s", cores=threads, kind="port",
                sample=f"config 1 in full (T={wl.dims['T']}, 32 v-heads), C/OpenMP fp32 "
                       f"chunked oracle (oracle/gdn_cpu.c), median of {runs} runs "
                       f"({med * 1e3:.1f} ms each)",
                host=oracle.host_info(threads))


def cpu_decode(runs=3):
    from avelang_amd import workloads as W
    from oracle import cpu as oracle

    threads = oracle.host_threads()
    wl = W.config("cfg2_decode_b256", seed=200)
    a = wl.numpy()
    d = wl.dims
    oracle.run("recurrent", **a, threads=threads)
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        oracle.run("recurrent", **a, threads=threads)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    nb = decode_bytes(d["N"], d["Hqk"], d["Hv"], d["K"], d["V"])
    return dict(value=nb / med / 1e9, unit="GB/s", cores=threads, kind="port",
                sample=f"one full config-2 decode step (256 x 32 state tiles), C/OpenMP fp32 "
                       f"recurrence (oracle/gdn_cpu.c), median of {runs}",
                host=oracle.host_info(threads))


def profile_pass(dev, reps=3, what="all"):
    """Fixed, untimed launch sequence for rocprofv3 counter runs.

    ``what`` = "prefill" stops after step 2 (counter passes over the prefill
    kernels alone); "all" runs every step below.

    1. one device-to-device copy of exactly 256 MiB (calibrates FETCH_SIZE /
       WRITE_SIZE against known bytes: 256 MiB read, 256 MiB written);
    2. ``reps`` config-1 prefill calls (chunk_prep, chunk_chain);
    3. ``reps`` config-2 decode steps (recurrent_kernel<128,128>);
    4. ``reps`` calls of each layer operator at the Qwen3-Next layer shape;
    5. ``reps`` config-1 backward calls (gdn_chunk_bwd with its recomputation).
    """
    from avelang_amd import chunk_gated_delta_rule, fused_recurrent_gated_delta_rule
    from avelang_amd import workloads as W

    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    wl = W.config("cfg1_prefill_qwen3next", seed=1)
    t = wl.torch(dev)
    dl = W.config("cfg2_decode_b256", seed=200)
    d = dl.torch(dev)
    torch.cuda.synchronize(dev)
    dst.copy_(src)
    torch.cuda.synchronize(dev)
    for _ in range(reps):
        chunk_gated_delta_rule(t["q"], t["k"], t["v"], t["g"], t["beta"],
                               initial_state=t["initial_state"], output_final_state=True)
    torch.cuda.synchronize(dev)
    if what == "prefill":
        print("profile pass done", flush=True)
        return
    for _ in range(reps):
        fused_recurrent_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"],
                                         initial_state=d["initial_state"],
                                         output_final_state=True, inplace_final_state=True)
    torch.cuda.synchronize(dev)
    from avelang_amd import layer_ops as L
    T, D, Hqk, Hv, K = 8192, 8192, 16, 32, 128
    x = torch.randn(1, T, D, device=dev).to(torch.bfloat16).transpose(1, 2)
    w = torch.randn(D, 4, device=dev).to(torch.bfloat16)
    xd = torch.randn(256, D, device=dev).to(torch.bfloat16)
    cs = torch.randn(256, D, 3, device=dev).to(torch.bfloat16)
    a = torch.randn(1, T, Hv, device=dev).to(torch.bfloat16)
    qk = torch.randn(1, T, Hqk, K, device=dev).to(torch.bfloat16)
    o = torch.randn(1, T, Hv, K, device=dev).to(torch.bfloat16)
    nw = torch.ones(K, device=dev, dtype=torch.bfloat16)
    zeros = torch.zeros(Hv, device=dev)
    torch.cuda.synchronize(dev)
    for _ in range(reps):
        L.causal_conv1d_fn(x, w, None, activation="silu")
        L.causal_conv1d_update(xd, cs, w, None, activation="silu")
        L.fused_gdn_gating(zeros, a, a, zeros)
        L.l2norm_fwd(qk)
        L.rms_norm_gated(o, o, nw)
    torch.cuda.synchronize(dev)
    from avelang_amd import chunk_gated_delta_rule_bwd
    do = torch.randn((1, T, Hv, K), device=dev).to(torch.bfloat16)
    for _ in range(reps):
        chunk_gated_delta_rule_bwd(t["q"], t["k"], t["v"], t["g"], t["beta"], do, None,
                                   initial_state=t["initial_state"])
    torch.cuda.synchronize(dev)
    print("profile pass done", flush=True)


def pmc_summary(fetch_dir, write_dir, out_path):
    """profiles/traffic.json from two rocprofv3 --pmc runs of --profile-pass.

    Each counter is averaged per kernel over its dispatches and scaled by
    what it reads for the pass's 256 MiB device copy (known bytes), so the
    figures are HBM bytes per launch.  Path totals: prefill = chunk_prep +
    chunk_chain (forward instantiations), backward = the four launches of
    gdn_chunk_bwd, decode = the recurrent kernel.
    """
    import csv
    import glob

    def per_kernel(d, counter):
        acc = {}
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if r["Counter_Name"] != counter:
                    continue
                name = r["Kernel_Name"].split("(")[0].replace("void ", "").strip()
                disp = (r.get("Dispatch_Id") or r.get("Correlation_Id"))
                acc.setdefault(name, {}).setdefault(disp, 0.0)
                acc[name][disp] += float(r["Counter_Value"])   # summed over dimensions
        return {k: float(np.mean(list(v.values()))) * 1024 for k, v in acc.items()}  # KiB -> B

    fetch, write = per_kernel(fetch_dir, "FETCH_SIZE"), per_kernel(write_dir, "WRITE_SIZE")
    copy = [k for k in fetch if "copyBuffer" in k]
    if not copy:
        raise SystemExit("pmc_summary: the calibration copy is missing")
    ff = (256 << 20) / fetch[copy[0]]
    wf = (256 << 20) / write[copy[0]]
    kern = {k: {"fetch_bytes": int(fetch[k] * ff), "write_bytes": int(write.get(k, 0) * wf)}
            for k in sorted(fetch) if k.startswith("gdn::")}

    def total(pred):
        return sum(v["fetch_bytes"] + v["write_bytes"] for k, v in kern.items() if pred(k))

    def named(k, *prefixes):
        # template arguments after these (the l2norm form, V tiles per
        # workgroup) do not change which launch of the path it is
        return any(k.startswith("gdn::" + p) and k[len("gdn::" + p)] in ",>" for p in prefixes)

    res = {
        "prefill": total(lambda k: named(k, "chunk_prep_kernel<128, false",
                                         "chunk_chain_sw_kernel<128, false, true")),
        "decode": total(lambda k: "recurrent_kernel<128, 128" in k),
        "backward": total(lambda k: named(k, "chunk_prep_kernel<128, true",
                                          "chunk_chain_sw_kernel<128, true, false",
                                          "chunk_rev_sw_kernel<128", "chunk_grad_kernel<128, 128")),
        "per_kernel": kern,
        "fetch_size_factor": round(ff, 4),
        "write_size_factor": round(wf, 4),
        "calibration": "one 256 MiB device-to-device copy in the same run",
    }
    with open(out_path, "w") as f:
        json.dump(res, f, indent=1)
    print(json.dumps({k: res[k] for k in ("prefill", "decode", "backward")}))


def pmc_table(dirs):
    """Per-kernel, per-dispatch averages of every counter in rocprofv3 --pmc CSV output.

    Values are summed over the counter's dimensions (SEs, XCDs) within a
    dispatch, then averaged over the dispatches of the kernel.  Printed as one
    JSON object per kernel, keyed by counter name.
    """
    import csv
    import glob

    acc = {}
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                name = r["Kernel_Name"].split("(")[0].replace("void ", "").strip()
                disp = r.get("Dispatch_Id") or r.get("Correlation_Id")
                key = (name, r["Counter_Name"])
                acc.setdefault(key, {}).setdefault(disp, 0.0)
                acc[key][disp] += float(r["Counter_Value"])
    table = {}
    for (name, ctr), per in acc.items():
        table.setdefault(name, {})[ctr] = float(np.mean(list(per.values())))
    for name in sorted(table):
        print(json.dumps({"kernel": name, **{k: round(v, 1) for k, v in sorted(table[name].items())}}))


def _backward_record(bwd, no_cpu):
    flops = backward_flops(bwd["T"], bwd["Hv"], bwd["K"], bwd["V"])
    tf = flops / (bwd["ms"] * 1e-3) / 1e12
    return {
        "workload": "cfg1 chunk_gated_delta_rule backward (gdn_chunk_bwd: forward recompute, "
                    "reverse state-gradient chain, per-chunk gradients)",
        "value": round(bwd["T"] / (bwd["ms"] * 1e-3), 1), "unit": "tokens/s",
        "ms_per_step": round(bwd["ms"], 5),
        "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                     "traffic": _load_traffic("backward"),
                     "traffic_source": TRAFFIC_SOURCE,
                     "kernel": "gdn_chunk_bwd = chunk_prep<bwd> + chunk_chain<save> + "
                               "chunk_rev + chunk_grad",
                     "algorithmic_flops_per_launch": flops,
                     "flops_per_token_per_vhead": flops // (bwd["T"] * bwd["Hv"])},
        "workspace_bytes": bwd["ws_bytes"],
        "training_step": {
            "what": "autograd path: forward keeping the backward's inputs (gdn_chunk_fwd_save) "
                    "+ backward from that workspace (gdn_chunk_bwd saved=1)",
            "fwd_ms": round(bwd["ms_fwd_save"], 5), "bwd_ms": round(bwd["ms_bwd_saved"], 5),
            "value": round(bwd["T"] / ((bwd["ms_fwd_save"] + bwd["ms_bwd_saved"]) * 1e-3), 1),
            "unit": "tokens/s (forward + backward)"},
        "cpu_baseline": None if no_cpu else cpu_backward(bwd["wl"]),
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--decode-steps", type=int, default=1000)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-layer-ops", action="store_true",
                    help="skip the layer-operator measurements")
    ap.add_argument("--headline-only", action="store_true",
                    help="only the config-1 prefill and config-2 decode lines (profiling runs)")
    ap.add_argument("--profile-pass", nargs="?", const="all", choices=("all", "prefill"),
                    help="run the fixed untimed launch sequence used for rocprofv3 --pmc runs "
                         "(prefill: the config-1 prefill calls only)")
    ap.add_argument("--pmc-table", nargs="+", metavar="DIR",
                    help="print per-kernel averages of every counter found in rocprofv3 --pmc "
                         "output directories (one JSON object per kernel)")
    ap.add_argument("--backward-only", action="store_true",
                    help="only the config-1 backward measurement (profiling runs)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="write profiles/traffic.json from two rocprofv3 --pmc runs of --profile-pass")
    args = ap.parse_args()
    if args.pmc_table:
        pmc_table(args.pmc_table)
        return
    if args.pmc_summary:
        pmc_summary(args.pmc_summary[0], args.pmc_summary[1],
                    os.path.join(ROOT, "profiles", "traffic.json"))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only; the GDN operator shards by "
              "heads with no communication, so --gpus N>1 is not run here.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.profile_pass:
        profile_pass(dev, what=args.profile_pass)
        return
    if args.backward_only:
        print(json.dumps(_backward_record(bench_backward(dev, args.steps, args.warmup), True)),
              flush=True)
        return

    pre = bench_prefill(dev, args.steps, args.warmup)
    dec = bench_decode(dev, args.decode_steps)
    extra = not args.headline_only
    layer = bench_layer_ops(dev) if extra and not args.no_layer_ops else None
    fusions = bench_fusions(dev) if extra and not args.no_layer_ops else None
    pre_l2 = bench_prefill(dev, max(args.steps // 2, 1), args.warmup, l2norm=True) if extra else None
    others = ([bench_prefill_config(dev, n) for n in ("cfg3_varlen_64seq", "cfg4_long_context")]
              if extra else None)
    bwd = bench_backward(dev, args.steps, args.warmup) if extra else None

    flops = prefill_flops(pre["T"], pre["Hv"], pre["K"], pre["V"])
    tflops = flops / (pre["ms"] * 1e-3) / 1e12
    tokens_s = pre["T"] / (pre["ms"] * 1e-3)
    dec_gbs = dec["bytes"] / (dec["ms"] * 1e-3) / 1e9

    cpu_pre = cpu_dec = None
    if not args.no_cpu:
        cpu_pre = cpu_prefill(pre["wl"])
        cpu_dec = cpu_decode()

    rec = {
        "metric": METRIC,
        "value": round(tokens_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(pre["ms"], 5),
        "ms_per_step_after_idle": round(pre["ms_after_idle"], 5),
        "clock_warmup_ms": CLOCK_WARMUP_MS,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded numpy PCG64; BASELINE config distributions)",
        "config": {"workload": "cfg1 GDN chunked prefill, Qwen3-Next shape", "B": 1, "T": pre["T"],
                   "qk_heads": 16, "v_heads": pre["Hv"], "K": pre["K"], "V": pre["V"], "chunk": C,
                   "state": "fp32, initial + final", "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                     "traffic": _load_traffic("prefill"),
                     "traffic_source": TRAFFIC_SOURCE,
                     "kernel": "gdn_chunk_fwd = chunk_prep + chunk_chain (+ chunk_table with cu_seqlens)",
                     "algorithmic_flops_per_launch": flops,
                     "flops_per_token_per_vhead": 6 * C * pre["K"] + 4 * C * pre["V"] + 6 * pre["K"] * pre["V"]},
        "cpu_baseline": cpu_pre,
        "decode": {
            "workload": "cfg2 fused recurrent decode, 256 seqs x 32 v-heads, state in place",
            "value": round(dec_gbs, 1), "unit": "GB/s", "ms_per_step": round(dec["ms"], 5),
            "steps": dec["steps"], "tokens_per_s": round(dec["N"] / (dec["ms"] * 1e-3), 1),
            "roofline": {"bound": "hbm", "achieved": round(dec_gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(dec_gbs / HBM_PEAK_GBS, 4),
                         "traffic": _load_traffic("decode"),
                     "traffic_source": TRAFFIC_SOURCE,
                         "kernel": "recurrent_kernel<128,128>",
                         "algorithmic_bytes_per_launch": dec["bytes"]},
            "cpu_baseline": cpu_dec,
        },
        "prefill_qk_l2norm_in_kernel": None if pre_l2 is None else {
            "workload": "cfg1 as the layer calls it: use_qk_l2norm_in_kernel=True (q, k normalised inside)",
            "value": round(pre_l2["T"] / (pre_l2["ms"] * 1e-3), 1), "unit": "tokens/s",
            "ms_per_step": round(pre_l2["ms"], 5)},
        "prefill_other_configs": others,
        "backward": None if bwd is None else _backward_record(bwd, args.no_cpu),
        "layer_ops": layer,
        "fusions": fusions,
        "host_wall_ms_per_step": round(pre["wall_ms"], 5),
        "host_enqueue_ms_per_step": round(pre["enqueue_ms"], 5),
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
