#!/usr/bin/env python3
"""Benchmark of the MI355X attention path on BASELINE.json's shapes.

One "step" is one call of the hot path over one batch of synthetic input
(seeded, generated on the GPU; see pelica_amd/workloads.py).  The headline
workload is config 3: gpt-oss-20b decode attention at 32K context, full
layer with sinks (value = KV GB/s).  Prefill (config 4, TFLOP/s) and the
other configs are reported beside it in the same JSON line.

Inputs are resident in HBM before the timed region; each step reads a
different copy of the KV cache (copies totalling >= 1 GiB), so the 256 MB
last-level cache cannot serve the bytes the HBM roofline counts.

The CPU baseline is the C port of the reference's cpu_attn.rs (oracle/,
kind "port") timed on this host's cores on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
F16_PEAK_TFLOPS = 2500.0    # MI355X dense f16 MFMA
# HBM bytes per launch of the dominant kernels come from rocprofv3 --pmc
# FETCH_SIZE / WRITE_SIZE runs summarised in this file (`--traffic` writes the
# summary); each entry records a hash of the kernel's sources, and an entry
# whose sources have changed since is not reported.
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "hbm_traffic_counters.md")
KERNEL_SOURCES = {
    "decode": ("attn_decode.hip", "attn_decode.hpp", "attn_common.hpp"),
    "prefill": ("attn_prefill.hip", "attn_prefill.hpp", "attn_common.hpp"),
}
# rocprofv3 kernel-name prefix and source set of each config's dominant kernel
TRAFFIC_KERNELS = {
    "c3_gptoss_decode_full": ("decode_kernel<64, 1, 8, 4", "decode"),
    "c4_gptoss_prefill_full": ("prefill_kernel<64, 2, false, false, 8", "prefill"),
    "c5_qwen3_spec_decode": ("decode_kernel<128", "decode"),
}


def sources_hash(kind: str) -> str:
    import hashlib

    h = hashlib.sha256()
    for f in KERNEL_SOURCES[kind]:
        with open(os.path.join(ROOT, "pelica_amd", "csrc", f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:12]


def recorded_traffic(config: str):
    """(bytes per launch, note) from the committed counter summary: None
    when it has no entry for the config or the kernel's sources changed."""
    try:
        lines = open(TRAFFIC_PROFILE).read().splitlines()
    except OSError:
        return None, "no counter summary"
    for ln in lines:
        f = ln.split()
        if len(f) == 4 and f[0] == "traffic" and f[1] == config:
            kind = TRAFFIC_KERNELS[config][1]
            if f[3] != "src=" + sources_hash(kind):
                return None, "counters predate this build of the kernel"
            return int(f[2]), "rocprofv3 FETCH_SIZE x calibration + WRITE_SIZE (profiles/hbm_traffic_counters.md)"
    return None, "no counter entry"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="", help="comma list of config names to time (default: all)")
    ap.add_argument("--profile", default="",
                    help="comma list of configs: just run each --steps times, eagerly, for rocprofv3 passes")
    ap.add_argument("--dtrace", default="",
                    help="comma list of decode configs: summarise the split kernel's per-wave stamps "
                         "(needs a library built with -DPELICA_DTRACE, loaded through PELICA_ATTN_LIB)")
    ap.add_argument("--traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="summarise two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of "
                         "--profile copy,<configs> into the lines the roofline's traffic is read from")
    ap.add_argument("--gemm", action="store_true",
                    help="calibration: the f16 rate of the platform's GEMM (torch.matmul, hipBLASLt) on this GPU")
    ap.add_argument("--ptrace", default="",
                    help="comma list of prefill configs: summarise the prefill kernel's per-wave stamps "
                         "(needs a library built with -DPELICA_PTRACE, loaded through PELICA_ATTN_LIB)")
    return ap.parse_args()


def rotating_copies(t, min_total=1 << 30):
    import torch

    n = max(1, -(-min_total // (t.numel() * t.element_size())))
    return [t] + [t.clone() for _ in range(n - 1)]


def time_calls(fn, n_copies, steps, warmup, graph=True):
    """ms per call.  The calls are recorded once into a HIP graph (one call
    per KV copy) and the graph is replayed, so host-side launch cost stays
    out of the figure, as it does for an engine that records its passes;
    HIP events on the launch stream bracket the replays."""
    import torch

    for i in range(warmup):
        fn(i % n_copies)
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    if graph:
        # enough calls per graph to amortise the replay's fixed cost (~20 us)
        per = n_copies * max(1, -(-64 // n_copies))
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(per):
                fn(i % n_copies)
        g.replay()
        torch.cuda.synchronize()
        reps = max(1, -(-steps // per))
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(reps):
            g.replay()
        e1.record(st)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / (reps * per)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for i in range(steps):
        fn(i % n_copies)
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def kernel_times(fn, n_copies, reps):
    """Average GPU time per kernel kind over `reps` eager calls, from the
    library's own per-kernel HIP events (pelica_attn_prof_*)."""
    import torch

    from pelica_amd import attn

    attn.prof_enable(True)
    for i in range(reps):
        fn(i % n_copies)
    torch.cuda.synchronize()
    recs = attn.prof_read()
    attn.prof_enable(False)
    out = {}
    for name, ms in recs:
        out.setdefault(name, []).append(ms)
    return {k: sum(v) / len(v) for k, v in out.items()}


def bench_decode(cfg, steps, warmup):
    import torch

    from pelica_amd import attn
    from pelica_amd import workloads as wl

    inp = wl.make_inputs(cfg, "cuda")
    ks = rotating_copies(inp.k)
    vs = [inp.v] + [inp.v.clone() for _ in range(len(ks) - 1)]
    out = torch.empty_like(inp.q)
    kw = dict(n_kv=cfg.n_kv, kv_len=inp.kv_len, sinks=inp.sinks, window=cfg.window)
    if inp.ragged:
        kw.update(seq_kv_len=inp.seq_len, seq_kv_offset=inp.seq_off)
    desc = attn.make_desc(cfg.n_head, cfg.n_kv, cfg.hd, n_seq=cfg.n_seq, q_tokens=cfg.q_tokens,
                          kv_len=inp.kv_len, seq_kv_len=kw.get("seq_kv_len"), seq_kv_offset=kw.get("seq_kv_offset"),
                          window=cfg.window)
    ws_n = attn.workspace_bytes(desc)
    ws = attn.new_workspace(desc)

    def call(i):
        attn.decode(inp.q, ks[i], vs[i], out=out, workspace=ws, **kw)

    def call_split(i):  # the key-split kernel alone (measurement flag)
        attn.decode(inp.q, ks[i], vs[i], out=out, workspace=ws, split_only=True, **kw)

    ms = time_calls(call, len(ks), steps, warmup)
    split_graph_ms = time_calls(call_split, len(ks), steps, warmup)
    ms_eager = time_calls(call, len(ks), steps, warmup, graph=False)
    kt = kernel_times(call, len(ks), steps)
    nbytes = wl.kv_bytes(cfg, inp.seq_len.tolist())
    gbs = nbytes / (ms * 1e-3) / 1e9
    return dict(config=cfg.name, ms=ms, ms_eager=ms_eager, bytes=nbytes, GBps=gbs, frac_hbm=gbs / HBM_PEAK_GBS,
                kernel_ms=kt, split_ms=split_graph_ms, split_GBps=nbytes / (split_graph_ms * 1e-3) / 1e9,
                workspace_bytes=ws_n, kv_copies=len(ks))


def bench_prefill(cfg, steps, warmup):
    import torch

    from pelica_amd import attn
    from pelica_amd import workloads as wl

    inp = wl.make_inputs(cfg, "cuda")
    out = torch.empty_like(inp.q)

    def call(i):
        attn.prefill(inp.q, inp.k, inp.v, n_kv=cfg.n_kv, kv_len=inp.kv_len, sinks=inp.sinks, window=cfg.window,
                     out=out)

    ms = time_calls(call, 1, steps, warmup)
    kt = kernel_times(call, 1, steps)
    flops = wl.attn_flops(cfg)
    tf = flops / (ms * 1e-3) / 1e12
    # one call is one prefill kernel: its per-launch time is the graph time per call
    return dict(config=cfg.name, ms=ms, flops=flops, TFLOPs=tf, frac_mfma=tf / F16_PEAK_TFLOPS, kernel_ms=kt,
                kernel_TFLOPs=tf)


def bench_mla(steps, warmup, n_head=32, kv_len=32768):
    """MLA decode over a 32K latent cache (not a BASELINE config; reported
    beside them): bytes = latent rows once + q + out."""
    import torch

    from pelica_amd import attn

    g = torch.Generator(device="cuda").manual_seed(12)
    q = torch.randn(1, 1, n_head, 512, generator=g, device="cuda") * 0.25
    lat = (torch.randn(kv_len, 512, generator=g, device="cuda") * 0.5).half()
    lats = rotating_copies(lat)
    out = torch.empty_like(q)
    desc = attn.make_desc(n_head, 1, 512, kv_len=kv_len)
    ws = torch.empty(max(1, attn.load_library().pelica_attn_mla_workspace_bytes(desc)), dtype=torch.uint8,
                     device="cuda")

    def call(i):
        attn.mla(q, lats[i], kv_len=kv_len, out=out, workspace=ws)

    ms = time_calls(call, len(lats), steps, warmup)
    kt = kernel_times(call, len(lats), steps)
    nbytes = kv_len * 512 * 2 + 2 * q.numel() * 4
    return dict(config=f"mla_decode_h{n_head}_32k", ms=ms, bytes=nbytes, GBps=nbytes / (ms * 1e-3) / 1e9,
                frac_hbm=nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, kernel_ms=kt)


def bench_qkv(steps, warmup, T=4096, n_head=64, n_kv=8, hd=64):
    """The step before attention over a 4096-token gpt-oss pass: q, k, v f32
    in, q f32 out, k/v f16 rows out (HBM-bound)."""
    import torch

    from pelica_amd import attn

    g = torch.Generator(device="cuda").manual_seed(13)
    q = torch.randn(1, T, n_head, hd, generator=g, device="cuda")
    k = torch.randn(1, T, n_kv, hd, generator=g, device="cuda")
    v = torch.randn(1, T, n_kv, hd, generator=g, device="cuda")
    pos = torch.arange(T, device="cuda", dtype=torch.float64)[:, None]
    th = pos * 150000.0 ** (-(2.0 * torch.arange(hd // 2, device="cuda", dtype=torch.float64)) / hd)
    table = torch.stack([th.cos(), th.sin()], -1).float().contiguous()
    kc = torch.empty(T, n_kv * hd, dtype=torch.float16, device="cuda")
    vc = torch.empty_like(kc)

    def call(i):
        attn.qkv_rope_cache(q, k, v, kc, vc, n_kv=n_kv, kv_len=T, table=table)

    ms = time_calls(call, 1, steps, warmup)
    kt = kernel_times(call, 1, steps)
    nbytes = q.numel() * 4 * 2 + (k.numel() + v.numel()) * (4 + 2) + T * (hd // 2) * 8
    return dict(config="qkv_rope_cache_gptoss_4096", ms=ms, bytes=nbytes, GBps=nbytes / (ms * 1e-3) / 1e9,
                frac_hbm=nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, kernel_ms=kt)


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), for the CPU baseline."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def bench_merge(steps, warmup, n_slots=512, n_tok=1, n_head=32, hd=128):
    """pelica_attn_partials_merge_batch at the MoE engine's CPU-tier layout
    (src/moe.rs:1713-1729: one slot per 64 positions, 512 at 32K keys;
    Qwen3 heads): bytes = the slots read once + the output written."""
    import torch

    from pelica_amd import attn

    g = torch.Generator(device="cuda").manual_seed(14)
    parts = torch.randn(n_slots, n_tok, n_head, hd + 2, generator=g, device="cuda")
    parts[..., 1] = parts[..., 1].abs() + 1.0
    sinks = torch.randn(n_head, generator=g, device="cuda")
    copies = rotating_copies(parts, 256 << 20)
    out = torch.empty(n_tok, n_head, hd, device="cuda")

    def call(i):
        attn.partials_merge_batch(copies[i], sinks=sinks, out=out)

    ms = time_calls(call, len(copies), steps, warmup)
    kt = kernel_times(call, len(copies), steps)
    nbytes = parts.numel() * 4 + out.numel() * 4
    return dict(config=f"partials_merge_{n_slots}slots_t{n_tok}_h{n_head}_hd{hd}", ms=ms, bytes=nbytes,
                GBps=nbytes / (ms * 1e-3) / 1e9, frac_hbm=nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, kernel_ms=kt)


def cpu_baseline_decode(cfg, reps=20):
    """The C port of cpu_attn.rs on every host core, full C3 workload: one
    warm-up call, then the median of `reps`."""
    import numpy as np

    from oracle import oracle as orc
    from pelica_amd import workloads as wl

    inp = wl.make_inputs(cfg, "cpu")
    q = inp.q.numpy()
    k = inp.k.numpy().view(np.uint16)
    v = inp.v.numpy().view(np.uint16)
    sinks = inp.sinks.numpy() if inp.sinks is not None else None
    threads = os.cpu_count() or 1
    orc.attention(q, k, v, n_kv=cfg.n_kv, kv_len=cfg.kv_len, sinks=sinks, window=cfg.window, threads=threads)
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        orc.attention(q, k, v, n_kv=cfg.n_kv, kv_len=cfg.kv_len, sinks=sinks, window=cfg.window, threads=threads)
        times.append(time.perf_counter() - t)
    sec = float(np.median(times))
    return dict(value=wl.kv_bytes(cfg) / sec / 1e9, unit="GB/s", cores=threads, kind="port", model=cpu_model(),
                sample=f"full {cfg.name} call (64 query heads x 32768 keys), median of {reps}",
                ms=sec * 1e3)


def cpu_baseline_prefill(cfg, rows=32, reps=20):
    """The same port on the last `rows` prompt tokens (the longest key
    ranges): one warm-up call, then the median of `reps`."""
    import numpy as np

    from oracle import oracle as orc
    from pelica_amd import workloads as wl

    inp = wl.make_inputs(cfg, "cpu")
    q = inp.q.numpy().view(np.uint16)
    k = inp.k.numpy().view(np.uint16)
    v = inp.v.numpy().view(np.uint16)
    sinks = inp.sinks.numpy()
    T = cfg.q_tokens
    threads = os.cpu_count() or 1
    def run():
        orc.attention(q, k, v, n_kv=cfg.n_kv, kv_len=cfg.kv_len, sinks=sinks, window=cfg.window, t_begin=T - rows,
                      t_end=T, threads=threads)

    run()
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        run()
        times.append(time.perf_counter() - t)
    sec = float(np.median(times))
    pairs = sum(min(p + 1, cfg.window) if cfg.window else p + 1 for p in range(T - rows, T))
    flops = 4 * cfg.hd * cfg.n_head * pairs
    return dict(value=flops / sec / 1e12, unit="TFLOP/s", cores=threads, kind="port", model=cpu_model(),
                sample=f"last {rows} of {T} prompt tokens of {cfg.name}, median of {reps}", ms=sec * 1e3)


def profile_only(args):
    """Run the named configs eagerly (no graphs, no timing) for profilers."""
    import torch

    from pelica_amd import attn
    from pelica_amd import workloads as wl

    for name in args.profile.split(","):
        if name == "mla_decode_h32_32k":  # MLA decode over rotating latent copies
            g = torch.Generator(device="cuda").manual_seed(12)
            q = torch.randn(1, 1, 32, 512, generator=g, device="cuda") * 0.25
            lats = rotating_copies((torch.randn(32768, 512, generator=g, device="cuda") * 0.5).half())
            for i in range(args.steps):
                attn.mla(q, lats[i % len(lats)], kv_len=32768)
            torch.cuda.synchronize()
            continue
        if name == "qkv_rope_cache_gptoss_4096":  # (its timed graph replays)
            bench_qkv(args.steps, 1)
            continue
        if name in ("partials_merge_t1", "partials_merge_t4"):
            bench_merge(args.steps, 1, n_tok=int(name[-1]))
            continue
        if name == "copy":  # calibration: a plain 256 MiB device copy
            x = torch.ones(256 << 20, dtype=torch.uint8, device="cuda")
            y = torch.empty_like(x)
            for _ in range(args.steps):
                y.copy_(x)
            torch.cuda.synchronize()
            continue
        cfg = wl.CONFIGS[name]
        inp = wl.make_inputs(cfg, "cuda")
        kw = dict(n_kv=cfg.n_kv, kv_len=inp.kv_len, sinks=inp.sinks, window=cfg.window)
        if inp.ragged:
            kw.update(seq_kv_len=inp.seq_len, seq_kv_offset=inp.seq_off)
        for _ in range(args.steps):
            if cfg.kind == "decode":
                attn.decode(inp.q, inp.k, inp.v, **kw)
            else:
                attn.prefill(inp.q, inp.k, inp.v, **kw)
        torch.cuda.synchronize()
        print(f"profiled {name} x{args.steps}", flush=True)


def ptrace_summary(args):
    """Shader clock and per-chunk cycles of the prefill kernel, from the
    per-wave stamps of a -DPELICA_PTRACE build (pelica_attn_debug_ptrace):
    [loop cycles (s_memtime), tile-wait cycles, barrier cycles, exact-path
    chunks << 32 | chunks, then 100 MHz real-time stamps at entry, loop
    start, loop end and exit, after the prologue's loads are issued, after
    they landed, after the workgroup barrier] per wave (16 words), of the
    last of --steps calls."""
    import ctypes

    import numpy as np
    import torch

    from pelica_amd import attn
    from pelica_amd import workloads as wl

    lib = attn.load_library()
    if not hasattr(lib, "pelica_attn_debug_ptrace"):
        sys.exit("--ptrace needs a library built with -DPELICA_PTRACE (PELICA_ATTN_LIB)")
    for name in args.ptrace.split(","):
        cfg = wl.CONFIGS[name]
        inp = wl.make_inputs(cfg, "cuda")
        for _ in range(args.steps):
            attn.prefill(inp.q, inp.k, inp.v, n_kv=cfg.n_kv, sinks=inp.sinks, window=cfg.window)
        torch.cuda.synchronize()
        buf = np.zeros(1 << 18, dtype=np.uint64)
        rc = lib.pelica_attn_debug_ptrace(buf.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(buf.nbytes))
        assert rc == 0, rc
        raw = buf.reshape(-1, 16)
        if (raw[:, 15] == 1).any():
            slide_summary(name, raw)
            continue
        n_chunks = raw[:, 3] & np.uint64(0xFFFFFFFF)
        keep = (raw[:, 7] > 0) & (n_chunks > 0)  # waves of the grid that ran the loop
        w = raw[keep].astype(np.float64)
        chunks = n_chunks[keep].astype(np.float64)
        loop_us = (w[:, 6] - w[:, 5]) / 100.0
        ghz = w[:, 0] / (loop_us * 1e3)
        q = lambda a, p: float(np.percentile(a, p))
        print(json.dumps({
            "config": name, "waves": int(len(w)),
            "shader_clock_GHz": {"median": round(q(ghz, 50), 3), "p10": round(q(ghz, 10), 3), "p90": round(q(ghz, 90), 3)},
            "loop_cycles_per_chunk": round(q(w[:, 0] / chunks, 50), 1),
            "exact_path_chunk_frac": round(float((raw[keep][:, 3] >> np.uint64(32)).astype(np.float64).sum() / chunks.sum()), 4),
            "tile_wait_frac": round(float(w[:, 1].sum() / w[:, 0].sum()), 4),
            "barrier_frac": round(float(w[:, 2].sum() / w[:, 0].sum()), 4),
            "entry_to_loop_us": round(q((w[:, 5] - w[:, 4]) / 100.0, 50), 2),
            # waves that started in the second half of the kernel's span (later generations)
            "entry_to_loop_us_late": round(q(((w[:, 5] - w[:, 4]) / 100.0)[w[:, 4] > np.median(w[:, 4])], 50), 2),
            "span_us": round(float((w[:, 7].max() - w[:, 4].min()) / 100.0), 2),
            "entry_to_issued_us": round(q((w[:, 8] - w[:, 4]) / 100.0, 50), 2),
            "issued_to_landed_us": round(q((w[:, 9] - w[:, 8]) / 100.0, 50), 2),
            "landed_to_barrier_us": round(q((w[:, 10] - w[:, 9]) / 100.0, 50), 2),
            "barrier_to_loop_us": round(q((w[:, 5] - w[:, 10]) / 100.0, 50), 2),
            "loop_us": round(q(loop_us, 50), 2),
            "loop_to_exit_us": round(q((w[:, 7] - w[:, 6]) / 100.0, 50), 2),
        }), flush=True)


def slide_summary(name, raw):
    """Timeline of the sliding-window prefill kernel (prefill_slide_kernel
    stamps): us from the earliest wave entry, p10/p50/p90 over waves, and
    per-wave compute time of the first block by wave index (waves 0-3 share
    their SIMDs with waves 4-7)."""
    import numpy as np

    keep = raw[:, 7] > 0
    w = raw[keep].astype(np.float64)
    t0 = w[:, 4].min()
    q3 = lambda a: [round(float(np.percentile(a, x)), 2) for x in (10, 50, 90)]
    chunks = (raw[keep][:, 3] & np.uint64(0xFFFFFFFF)).astype(np.float64)
    comp_us = (w[:, 9] - w[:, 8] + np.where(w[:, 11] > 0, w[:, 11] - w[:, 10], 0)) / 100.0
    wg = raw[: len(raw) // 8 * 8].reshape(-1, 8, 16).astype(np.float64)
    wg = wg[(wg[:, :, 7] > 0).all(axis=1)]
    b0 = (wg[:, :, 9] - wg[:, :, 8]) / 100.0
    out = {"config": name, "kernel": "prefill_slide_kernel", "waves": int(len(w)),
           "shader_clock_GHz": q3(w[:, 0] / (comp_us * 1e3)),
           "compute_cycles_per_chunk": q3(w[:, 0] / chunks),
           "exact_path_chunk_frac": round(float((raw[keep][:, 3] >> np.uint64(32)).astype(np.float64).sum() / chunks.sum()), 4),
           "block0_compute_us_by_wave": [round(float(np.median(b0[:, k])), 2) for k in range(8)]}
    for key, col in [("first_compute", 5), ("block0_end", 9), ("block1_barrier", 12), ("block1_queries_read", 13),
                     ("block0_output_stored", 14), ("block1_start", 10), ("block1_end", 11), ("exit", 7)]:
        if (w[:, col] > 0).any():
            out[key + "_us"] = q3((w[w[:, col] > 0][:, col] - t0) / 100.0)
    print(json.dumps(out), flush=True)


def dtrace_summary(args):
    """Timeline of the decode split kernel from the per-wave stamps of a
    -DPELICA_DTRACE build (pelica_attn_debug_trace): 100 MHz real-time
    stamps at wave start, first K block landed, V blocks 0 and 1 landed,
    loop end, merge hand-off (waves that do not merge) and end, plus the
    wave's XCC/hardware id; of the last of --steps calls, in us from the
    earliest wave start."""
    import ctypes

    import numpy as np
    import torch

    from pelica_amd import attn
    from pelica_amd import workloads as wl

    lib = attn.load_library()
    if not hasattr(lib, "pelica_attn_debug_trace"):
        sys.exit("--dtrace needs a library built with -DPELICA_DTRACE (PELICA_ATTN_LIB)")
    for name in args.dtrace.split(","):
        cfg = wl.CONFIGS[name]
        inp = wl.make_inputs(cfg, "cuda")
        kw = dict(n_kv=cfg.n_kv, kv_len=inp.kv_len, sinks=inp.sinks, window=cfg.window)
        if inp.ragged:
            kw.update(seq_kv_len=inp.seq_len, seq_kv_offset=inp.seq_off)
        for _ in range(args.steps):
            attn.decode(inp.q, inp.k, inp.v, **kw)
        torch.cuda.synchronize()
        buf = np.zeros(1 << 16, dtype=np.uint64)
        rc = lib.pelica_attn_debug_trace(buf.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(buf.nbytes))
        assert rc == 0, rc
        w = buf.reshape(-1, 8)
        w = w[w[:, 0] > 0]
        # this call's waves: stamps within 1 ms of the latest start (the
        # buffer keeps earlier calls' entries past this grid's waves)
        w = w[w[:, 0] + 100000 > w[:, 0].max()]
        t0 = float(w[:, 0].min())
        rel = lambda col: (w[:, col].astype(np.float64) - t0) / 100.0
        q = lambda a: [round(float(np.percentile(a, p)), 2) for p in (10, 50, 90)]
        ok = lambda col: w[:, col] >= w[:, 0]  # (stamps of this call: not before the wave's own start)
        out = {"config": name, "waves": int(len(w)), "pct": "p10/p50/p90 us from the first wave's start"}
        last = ok(6)  # waves that wrote a result (the merging wave of each head)
        for col, key in ((0, "start"), (1, "first_k_landed"), (2, "v0_landed"), (3, "v1_landed_or_b0_issued"),
                         (4, "loop_end"), (6, "end")):
            m = ok(col)
            if m.any():
                out[key] = q(rel(col)[m])
        both = ok(3) & ok(4)
        if both.any():  # per wave: the last block's V landed -> its PV done
            out["v1_landed_to_loop_end_us"] = q(((w[:, 4].astype(np.float64) - w[:, 3]) / 100.0)[both])
        if (last & ok(5)).any():  # (workgroups of more than one wave per head)
            out["merging_wave_loop_to_merged_us"] = q(((w[:, 5].astype(np.float64) - w[:, 4]) / 100.0)[last & ok(5)])
            out["merging_wave_merged_to_end_us"] = q(((w[:, 6].astype(np.float64) - w[:, 5]) / 100.0)[last & ok(5)])
        out["last_end_us"] = round(float(rel(6)[ok(6)].max()), 2) if ok(6).any() else None
        print(json.dumps(out), flush=True)


def traffic_summary(args):
    """HBM bytes per dispatch of each config's dominant kernel from two
    rocprofv3 counter CSVs of `--profile copy,<configs>`: FETCH_SIZE scaled
    by what it reads for the plain 256 MiB copy (which moves 256 MiB in),
    WRITE_SIZE likewise; printed as the `traffic` lines bench.py reads."""
    import csv

    def per_kernel(path, counter):
        acc = {}
        with open(path) as fh:
            for row in csv.DictReader(fh):
                if row["Counter_Name"] != counter:
                    continue
                acc.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
        out = {k: sum(v) / len(v) for k, v in acc.items()}
        # the calibration copy: the largest copy dispatches (torch's small host copies use the same kernel)
        cp = acc.get("__amd_rocclr_copyBuffer", [])
        if cp:
            big = [x for x in cp if x >= 0.5 * max(cp)]
            out["__amd_rocclr_copyBuffer"] = sum(big) / len(big)
        return out

    fetch, write = per_kernel(args.traffic[0], "FETCH_SIZE"), per_kernel(args.traffic[1], "WRITE_SIZE")
    copy_kib = 256 * 1024
    ff = copy_kib / fetch["__amd_rocclr_copyBuffer"]
    wf = copy_kib / write["__amd_rocclr_copyBuffer"]
    print(f"calibration (256 MiB copy): FETCH_SIZE {fetch['__amd_rocclr_copyBuffer']:.1f} KiB -> x{ff:.3f}, "
          f"WRITE_SIZE {write['__amd_rocclr_copyBuffer']:.1f} KiB -> x{wf:.3f}")
    for cfg, (prefix, kind) in TRAFFIC_KERNELS.items():
        names = [k for k in fetch if k.startswith(prefix) or k.startswith("void pelica::" + prefix)]
        if not names:
            continue
        k = names[0]
        fb, wb = fetch[k] * ff * 1024, write.get(k, 0.0) * wf * 1024
        print(f"| {cfg} | `{k[:60]}` | {fetch[k]:.1f} | {fb / 1e6:.2f} MB | {write.get(k, 0.0):.1f} | {wb / 1e6:.2f} MB |")
        print(f"traffic {cfg} {int(round(fb + wb))} src={sources_hash(kind)}")


def gemm_rate():
    """Dense f16 GEMM rate of the platform library on this GPU (square
    problems, HIP events over 20 back-to-back calls): the MFMA rate a
    GEMM-only kernel reaches under the chip's power and clock limits."""
    import torch

    for n in (8192, 16384):
        a = torch.randn(n, n, dtype=torch.float16, device="cuda")
        b = torch.randn(n, n, dtype=torch.float16, device="cuda")
        for _ in range(3):
            a @ b
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(20):
            a @ b
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / 20
        tf = 2 * n ** 3 / (ms * 1e-3) / 1e12
        print(json.dumps({"gemm": f"f16 {n}x{n}x{n}", "us": round(ms * 1e3, 1), "TFLOPs": round(tf, 1),
                          "frac_of_2500": round(tf / F16_PEAK_TFLOPS, 3)}), flush=True)


def main():
    args = parse()
    if args.traffic:
        return traffic_summary(args)
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); "
              "the attention path is measured at its single-GPU shape", file=sys.stderr)
        sys.exit(2)
    import torch

    from pelica_amd import workloads as wl

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.gemm:
        return gemm_rate()
    if args.profile:
        return profile_only(args)
    if args.ptrace:
        return ptrace_summary(args)
    if args.dtrace:
        return dtrace_summary(args)
    only = set(filter(None, args.only.split(",")))

    def want(c):
        return not only or c.name in only

    results = {}
    for cfg in (wl.C3_FULL, wl.C3_SWA, wl.C1, wl.C2, wl.C5):
        if want(cfg):
            results[cfg.name] = bench_decode(cfg, args.steps, args.warmup)
    for cfg in (wl.C4_FULL, wl.C4_SWA):
        if want(cfg):
            results[cfg.name] = bench_prefill(cfg, args.steps, args.warmup)
    # the path's other kernels (no BASELINE config of their own)
    if not only or "mla_decode_h32_32k" in only:
        results["mla_decode_h32_32k"] = bench_mla(args.steps, args.warmup)
    if not only or "qkv_rope_cache_gptoss_4096" in only:
        results["qkv_rope_cache_gptoss_4096"] = bench_qkv(args.steps, args.warmup)
    for nt in (1, 4):
        r = bench_merge(args.steps, args.warmup, n_tok=nt) if (not only or f"partials_merge_t{nt}" in only) else None
        if r:
            results[r["config"]] = r

    head = results.get(wl.C3_FULL.name)
    pre = results.get(wl.C4_FULL.name)
    cpu = None if args.no_cpu else cpu_baseline_decode(wl.C3_FULL)
    cpu_pre = None if args.no_cpu else cpu_baseline_prefill(wl.C4_FULL)
    line = {
        "metric": "decode-attn KV GB/s (% HBM peak); prefill-attn TFLOP/s (% MFMA peak)",
        "value": round(head["GBps"], 1) if head else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 5) if head else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 KV, f32 softmax/accumulate",
        "data": "synthetic (seeded N(0,1) per BASELINE.json configs)",
        "config": {"workload": wl.C3_FULL.name, "n_head": 64, "n_kv": 8, "hd": 64, "kv_len": 32768,
                   "sinks": True, "window": 0, "batch": 1},
        "roofline": None,
        "cpu_baseline": cpu,
        "prefill": None,
        "configs": {k: {kk: (round(vv, 6) if isinstance(vv, float) else vv) for kk, vv in r.items()}
                    for k, r in results.items()},
    }
    if head:
        sg = head["split_GBps"]
        traffic, note = recorded_traffic(wl.C3_FULL.name)
        # achieved = algorithmic bytes (K/V once per kv head + q + out) per launch / launch time;
        # traffic = the bytes the counters saw (reads + the split partials written)
        line["roofline"] = {"bound": "hbm", "achieved": round(sg, 1), "peak": HBM_PEAK_GBS,
                            "unit": "GB/s", "frac": round(sg / HBM_PEAK_GBS, 4), "traffic": traffic,
                            "algorithmic_bytes": wl.kv_bytes(wl.C3_FULL), "traffic_source": note,
                            "kernel": "decode split kernel (decode_kernel<64,1,8,4>): HIP events over graph "
                                      "replays of split-only calls, per launch",
                            "kernel_ms": round(head["split_ms"], 5)}
    if pre:
        traffic, note = recorded_traffic(wl.C4_FULL.name)
        line["prefill"] = {"workload": wl.C4_FULL.name, "value": round(pre["TFLOPs"], 1), "unit": "TFLOP/s",
                           "ms_per_step": round(pre["ms"], 5),
                           "roofline": {"bound": "mfma", "achieved": round(pre["kernel_TFLOPs"], 1),
                                        "peak": F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                        "frac": round(pre["kernel_TFLOPs"] / F16_PEAK_TFLOPS, 4),
                                        "traffic": traffic, "traffic_source": note,
                                        "kernel": "prefill_kernel<64,2,..,8> (8 waves): HIP events over graph replays, per launch",
                                        "kernel_ms": round(pre["ms"], 5)},
                           "cpu_baseline": cpu_pre}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
