"""Benchmark of the MOSS-TTS-Nano LLM decode hot path on one MI355X.

Workload (one "step" = one decoded frame): batch 1, a seeded random-init model
with the reference's dims (12 layers, d 768, 12x64 heads, FF 3072, vocab 16384,
W8A16 Q8_0_4X4 weights), KV cache prefilled to context 512 with N(0,1) values
(fp16 cache), --steps greedy frames (min_frames = steps, so the end gate never
stops it; 256 frames fill the cache to position 767), two fused kernel launches
per frame.  A frame is what the reference's "ms/frame" counts: local 1-layer
transformer x 17, 16 audio heads + greedy picks, the W8A8 end gate, and the
12-layer global step.  The frame is timed without per-launch events; a second
run of the same frames records HIP events around each launch on the model's
stream, which gives the global-step and local-half times.

roofline: the frame's dominant kernel (the longer of decode_global_kernel and
decode_local_kernel): algorithmic bytes per launch over its average launch
duration from those events.  roofline_decode holds both kernels, roofline_gemv
the W8A16 GEMV at large N (K = 768, N = 262144, weights cycled through a 1 GiB
pool so they stream from HBM, not the 256 MB Infinity Cache).

cpu_baseline: the reference's own AVX2 CPU path (oracle/_ref, compiled from the
reference sources) decoding the same frames from the same context-512 state on
this host, at T = 4 threads (its published setting) and T = the CPU share of
this process (physical cores, affinity, cgroup quota and OMP_NUM_THREADS,
whichever is smallest); host_cpu reports lscpu's model, sockets and cores.

Also reported: the single GEMV (K = 768, N = 2304) replayed from a graph beside
the reference's gemv_par; single-query decode attention (12 x 64 heads, fp16
K/V) at contexts 128, 512, 1024 and 2048, warm and cold, beside the reference's
AVX2 attention on one host core; the 256-row prefill (ms; W8A8 as the
reference's prefill, against the 5.0 POP/s int8 MFMA peak, and W8A16 against
the 2.5 PFLOP/s fp16 peak) and 64 streams with contexts ~ U[64, 1024] decoded
128 frames in lock-step (aggregate frames/s), each next to the reference on the
host cores; the 64-stream engine's paged global attention alone
(attention_paged_64, moss_hip_attn_paged at those contexts and at their mean,
GB/s against the 8 TB/s HBM peak).

The audio codec decoder (decode_chunk, the engine's 8-frame chunks on a stream
past every window; ms/frame and the real-time factor, 80 ms of audio per frame)
is reported beside the reference AudioDecoder on min(6, share) host threads.

The same frames with an fp32 KV cache (the reference's precision) are timed as well
(decode_kv_fp32), and the W8A8 decode from the same state (decode_w8a8: the reference's
decode when MOSS_A16 is unset).  --mode gemm64 runs the 64-stream engine's GEMM shapes (M = 64) through
the operator ABI eagerly, for hardware-counter passes; --mode mall runs global steps warm and
with a 1 GiB sweep before each (Infinity Cache residency of the weights, A/B); --mode handoff
times a cross-workgroup hand-off of 4-64 KB per workgroup inside one launch (LL words, fenced
counter barriers) against a launch boundary (libmoss_probe.so).

Usage: python bench.py [--gpus 1] [--steps 256] [--warmup 8] [--no-cpu]
                       [--mode full|gemv|attn|attn64|decode|prefill|streams|codec|gemm64|mall|handoff]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "dsh-moss-tts_amd"))

HBM_PEAK_GBS = 8000.0
CTX = 512
GEMV_N, GEMV_K = 262144, 768
CAL_BYTES = 256 << 20
# HBM bytes per launch of the roofline kernel, from two hardware-counter passes over
# `bench.py --mode gemv` (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE; KiB per dispatch
# scaled by the 256 MiB calibration copy of that same run: fetch x2.0, write x1.0).
GEMV_TRAFFIC_BYTES = 214_956_032
CONFIG0_BYTES = 1_886_208  # (2304/4)(768/32)*136 weights + 2*768 x + 2*2304 y (fp16)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_state(seed: int = 2024):
    from mosship import moss_format as mf
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((12, CTX, 768), dtype=np.float32).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((12, CTX, 768), dtype=np.float32).astype(np.float16).astype(np.float32)
    hidden = rng.standard_normal(768, dtype=np.float32)
    rows = mf.text_rows(rng.integers(0, mf.VOCAB, CTX))
    return k, v, hidden, rows


def bench_decode(blob, state, steps, warmup, kv_fp32: bool = False, a8: bool = False):
    """The headline frame loop (fp16 KV), or with kv_fp32 the reference's own KV precision, or
    with a8 the W8A8 decode (the reference's with MOSS_A16 unset)."""
    import torch

    from mosship import HipLLM, SampleParams
    k, v, hidden, _ = state
    m = HipLLM(blob, device=0, kv_fp32=kv_fp32, decode_a8=a8)
    m.kv_import(k, v, hidden)
    m.snapshot_prefix()
    p = SampleParams.make(greedy=True, min_frames=max(steps, warmup))
    if warmup:
        m.generate(warmup, p)
        m.restore_prefix()
    m.set_hidden(hidden)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = m.generate(steps, p)  # as a caller runs it: no per-launch timing events
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    frames = len(out["rows"])
    assert frames == steps, f"decoded {frames} of {steps} frames"
    # the global / local split from a second run of the same frames with events
    m.restore_prefix()
    m.set_hidden(hidden)
    t = m.generate(steps, p, timing=True)["timing"]
    res = {
        "ms_per_frame": (t1 - t0) * 1e3 / frames,
        "global_ms_event": float(np.mean(t[:-1, 0])) if frames > 1 else 0.0,
        "local_ms_event": float(np.mean(t[:, 1])),
        "frames": frames,
        "end_position": m.position,
    }
    m.close()
    return res


def bench_gemv(reps: int = 60):
    """Large-N W8A16 GEMV on torch's current stream, timed with HIP events around
    `reps` launches; weights rotate through a pool larger than the MALL (cold) and,
    separately, one buffer is reused (warm)."""
    import torch

    from mosship import lib
    from mosship import moss_format as mf
    rows, cols = GEMV_N, GEMV_K
    wbytes = (rows // 4) * (cols // 32) * 136
    algo = wbytes + 2 * cols + 2 * rows
    rng = np.random.default_rng(42)
    host = mf.synth_q8x4(rng, rows, cols)
    pool_n = max(2, -(-(1 << 30) // wbytes))  # >= 1 GiB of distinct weights
    base = torch.from_numpy(host.reshape(-1)).cuda()
    pool = [base] + [torch.roll(base, 136 * 4 * (i + 1)) for i in range(pool_n - 1)]
    x = torch.from_numpy(rng.standard_normal(cols).astype(np.float16)).cuda()
    y = torch.empty(rows, dtype=torch.float16, device="cuda")
    s = torch.cuda.current_stream()
    for w in pool:
        lib.gemv_q8x4(w, rows, cols, x, y)
    torch.cuda.synchronize()
    out = {}
    for mode in ("cold", "warm"):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for i in range(reps):
            lib.gemv_q8x4(pool[i % pool_n] if mode == "cold" else pool[0], rows, cols, x, y)
        e1.record(s)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        out[mode] = {"us": us, "GBps": algo / us / 1e3}
    out["algo_bytes"] = algo
    out["pool_buffers"] = pool_n
    # the single GEMV at K=768, N=2304 (fp16 in/out): 200 launches captured in a graph
    # and replayed, so the time is the kernel's, not the host's launch rate
    w0 = torch.from_numpy(mf.synth_q8x4(rng, 2304, 768).reshape(-1)).cuda()
    y0 = torch.empty(2304, dtype=torch.float16, device="cuda")
    cap = torch.cuda.Stream()
    with torch.cuda.stream(cap):
        for _ in range(10):
            lib.gemv_q8x4(w0, 2304, 768, x, y0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        for _ in range(200):
            lib.gemv_q8x4(w0, 2304, 768, x, y0)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us0 = e0.elapsed_time(e1) * 1e3 / 200
    out["config0"] = {"us": us0, "GBps": CONFIG0_BYTES / us0 / 1e3, "timing": "200 launches replayed from a graph"}
    calibration_copy()
    return out


def calibration_copy():
    """One plain device copy of exactly 256 MiB: what FETCH_SIZE / WRITE_SIZE read for it
    scales the hardware byte counters of the kernels profiled in the same run."""
    import torch
    cal_src = torch.ones(CAL_BYTES, dtype=torch.uint8, device="cuda")
    cal_dst = torch.empty_like(cal_src)
    cal_dst.copy_(cal_src)
    torch.cuda.synchronize()


PREFILL_ROWS = 256
PREFILL_FLOP = 44_699_222_016  # 2*256*84,934,656 (GEMMs) + 144*256*32,896 (causal attention)
MFMA_F16_PEAK_TFLOPS = 2500.0
MFMA_I8_PEAK_TOPS = 5000.0
STREAMS, STREAM_STEPS = 64, 128


def prefill_rows(seed: int = 7):
    from mosship import moss_format as mf
    rng = np.random.default_rng(seed)
    return mf.text_rows(rng.integers(0, mf.VOCAB, PREFILL_ROWS))  # codes = pad, as make_text_row


def bench_prefill(blob, reps: int = 20, a16: bool = False):
    """256-row prefill from position 0 (KV written for decode), MFMA GEMMs: W8A8 (int8
    activations, the reference's prefill) by default, W8A16 with a16=True."""
    import torch

    from mosship import HipLLM
    rows = prefill_rows()
    m = HipLLM(blob, device=0, prefill_a16=a16)
    for _ in range(2):
        m.prefill(rows)
    times = []
    for _ in range(reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        m.prefill(rows)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    m.close()
    ms = float(np.median(times)) * 1e3
    tflops = PREFILL_FLOP / (ms * 1e-3) / 1e12
    # against the dense matrix-core peak of the arithmetic used: int8 (W8A8) or fp16 (W8A16)
    peak = MFMA_F16_PEAK_TFLOPS if a16 else MFMA_I8_PEAK_TOPS
    return {"ms": ms, "TFLOPs": tflops, "mfma_frac": tflops / peak}


GEMM64_SHAPES = ((2304, 768), (3072, 768), (768, 3072), (1024, 768))  # QKV, fc_in, fc_out, an audio head
SWEEP_BYTES = 1 << 30  # more than the 256 MB Infinity Cache (MALL) and every L2


def bench_mall(blob, state, steps: int = 40):
    """Infinity Cache residency of the global step's weights, shown by an A/B: `steps` global
    steps back to back (warm: the 90 MB of layer weights stay in the 256 MB MALL between
    steps), then `steps` more with a 1 GiB read-and-write sweep on the model's device before
    each (cold: every weight byte comes from HBM).  Each step is one decode_global_kernel
    launch; moss_hip_llm_global_step returns after it, so host time per step = launch and
    copies + kernel, the same overhead in both halves.  The kernel's own duration per half
    comes from a --kernel-trace run of this mode (launches in order: warm first)."""
    import torch

    from mosship import HipLLM
    from mosship import moss_format as mf
    k, v, hidden, _ = state
    m = HipLLM(blob, device=0)
    m.kv_import(k, v, hidden)
    rng = np.random.default_rng(3)
    rows = [np.array([mf.SLOT] + list(rng.integers(0, 1024, 16)), np.int32) for _ in range(2 * steps)]
    sweep = torch.empty(SWEEP_BYTES // 4, dtype=torch.float32, device="cuda")
    for r in rows[:4]:  # warm-up: the kernel and the weights resident
        m.global_step(r)
    m.kv_import(k, v, hidden)
    out = {}
    for mode in ("warm", "cold"):
        ts = []
        for r in rows[:steps] if mode == "warm" else rows[steps:]:
            if mode == "cold":
                sweep.add_(1.0)  # reads and writes 1 GiB: evicts the MALL and the L2s
                torch.cuda.synchronize()
            t0 = time.perf_counter()
            m.global_step(r)
            ts.append(time.perf_counter() - t0)
        out[mode] = {"host_us_per_step_median": round(float(np.median(ts)) * 1e6, 1)}
    out["steps_each"] = steps
    out["sweep_bytes"] = SWEEP_BYTES
    m.close()
    return out


HANDOFF_MODES = (("launch per round (graph)", 3), ("LL words, one launch", 2),
                 ("fence in every thread, one launch", 0), ("fence in one thread per workgroup, one launch", 1))
HANDOFF_BYTES = (4096, 16384, 65536)


def bench_handoff(rounds: int = 50):
    """Cost of handing bulk data from each of 256 workgroups to a workgroup on another XCD,
    per round, four ways: a kernel boundary (one launch per round, replayed from a graph),
    LL words inside one persistent launch, and a counter barrier with __threadfence() in every
    thread or in one thread per workgroup (libmoss_probe.so, csrc/probe_handoff.hip); 4, 16
    and 64 KB per workgroup.  Every value is checked; device time from HIP events."""
    import ctypes as C

    import torch
    torch.zeros(1, device="cuda")
    lib = C.CDLL(os.path.join(ROOT, "dsh-moss-tts_amd", "libmoss_probe.so"))
    lib.moss_probe_handoff.argtypes = [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_double)]
    out = {}
    for name, mode in HANDOFF_MODES:
        row = {}
        for nbytes in HANDOFF_BYTES:
            us = C.c_double(0.0)
            rc = lib.moss_probe_handoff(mode, rounds, nbytes // 4, C.byref(us))
            if rc != 0:
                raise RuntimeError(f"handoff probe {name}, {nbytes} B: error {rc}")
            row[f"{nbytes // 1024}KB"] = round(us.value, 2)
        out[name] = row
    out["unit"] = "us per round, 256 workgroups"
    return out


def bench_gemm64(reps: int = 20):
    """The 64-stream engine's GEMM shapes (M = 64) through the operator ABI, eagerly (no graphs):
    W8A16 (moss_hip_gemm_q8x4, fp32 activations) and W8A8 (moss_hip_gemm_q8x4_w8a8, int8
    activations quantised by moss_hip_quantize_rows), `reps` calls each -- the launches a
    hardware-counter pass profiles (rocprofv3 --pmc); times from HIP events on the stream."""
    import torch

    from mosship import lib
    from mosship import moss_format as mf
    M = 64
    rng = np.random.default_rng(64)
    s = torch.cuda.current_stream()
    out = {}
    for N, K in GEMM64_SHAPES:
        w = torch.from_numpy(mf.synth_q8x4(rng, N, K).reshape(-1)).cuda()
        x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()
        y = torch.empty((M, N), dtype=torch.float32, device="cuda")
        q = torch.empty((M, K), dtype=torch.int8, device="cuda")
        d = torch.empty((M, K // 32), dtype=torch.float32, device="cuda")
        lib.quantize_rows(x, M, K, q, d)
        res = {}
        for mode in ("w8a16", "w8a8"):
            call = (lambda: lib.gemm_q8x4(w, N, K, x, M, y)) if mode == "w8a16" else \
                (lambda: lib.gemm_q8x4_w8a8(w, N, K, q, d, M, y))
            call()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(reps):
                call()
            e1.record(s)
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / reps
            res[mode] = {"us": round(us, 2), "TOP/s": round(2 * M * N * K / us / 1e6, 2)}
        out[f"{N}x{K}"] = res
    return out


ATTN_CTX = (128, 512, 1024, 2048)


def bench_attention(reps: int = 100):
    """Single-query decode attention (12 heads x 64, fp16 K/V [12][ctx][64], fp32 q,
    fp16 output) at each context length: warm (one cache, Infinity-Cache resident) and
    cold (caches cycled through a pool of more than 512 MB), `reps` calls replayed from
    a graph.  Algorithmic bytes per call: K and V (2 * 2 * 768 * ctx) + q (4 * 768) +
    output (2 * 768)."""
    import torch

    from mosship import lib
    res = {}
    cap = torch.cuda.Stream()
    for ctx in ATTN_CTX:
        per = 2 * 12 * ctx * 64 * 2  # bytes of one K + V pair
        pool_n = max(2, -(-(512 << 20) // per))
        g = torch.Generator(device="cuda").manual_seed(ctx)
        kv = torch.randn((pool_n, 2, 12, ctx, 64), generator=g, device="cuda").to(torch.float16)
        q = torch.randn(768, generator=g, device="cuda")
        out = torch.empty(768, dtype=torch.float16, device="cuda")
        algo = 3072 * ctx + 4608
        r = {"algo_bytes": algo}
        with torch.cuda.stream(cap):  # warm-up on the capture stream (its split-KV scratch is made here)
            for i in range(min(pool_n, 16)):
                lib.attn_decode(q, kv[i, 0], kv[i, 1], 12, ctx, ctx, out)
        torch.cuda.synchronize()
        # the calls are captured in a graph and replayed, so the time is the kernels', not the host's
        for mode in ("cold", "warm"):
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=cap):
                for i in range(reps):
                    j = i % pool_n if mode == "cold" else 0
                    lib.attn_decode(q, kv[j, 0], kv[j, 1], 12, ctx, ctx, out)
            graph.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            graph.replay()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / reps
            r[f"us_{mode}"] = round(us, 3)
            r[f"GBps_{mode}"] = round(algo / us / 1e3, 1)
        r["frac_cold"] = round(r["GBps_cold"] / HBM_PEAK_GBS, 4)
        res[str(ctx)] = r
        del kv
    return res


def bench_attn64(reps: int = 20):
    """The 64-stream engine's paged global attention through moss_hip_attn_paged: 64 rows
    (one per stream, contexts ~ U[64, 1024] as the 64-stream workload), 12 heads x 64, fp16
    pages of 64 positions laid out as the engine lays them (page j of stream s at j * 64 + s),
    fp32 q and output.  12 launches per replay, one per layer's pools (2.3 GB in all, so
    every launch reads its pages from HBM, as a frame's 12 layers do), `reps` replays of a
    captured graph timed with HIP events on the capture stream.  Algorithmic bytes per
    launch: the rows' K and V (2 * 2 * 768 bytes per key) + q and output (2 * 64 * 768 * 4).
    Also timed: every row at the mean context (same bytes, no ragged tail)."""
    import torch

    from mosship import lib
    ctx = stream_contexts()
    rows, layers, page = STREAMS, 12, 64
    per = -(-int(ctx.max()) // page)
    g = torch.Generator(device="cuda").manual_seed(64)
    k = torch.randn((layers, per * rows, 12, page, 64), generator=g, device="cuda").to(torch.float16)
    v = torch.randn((layers, per * rows, 12, page, 64), generator=g, device="cuda").to(torch.float16)
    table = (torch.arange(per, device="cuda", dtype=torch.int32)[None, :] * rows +
             torch.arange(rows, device="cuda", dtype=torch.int32)[:, None]).contiguous()
    q = torch.randn((rows, 768), generator=g, device="cuda")
    out = torch.empty((rows, 768), dtype=torch.float32, device="cuda")
    cap = torch.cuda.Stream()
    res = {}
    order = np.argsort(-ctx, kind="stable").astype(np.int32)
    for kind, keys, rs in (("ragged", ctx, None), ("uniform", np.full_like(ctx, int(round(ctx.mean()))), None),
                           ("ragged_longest_first", ctx, order)):
        pos = torch.from_numpy(((keys if rs is None else keys[rs]) - 1).astype(np.int32)).cuda()
        rsd = None if rs is None else torch.from_numpy(rs).cuda()
        mk = int(keys.max())
        algo = int(3072 * keys.sum()) + 2 * rows * 768 * 4
        with torch.cuda.stream(cap):
            for l in range(layers):
                lib.attn_paged(q, k[l], v[l], 12, table, per, page, pos, mk, out, row_stream=rsd)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=cap):
            for l in range(layers):
                lib.attn_paged(q, k[l], v[l], 12, table, per, page, pos, mk, out, row_stream=rsd)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(cap):
            e0.record(cap)
            for _ in range(reps):
                graph.replay()
            e1.record(cap)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * layers)
        res[kind] = {"keys_total": int(keys.sum()), "keys_max": mk, "algo_bytes": algo, "us": round(us, 3),
                     "GBps": round(algo / us / 1e3, 1), "frac": round(algo / us / 1e3 / HBM_PEAK_GBS, 4)}
    del k, v
    return res


def cpu_attention(reps: int = 20):
    """The reference's AVX2 single-query attention (attn_avx2.cpp:93, one thread) at the
    same context lengths: ctx - 1 cached keys plus the query row's own k/v."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import RefCpu
    r = RefCpu(a16_mode="decode")
    rng = np.random.default_rng(5)
    out = {}
    for ctx in ATTN_CTX:
        qkv = rng.standard_normal(3 * 768).astype(np.float32)
        kc = rng.standard_normal((ctx - 1, 768)).astype(np.float16).astype(np.float32)
        vc = rng.standard_normal((ctx - 1, 768)).astype(np.float16).astype(np.float32)
        r.attention_window(qkv, kc, vc)
        t0 = time.perf_counter()
        for _ in range(reps):
            r.attention_window(qkv, kc, vc)
        out[str(ctx)] = round((time.perf_counter() - t0) / reps * 1e6, 2)
    return {"us": out, "threads": 1}


def stream_contexts(seed: int = 64, lo: int = 64, hi: int = 1024):
    return np.random.default_rng(seed).integers(lo, hi + 1, STREAMS)


def bench_streams(blob, steps: int = STREAM_STEPS):
    """64 independent streams, contexts ~ U[64, 1024], paged fp16 KV, `steps` greedy frames in lock-step."""
    from mosship import HipBatch, HipLLM, SampleParams
    ctx = stream_contexts()
    rng = np.random.default_rng(99)
    kmax = int(ctx.max())
    # N(0,1) fp16-representable KV; stream s uses the first ctx[s] positions
    k = rng.standard_normal((12, kmax, 768), dtype=np.float32).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((12, kmax, 768), dtype=np.float32).astype(np.float16).astype(np.float32)
    m = HipLLM(blob, device=0)
    b = HipBatch(m, max_streams=STREAMS, capacity=kmax + steps + 1)
    for s in range(STREAMS):
        b.set_stream(s, k[:, :ctx[s]], v[:, :ctx[s]], rng.standard_normal(768, dtype=np.float32))
    p = SampleParams.make(greedy=True, min_frames=steps)
    b.generate(STREAMS, 2, p)  # warm-up (captures the graphs)
    for s in range(STREAMS):
        b.set_stream(s, k[:, :ctx[s]], v[:, :ctx[s]], rng.standard_normal(768, dtype=np.float32))
    out = b.generate(STREAMS, steps, p)
    assert (out["frames"] == steps).all()
    b.close()
    m.close()
    kv_bytes = int(np.sum(36864 * (ctx + steps // 2 + 1)))  # mean context over the run, fp16 K+V, 12 layers
    step_bytes = 90728448 + STREAMS * 13872 + kv_bytes
    return {"ms_total": out["ms"], "frames_per_s": STREAMS * steps / (out["ms"] * 1e-3),
            "ms_per_step": out["ms"] / steps, "global_stack_GBps": step_bytes / (out["ms"] / steps * 1e-3) / 1e9}


CODEC_WARM_FRAMES = 130   # fills every stage's window (d1: 500 positions = 125 frames)
CODEC_CHUNK = 8           # the engine's default chunk_frames (engine.h:35)
CODEC_CHUNKS = 16
FP32_MFMA_PEAK_TFLOPS = 157.3


def codec_flops(blob, frames: int) -> float:
    """Algorithmic flops of `frames` frames of the codec decoder at steady state (every
    window full): the GEMMs (2 flops per multiply-add) and the windowed attention (QK^T and
    PV: 2 x 2 flops per query, key and channel)."""
    from mosship import codec_format as cf
    from mosship.moss_format import read_moss_index
    idx = read_moss_index(blob)
    dims = {n: (r, c) for n, (_, r, c, _, _) in idx.items()}
    f = frames * (cf.NQ * cf.Z_DIM * cf.CB_DIM * 2 + 2 * dims["q.out.w"][0] * dims["q.out.w"][1])
    rows = frames
    for s, p, nl, w in zip(cf.STAGES, cf.PATCHES, cf.LAYERS, cf.CONTEXTS):
        rows *= p
        f += 2 * rows * (dims[f"d{s}.in.w"][0] * dims[f"d{s}.in.w"][1] + dims[f"d{s}.out.w"][0] * dims[f"d{s}.out.w"][1])
        for n in range(nl):
            lp = f"d{s}.l{n}."
            macs = sum(dims[lp + m][0] * dims[lp + m][1] for m in ("attn.w", "proj.w", "f1.w", "f2.w"))
            f += 2 * rows * macs + 4 * rows * w * cf.D_MODEL
    return float(f)


def bench_codec(chunks: int = CODEC_CHUNKS):
    """Streaming codec decode (decoder.cpp:203-221) on the GPU: a stream warmed past every
    stage's window, then `chunks` chunks of 8 frames through decode_chunk (codes from the
    host, samples back to the host, one hipGraph replay per chunk), timed on the host."""
    from mosship import HipCodec
    from mosship import codec_format as cf
    from mosship.moss_format import DT_F16
    blob = cf.synth_codec(seed=3, dtype=DT_F16)
    rng = np.random.default_rng(5)
    c = HipCodec(blob)
    c.reset_stream()
    c.decode_chunk(rng.integers(0, cf.CB_SIZE, (cf.NQ, CODEC_WARM_FRAMES)))
    codes = [rng.integers(0, cf.CB_SIZE, (cf.NQ, CODEC_CHUNK)).astype(np.int32) for _ in range(chunks)]
    c.decode_chunk(codes[0])  # graph for 8-frame pieces captured
    t0 = time.perf_counter()
    for cc in codes:
        c.decode_chunk(cc)
    ms = (time.perf_counter() - t0) * 1e3 / chunks
    # whole-utterance decode of 64 frames (the reference's decode(), stage times from events)
    c.decode(rng.integers(0, cf.CB_SIZE, (cf.NQ, 64)))
    whole = {"frames": 64, "ms": round(c.last_ms, 3), "stage_ms": [round(x, 3) for x in c.stage_ms]}
    c.close()
    fl = codec_flops(blob, CODEC_CHUNK)
    tfs = fl / (ms * 1e-3) / 1e12
    return {"chunk_frames": CODEC_CHUNK, "ms_per_chunk": round(ms, 4), "ms_per_frame": round(ms / CODEC_CHUNK, 4),
            "rtf": round(ms / CODEC_CHUNK / 80.0, 5), "gflop_per_chunk": round(fl / 1e9, 3),
            "TFLOPs": round(tfs, 2), "fp32_mfma_frac": round(tfs / FP32_MFMA_PEAK_TFLOPS, 4), "whole_decode": whole,
            "blob": blob}


def cpu_codec(blob, threads: int, chunks: int = 4):
    """The reference AudioDecoder (oracle/_ref) on the same protocol: the stream warmed
    past every window, then `chunks` chunks of 8 frames, `threads` threads."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import RefCpu, RefDecoder
    from mosship import codec_format as cf
    rng = np.random.default_rng(5)
    d = RefDecoder(RefCpu(a16_mode="decode"), blob, threads=threads)
    try:
        d.reset_stream()
        d.decode_chunk(rng.integers(0, cf.CB_SIZE, (cf.NQ, CODEC_WARM_FRAMES)))
        codes = [rng.integers(0, cf.CB_SIZE, (cf.NQ, CODEC_CHUNK)).astype(np.int32) for _ in range(chunks)]
        t0 = time.perf_counter()
        for cc in codes:
            d.decode_chunk(cc)
        ms = (time.perf_counter() - t0) * 1e3 / chunks
    finally:
        d.close()
    return {"ms_per_frame": round(ms / CODEC_CHUNK, 3), "threads": threads,
            "sample": f"{chunks} chunks of {CODEC_CHUNK} frames after {CODEC_WARM_FRAMES} warm-up frames"}


def host_cpu():
    """The host's CPU as lscpu reports it, and the share of it this process may use:
    the smallest of the physical cores, the CPUs in its affinity mask, its cgroup
    quota and OMP_NUM_THREADS (the per-GPU share a shared GPU host sets)."""
    import subprocess
    info = {"model": "", "sockets": None, "physical_cores": None, "logical_cpus": os.cpu_count()}
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = {ln.split(":", 1)[0].strip(): ln.split(":", 1)[1].strip() for ln in txt.splitlines() if ":" in ln}
        info["model"] = kv.get("Model name", "")
        sockets = int(kv.get("Socket(s)", "0") or 0)
        per = int(kv.get("Core(s) per socket", "0") or 0)
        info["sockets"] = sockets or None
        info["physical_cores"] = sockets * per or None
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    if not info["model"]:
        try:
            with open("/proc/cpuinfo") as f:
                info["model"] = next(ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name"))
        except (OSError, StopIteration):
            pass
    limits = [n for n in (info["physical_cores"], len(os.sched_getaffinity(0))) if n]
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()[:2]
        if quota != "max":
            limits.append(max(1, int(int(quota) / int(period))))
    except (OSError, ValueError):
        pass
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        limits.append(int(os.environ["OMP_NUM_THREADS"]))
    info["cpu_share"] = max(1, min(limits)) if limits else 1
    return info


def cpu_prefill(blob, threads: int):
    """Reference prefill of the same 256 rows on `threads` threads: W8A8 (its release
    default) in this process, A16 (MOSS_A16=1) in a child process (the mode is read
    once per process, gemv.cpp:26-35)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import REF_SO, RefCpu
    if not os.path.exists(REF_SO):
        return None
    rows = prefill_rows()
    r = RefCpu(a16_mode="decode")
    m = r.model(blob, threads=threads)
    m.prefill(rows[:16])  # warm the thread pool and the weights
    t0 = time.perf_counter()
    m.prefill(rows)
    w8a8 = (time.perf_counter() - t0) * 1e3
    m.close()
    code = ("import sys, time, numpy as np; sys.path[:0] = [%r, %r]; from oracle import RefCpu;"
            "from mosship import moss_format as mf; r = RefCpu(a16_mode='1'); blob = open(sys.argv[1], 'rb').read();"
            "rows = np.load(sys.argv[2]); m = r.model(blob, threads=int(sys.argv[3])); m.prefill(rows[:16]);"
            "t0 = time.perf_counter(); m.prefill(rows);"
            "print((time.perf_counter() - t0) * 1e3)" % (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "dsh-moss-tts_amd")))
    import subprocess
    with tempfile.TemporaryDirectory() as td:
        bp, rp = os.path.join(td, "w.moss"), os.path.join(td, "rows.npy")
        with open(bp, "wb") as f:
            f.write(blob)
        np.save(rp, rows)
        a16 = float(subprocess.run([sys.executable, "-c", code, bp, rp, str(threads)], check=True,
                                   capture_output=True, text=True).stdout.strip().splitlines()[-1])
    return {"w8a8_ms": w8a8, "a16_ms": a16, "threads": threads}


def cpu_streams(blob, share: int, threads: int, frames: int = 32):
    """P = share // T concurrent reference LlmModels (T threads each) decoding greedy
    frames from their own states; contexts ~ U[64, 640] (the reference caps at 768)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import threading

    from oracle import REF_SO, RefCpu, SampleParams

    from mosship import moss_format as mf
    if not os.path.exists(REF_SO):
        return None
    procs = max(1, share // threads)
    ctx = stream_contexts(lo=64, hi=640)[:procs]
    rng = np.random.default_rng(99)
    r = RefCpu(a16_mode="decode")
    models, paths = [], []
    td = tempfile.mkdtemp(prefix="mossref_streams_")
    for i in range(procs):
        n = int(ctx[i % len(ctx)])
        k = rng.standard_normal((12, n, 768), dtype=np.float32).astype(np.float16).astype(np.float32)
        v = rng.standard_normal((12, n, 768), dtype=np.float32).astype(np.float16).astype(np.float32)
        rows = mf.text_rows(rng.integers(0, mf.VOCAB, n))
        path = os.path.join(td, f"s{i}.state")
        with open(path, "wb") as f:
            f.write(mf.write_state(k, v, rng.standard_normal(768, dtype=np.float32), rows, mf.fp_weights(blob)))
        mm = r.model(blob, threads=threads)
        mm.load_state(path, rows, ignore_fp=False)
        models.append(mm)
        paths.append(path)
    p = SampleParams.make(greedy=True, min_frames=frames)
    counts = [0] * procs

    def run(i):
        counts[i] = len(models[i].generate(frames, p)["rows"])

    ths = [threading.Thread(target=run, args=(i,)) for i in range(procs)]
    t0 = time.perf_counter()
    for t in ths:
        t.start()
    for t in ths:
        t.join()
    wall = time.perf_counter() - t0
    for mm in models:
        mm.close()
    for pth in paths:
        os.remove(pth)
    os.rmdir(td)
    return {"frames_per_s": sum(counts) / wall, "instances": procs, "threads_each": threads, "cores": procs * threads,
            "sample": f"{procs} concurrent LlmModel x {threads} threads, {frames} greedy frames each, "
                      f"ctx ~ U[64, 640]"}


def cpu_gemv(share: int):
    """The reference's gemv_par (MOSS_A16 on: row_dot_q8_4x4_actf32) on the single-GEMV
    shape K=768, N=2304: median of 1000 calls at T = 1 and T = the CPU share."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import REF_SO, RefCpu

    from mosship import moss_format as mf
    if not os.path.exists(REF_SO):
        return None
    rng = np.random.default_rng(42)
    w = mf.synth_q8x4(rng, 2304, 768).reshape(-1)
    x = rng.standard_normal(768).astype(np.float16).astype(np.float32)
    r = RefCpu(a16_mode="decode")
    out = {}
    for t in sorted({1, share}):
        us = r.gemv_median_us(w, 2304, 768, x, threads=t, reps=1000)
        out[f"T{t}"] = {"us": round(us, 2), "GBps": round(CONFIG0_BYTES / us / 1e3, 2)}
    return out


def cpu_baseline(blob, state, frames: int, share: int):
    """The compiled reference (oracle/_ref) decoding the same frames from the same
    ctx-512 state (MOSS_A16=decode, its release setting) at T = 4 (its published
    setting, README.md:40) and T = the CPU share; the faster is the baseline."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import REF_SO, RefCpu, SampleParams

    from mosship import moss_format as mf
    if not os.path.exists(REF_SO):
        return None
    k, v, hidden, rows = state
    r = RefCpu(a16_mode="decode")
    runs = {}
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "ctx512.state")
        with open(path, "wb") as f:
            f.write(mf.write_state(k, v, hidden, rows, mf.fp_weights(blob)))
        for threads in sorted({4, share}):
            m = r.model(blob, threads=threads)
            m.load_state(path, rows, ignore_fp=False)
            p = SampleParams.make(greedy=True, min_frames=frames)
            m.generate(3, p)  # 3-frame warmup (the reference's protocol)
            m.load_state(path, rows, ignore_fp=False)
            t0 = time.perf_counter()
            out = m.generate(frames, p, timing=True)
            t1 = time.perf_counter()
            n = len(out["rows"])
            t = out["timing"]
            m.close()
            runs[threads] = {"ms_per_frame": (t1 - t0) * 1e3 / n, "frames": n,
                             "global_ms": float(np.mean(t[:-1, 0])) if n > 1 else 0.0,
                             "local_ms": float(np.mean(t[:, 1]))}
    best = min(runs, key=lambda th: runs[th]["ms_per_frame"])
    b = runs[best]
    return {
        "value": round(b["ms_per_frame"], 3),
        "unit": "ms/frame",
        "cores": best,
        "kind": "reference",
        "sample": f"{b['frames']} greedy frames from the ctx-512 state (the GPU run's frames), MOSS_A16=decode; "
                  f"faster of T=" + " and T=".join(str(th) for th in sorted(runs)) + " threads",
        "by_threads": {str(th): {kk: round(vv, 3) for kk, vv in rr.items()} for th, rr in runs.items()},
    }


# Algorithmic bytes of the two launches of a batch-1 greedy frame (fp16 KV):
#  global step at position p: 12 layers of Q8_0_4X4 weights 90,243,072 + fp32 vectors
#  485,376 + embedding rows 13,872 + K/V read 36,864 (p + 1) + K/V write 36,864;
#  local half: 17 local steps x 7,566,336 + 16 audio heads 13,369,344 + the gate's
#  2 rows and the picks 15,504.
GLOBAL_FIXED_BYTES = 90_243_072 + 485_376 + 13_872 + 36_864
LOCAL_BYTES = 17 * 7_566_336 + 13_369_344 + 15_504
# Bytes per launch that leave the XCDs' L2 (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, over
# the default `bench.py --mode decode`, positions 512..767; KiB per dispatch scaled as the GEMV's:
# fetch x2.0, write x1.0, from the 256 MiB calibration copy of the same runs).  The global step
# fetches 1.08x its algorithmic bytes; the local half 0.22x (its layer's weights, re-read by each
# of the 17 local steps, stay in L2).
DECODE_TRAFFIC = {"decode_global_kernel": 123_908_065, "decode_local_kernel": 31_675_238}


def global_bytes(p: int) -> int:
    return GLOBAL_FIXED_BYTES + 36_864 * (p + 1)


def decode_rooflines(d):
    """Roofline objects of the frame's two kernels from the event-timed run: algorithmic
    bytes per launch (the global step's averaged over the positions it ran at) over the
    average launch duration."""
    p0, n = CTX, d["frames"]
    gb = float(np.mean([global_bytes(p) for p in range(p0, p0 + n - 1)])) if n > 1 else float(global_bytes(p0))
    out = {}
    for name, ms, nbytes in (("decode_global_kernel", d["global_ms_event"], gb),
                             ("decode_local_kernel", d["local_ms_event"], float(LOCAL_BYTES))):
        ach = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"kernel": name, "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": DECODE_TRAFFIC[name],
                     "algo_bytes_per_launch": round(nbytes), "us_per_launch": round(ms * 1e3, 2)}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--mode", choices=["full", "gemv", "attn", "attn64", "decode", "prefill", "streams", "codec", "gemm64",
                                       "mall", "handoff"], default="full")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    if args.steps < 2 or args.steps > 256:
        sys.exit("--steps must be in [2, 256]: the ctx-512 cache holds 256 more positions (kMaxCtx 768)")
    import torch
    if not torch.cuda.is_available():
        sys.exit("no GPU visible")
    from mosship import moss_format as mf

    if args.mode == "gemv":
        g = bench_gemv()
        print(json.dumps({"gemv": g}), flush=True)
        return
    if args.mode == "attn":
        print(json.dumps({"attention_decode": bench_attention()}), flush=True)
        return
    if args.mode == "gemm64":
        print(json.dumps({"gemm64": bench_gemm64()}), flush=True)
        return
    if args.mode == "attn64":
        print(json.dumps({"attention_paged_64": bench_attn64()}), flush=True)
        calibration_copy()  # scales the byte counters of a counter pass over this mode
        return
    if args.mode == "handoff":
        print(json.dumps({"handoff": bench_handoff()}), flush=True)
        return
    if args.mode == "codec":
        cd = bench_codec()
        cd.pop("blob")
        print(json.dumps({"codec": cd}), flush=True)
        return

    log("generating synthetic model + ctx-512 state")
    blob = mf.synth_model(1234)
    state = make_state()
    if args.mode == "prefill":
        print(json.dumps({"prefill": bench_prefill(blob), "prefill_a16": bench_prefill(blob, a16=True)}), flush=True)
        return
    if args.mode == "streams":
        print(json.dumps({"streams": bench_streams(blob)}), flush=True)
        return
    if args.mode == "mall":
        print(json.dumps({"mall": bench_mall(blob, state)}), flush=True)
        return
    log("decode")
    d = bench_decode(blob, state, args.steps, args.warmup)
    roof = decode_rooflines(d)
    if args.mode == "decode":
        calibration_copy()
        print(json.dumps({"decode": d, "rooflines": roof}), flush=True)
        return
    log("decode, fp32 KV")
    d32 = bench_decode(blob, state, args.steps, args.warmup, kv_fp32=True)
    log("decode, W8A8")
    da8 = bench_decode(blob, state, args.steps, args.warmup, a8=True)
    log("gemv roofline")
    g = bench_gemv()
    log("decode attention")
    at = bench_attention()
    log("prefill (256 rows)")
    pf = bench_prefill(blob)
    pf16 = bench_prefill(blob, a16=True)
    log("64 streams")
    st = bench_streams(blob)
    log("64-stream paged attention")
    a64 = bench_attn64()
    log("codec decoder")
    cd = bench_codec()
    cblob = cd.pop("blob")
    host = host_cpu()
    cpu = cpu_pf = cpu_at = cpu_gv = cpu_cd = None
    cpu_st = {}
    if not args.no_cpu:
        share = host["cpu_share"]
        log(f"cpu baseline (reference), share {share} cores")
        cpu = cpu_baseline(blob, state, args.steps, share)
        cpu_gv = cpu_gemv(share)
        cpu_at = cpu_attention()
        cpu_pf = cpu_prefill(blob, share)
        cpu_cd = cpu_codec(cblob, min(6, share))
        for t in sorted({1, 4}):
            r = cpu_streams(blob, share, t)
            if r:
                cpu_st[f"T{t}"] = r
    best_st = max(cpu_st.values(), key=lambda r: r["frames_per_s"]) if cpu_st else None
    # the roofline object is the frame's dominant kernel (the longer of its two launches)
    dom = max(roof.values(), key=lambda r: r["us_per_launch"])
    gemv_roof = {
        "kernel": f"gemv_stream_kernel (fp16 in/out), N={GEMV_N} K={GEMV_K}, weights cycled over "
                  f"{g['pool_buffers']} buffers (cold)",
        "bound": "hbm", "achieved": round(g["cold"]["GBps"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(g["cold"]["GBps"] / HBM_PEAK_GBS, 4), "traffic": GEMV_TRAFFIC_BYTES,
        "traffic_note": "bytes/launch from rocprofv3 FETCH_SIZE + WRITE_SIZE (calibrated), "
                        f"{GEMV_TRAFFIC_BYTES / g['algo_bytes']:.3f}x the algorithmic bytes",
    }
    end = d["end_position"]
    line = {
        "metric": "LLM decode ms/frame (bs1, ctx 512); frames/s @64 streams; GEMV GB/s",
        "value": round(d["ms_per_frame"], 4),
        "unit": "ms/frame",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(d["ms_per_frame"], 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "w8a16 (int8 weights, fp32 activations/accumulation, fp16 KV)",
        "data": "synthetic (seeded random-init weights with the reference's dims; N(0,1) fp16 KV at ctx 512)",
        "config": {"workload": f"LLM decode, batch 1, from ctx {CTX}: {d['frames']} greedy frames (positions "
                               f"{CTX}..{end}), two fused launches per frame (full frame = 17 local steps + "
                               f"16 heads + end gate + 12-layer global step)",
                   "global_batch": 1, "seq_len": CTX, "parallelism": "none (1 GPU)"},
        "frames_per_s": round(1e3 / d["ms_per_frame"], 1),
        "global_step_ms": round(d["global_ms_event"], 4),
        "local_ms_per_frame": round(d["local_ms_event"], 4),
        "decode_kv_fp32": {"ms_per_frame": round(d32["ms_per_frame"], 4),
                           "global_step_ms": round(d32["global_ms_event"], 4),
                           "local_ms_per_frame": round(d32["local_ms_event"], 4),
                           "note": "the same frames with an fp32 KV cache, the reference's own KV precision"},
        "decode_w8a8": {"ms_per_frame": round(da8["ms_per_frame"], 4),
                        "global_step_ms": round(da8["global_ms_event"], 4),
                        "local_ms_per_frame": round(da8["local_ms_event"], 4),
                        "note": "W8A8 decode (int8 activations, the reference's decode with MOSS_A16 unset), "
                                "fp16 KV, from the same state; its codes differ from the W8A16 run's"},
        "roofline": dom,
        "roofline_decode": roof,
        "roofline_gemv": gemv_roof,
        "gemv": {"cold_GBps": round(g["cold"]["GBps"], 1), "warm_GBps": round(g["warm"]["GBps"], 1),
                 "config0_us": round(g["config0"]["us"], 3), "config0_GBps": round(g["config0"]["GBps"], 1),
                 "config0_timing": g["config0"]["timing"], "cpu_ref": cpu_gv},
        "attention_decode": {"ctx": at, "cpu_ref": cpu_at},
        "prefill_256": {"mode": "w8a8 (the reference's prefill)", "ms": round(pf["ms"], 3),
                        "TOP/s": round(pf["TFLOPs"], 2), "mfma_frac": round(pf["mfma_frac"], 4),
                        "a16_ms": round(pf16["ms"], 3), "a16_mfma_frac": round(pf16["mfma_frac"], 4),
                        "cpu_ref": cpu_pf},
        "streams_64": {"frames_per_s": round(st["frames_per_s"], 1), "ms_per_step": round(st["ms_per_step"], 4),
                       "global_stack_GBps": round(st["global_stack_GBps"], 1), "cpu_ref": cpu_st or None,
                       "vs_cpu": round(st["frames_per_s"] / best_st["frames_per_s"], 1) if best_st else None},
        "attention_paged_64": a64,
        "codec": dict(cd, cpu_ref=cpu_cd,
                      vs_cpu=round(cpu_cd["ms_per_frame"] / cd["ms_per_frame"], 1) if cpu_cd else None),
        "host_cpu": host,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
