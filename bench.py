#!/usr/bin/env python3
"""Benchmark of the MI355X execution provider's hot path on one GPU.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--workload all|gemv|gemm|gqa|gqa_growing|gqa_shared|paged|decoder|
                                decoder_layouts|copy]

Primary line: int4 MatMulNBits decode GEMV (K=4096, N=11008, block 32, fp32
activations) as achieved HBM GB/s. A step is one MatMulNBits call; consecutive
steps rotate over >= 512 MB of distinct weight copies so every call streams its
weights from HBM, not from the 256 MB Infinity Cache. Launches are captured in a
HIP graph and replayed, and the per-launch duration is taken from HIP events
recorded on the stream the kernels run on.

Secondary measurements (same JSON line, "secondary"):
- the same GEMV at one GPU's share of an 8-way N split (N = 1376);
- the MFMA prefill GEMM (M=512, K=N=4096, fp16);
- the GQA decode step (B=8, H=32/8, hd=128, 4K context), with the growing and
  with the shared KV contract;
- the PagedAttention mixed batch;
- the int4 decoder (decode tokens/s and the prompt prefill).
On request (--workload decoder_layouts, not part of "all"): the Qwen2.5-0.5B,
Llama-3.2-1B, Phi-3.5-mini, Phi-4-mini and Mistral-7B decoder layouts, decode
program (where it applies) against the op-by-op path.

cpu_baseline: the same GEMV (and, for the decoder, its decode steps) on this
machine's host cores through the oracle's fp32 AVX2 MatMulNBits (oracle/fast.c,
OpenMP), timed on a bounded sample.
"""

from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "onnxruntime-mlx_amd")

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FP16_DENSE_TFLOPS = 2500.0     # MI355X dense fp16 MFMA
MALL_BYTES = 256 << 20         # Infinity Cache

METRIC = "int4 MatMulNBits GB/s (% HBM peak); int4 decoder decode tokens/sec, 1 GPU"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def load_pkg():
    if "ortmi" in sys.modules:
        return sys.modules["ortmi"]
    spec = importlib.util.spec_from_file_location(
        "ortmi", os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["ortmi"] = mod
    spec.loader.exec_module(mod)
    return mod


MIN_REPLAYS = 100
MIN_WARM_S = 0.2  # warm-up replays continue until this much wall time has passed


def timed_graph(torch, launch_batch, batch_len, steps, warmup):
    """Capture `launch_batch()` (batch_len launches) in a HIP graph and replay it:
    warm-up replays covering `warmup` launches and at least MIN_WARM_S seconds (the
    first tenths of a second of a fresh process measured up to 5% slower), then
    max(100, steps / batch_len) timed replays, each bracketed by HIP events on the
    replay stream. Returns
    (median gpu ms per launch, wall ms per launch, launches timed)."""
    import numpy as np

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        launch_batch()  # eager warm-up outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch_batch()
    reps_w = max(1, -(-warmup // batch_len))
    reps = max(MIN_REPLAYS, -(-steps // batch_len))
    tw = time.perf_counter()
    for _ in range(reps_w):
        g.replay()
    torch.cuda.synchronize()
    while time.perf_counter() - tw < MIN_WARM_S:
        for _ in range(reps_w):
            g.replay()
        torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    t0 = time.perf_counter()
    ev[0].record()
    for i in range(reps):
        g.replay()
        ev[i + 1].record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    per = np.array([ev[i].elapsed_time(ev[i + 1]) for i in range(reps)]) / batch_len
    n = reps * batch_len
    return float(np.median(per)), (t1 - t0) * 1e3 / n, n


def launched_kernel_names(torch, launch_one):
    """Names of the GPU kernels one call launches, read from the profiler's trace of
    that call (outside any timed region); [] if the profiler is unavailable."""
    try:
        from torch.profiler import ProfilerActivity, profile

        torch.cuda.synchronize()
        with profile(activities=[ProfilerActivity.CUDA]) as prof:
            launch_one()
            torch.cuda.synchronize()
        names = []
        for e in prof.events():
            if getattr(e, "device_type", None) is not None and "CUDA" in str(e.device_type):
                if e.name not in names and "Memcpy" not in e.name and "Memset" not in e.name:
                    names.append(e.name)
        return names
    except Exception as exc:  # the profiler is optional here
        log(f"kernel names unavailable: {exc}")
        return []


def timed_eager(torch, launch_one, steps, warmup):
    for i in range(warmup):
        launch_one(i)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for i in range(steps):
        launch_one(i)
    e1.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return e0.elapsed_time(e1) / steps, (t1 - t0) * 1e3 / steps, steps


# ------------------------------------------------------------------- workloads --

def bench_gemv(torch, ortmi, steps, warmup, shard=1):
    """The cfg1 GEMV; shard > 1 runs one GPU's share of an N-sharded layer (the
    first N / shard rows), the shape each GPU would run under tensor parallelism."""
    import ctypes

    from ortmi import workloads  # noqa: F401  (loaded as a submodule)

    wl = sys.modules["ortmi.workloads"]
    K, N = 4096, 11008
    A, B, s, zp = wl.mnb_gemv_config()
    if shard > 1:
        rows = N // shard
        B, s, zp = (x.reshape(N, -1)[:rows].copy() for x in (B, s, zp))
        N = rows
    bytes_per_call = B.nbytes + s.nbytes + zp.nbytes + A.nbytes + N * 4
    copies = max(2, -(-(2 * MALL_BYTES) // bytes_per_call))
    dA = torch.from_numpy(A).cuda()
    dB0, ds0, dz0 = (torch.from_numpy(x).cuda() for x in (B, s, zp))
    bufs = [(dB0, ds0, dz0)] + [(dB0.clone(), ds0.clone(), dz0.clone()) for _ in range(copies - 1)]
    Y = torch.empty((1, N), dtype=torch.float32, device="cuda")
    lib = ortmi.load_kernels()
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    args = [(ptr(dA), ptr(b), ptr(sc), ptr(z), ptr(Y)) for b, sc, z in bufs]

    def launch_batch():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for a, b, sc, z, y in args:
            rc = lib.ortmi_matmul_nbits(a, b, sc, z, y, 1, N, K, 4, 32, 1, st)
            if rc:
                raise RuntimeError(lib.ortmi_last_error().decode())

    def launch_one():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        a, b, sc, z, y = args[0]
        lib.ortmi_matmul_nbits(a, b, sc, z, y, 1, N, K, 4, 32, 1, st)

    names = launched_kernel_names(torch, launch_one)
    gpu_ms, wall_ms, n = timed_graph(torch, launch_batch, len(args), steps, warmup)
    gbs = bytes_per_call / (gpu_ms * 1e-3) / 1e9
    return dict(kernel=names[0] if len(names) == 1 else (names or None),
                bytes_per_call=bytes_per_call, copies=copies, gpu_ms=gpu_ms, wall_ms=wall_ms,
                launches=n, gbs=gbs, inputs=(A, B, s, zp))


def bench_gemm(torch, ortmi, steps, warmup, bf16=False):
    """The prefill GEMM config (fp16), or the same shape in bf16 (activations and
    scales rounded to bf16, the bf16 matrix-core path)."""
    import ctypes

    wl = sys.modules["ortmi.workloads"]
    M, K, N = 512, 4096, 4096
    A, B, s, zp = wl.mnb_gemm_config()
    tdt = torch.bfloat16 if bf16 else torch.float16
    dA, ds = (torch.from_numpy(x).to(tdt).cuda() for x in (A, s))
    dB, dz = (torch.from_numpy(x).cuda() for x in (B, zp))
    Y = torch.empty((M, N), dtype=tdt, device="cuda")
    code = 16 if bf16 else 10
    lib = ortmi.load_kernels()
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    a = (ptr(dA), ptr(dB), ptr(ds), ptr(dz), ptr(Y))

    def launch_batch():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for _ in range(10):
            rc = lib.ortmi_matmul_nbits(*a, M, N, K, 4, 32, code, st)
            if rc:
                raise RuntimeError(lib.ortmi_last_error().decode())

    gpu_ms, wall_ms, n = timed_graph(torch, launch_batch, 10, max(10, steps // 10),
                                     max(10, warmup // 10))
    flops = 2.0 * M * N * K
    tflops = flops / (gpu_ms * 1e-3) / 1e12
    return dict(kernel="mnb_gemm4_kernel", flops_per_call=flops, gpu_ms=gpu_ms, wall_ms=wall_ms,
                launches=n, tflops=tflops, mfma_frac=tflops / FP16_DENSE_TFLOPS)


def bench_gqa(torch, ortmi, steps, warmup):
    import ctypes

    wl = sys.modules["ortmi.workloads"]
    cfg = wl.gqa_decode_config()
    B, H, KV, hd, past = 8, 32, 8, 128, 4096
    kv_bytes = cfg["pk"].nbytes + cfg["pv"].nbytes
    copies = max(2, -(-(2 * MALL_BYTES) // (2 * kv_bytes)))
    dq, dk, dv = (torch.from_numpy(cfg[x]).cuda() for x in ("q", "k", "v"))
    dcos, dsin = torch.from_numpy(cfg["cos"]).cuda(), torch.from_numpy(cfg["sin"]).cuda()
    pk0, pv0 = torch.from_numpy(cfg["pk"]).cuda(), torch.from_numpy(cfg["pv"]).cuda()
    pasts = [(pk0, pv0)] + [(pk0.clone(), pv0.clone()) for _ in range(copies - 1)]
    presents = [(torch.empty((B, KV, past + 1, hd), dtype=torch.float16, device="cuda"),
                 torch.empty((B, KV, past + 1, hd), dtype=torch.float16, device="cuda"))
                for _ in range(copies)]
    out = torch.empty((B, 1, H * hd), dtype=torch.float16, device="cuda")
    lib = ortmi.load_kernels()
    ws_bytes = lib.ortmi_group_query_attention_workspace_size(B, 1, H, hd, past + 1)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    total = past + 1

    def launch_batch():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for (pk, pv), (prk, prv) in zip(pasts, presents):
            rc = lib.ortmi_group_query_attention(
                ptr(dq), ptr(dk), ptr(dv), ptr(pk), ptr(pv), past, total, ptr(dcos), ptr(dsin),
                hd // 2, 8192, ptr(out), ptr(prk), ptr(prv), B, 1, H, KV, hd, 0.0, 0, 10, ptr(ws),
                ws_bytes, st)
            if rc:
                raise RuntimeError(lib.ortmi_last_error().decode())

    gpu_ms, wall_ms, n = timed_graph(torch, launch_batch, copies, max(copies, steps // 20),
                                     max(copies, warmup // 20))
    read = kv_bytes
    write = 2 * B * KV * (past + 1) * hd * 2
    small = (B * H * hd * 2) * 2 + (B * KV * hd * 2) * 2
    total_bytes = read + write + small
    return dict(kernels="gqa_prep + gqa_decode + attn_merge", contract="growing",
                bytes_per_call=total_bytes, copies=copies, gpu_ms=gpu_ms, wall_ms=wall_ms,
                launches=n, gbs=total_bytes / (gpu_ms * 1e-3) / 1e9)


def bench_gqa_shared(torch, ortmi, steps, warmup):
    """The same decode step with present bound to past (in-place contract): the
    4096 cached rows are read, only the new row is written."""
    import ctypes

    wl = sys.modules["ortmi.workloads"]
    cfg = wl.gqa_decode_config()
    B, H, KV, hd, past = 8, 32, 8, 128, 4096
    cap = past + 1
    kv_bytes = cfg["pk"].nbytes + cfg["pv"].nbytes
    copies = max(2, -(-(2 * MALL_BYTES) // kv_bytes))
    dq, dk, dv = (torch.from_numpy(cfg[x]).cuda() for x in ("q", "k", "v"))
    dcos, dsin = torch.from_numpy(cfg["cos"]).cuda(), torch.from_numpy(cfg["sin"]).cuda()
    caches = []
    for _ in range(copies):
        kc = torch.empty((B, KV, cap, hd), dtype=torch.float16, device="cuda")
        vc = torch.empty_like(kc)
        kc[:, :, :past].copy_(torch.from_numpy(cfg["pk"]))
        vc[:, :, :past].copy_(torch.from_numpy(cfg["pv"]))
        caches.append((kc, vc))
    out = torch.empty((B, 1, H * hd), dtype=torch.float16, device="cuda")
    lib = ortmi.load_kernels()
    ws_bytes = lib.ortmi_group_query_attention_workspace_size(B, 1, H, hd, cap)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

    def launch_batch():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for kc, vc in caches:
            rc = lib.ortmi_group_query_attention(
                ptr(dq), ptr(dk), ptr(dv), ptr(kc), ptr(vc), cap, past + 1, ptr(dcos), ptr(dsin),
                hd // 2, 8192, ptr(out), ptr(kc), ptr(vc), B, 1, H, KV, hd, 0.0, 0, 10, ptr(ws),
                ws_bytes, st)
            if rc:
                raise RuntimeError(lib.ortmi_last_error().decode())

    gpu_ms, wall_ms, n = timed_graph(torch, launch_batch, copies, max(copies, steps // 20),
                                     max(copies, warmup // 20))
    small = (B * H * hd * 2) * 2 + (B * KV * hd * 2) * 2 * 2
    total_bytes = kv_bytes + small
    return dict(kernels="gqa_decode + attn_merge", contract="shared",
                bytes_per_call=total_bytes, copies=copies, gpu_ms=gpu_ms, wall_ms=wall_ms,
                launches=n, gbs=total_bytes / (gpu_ms * 1e-3) / 1e9)


def bench_paged(torch, ortmi, steps, warmup):
    """The mixed batch through the C ABI with a preallocated workspace; each call is
    timed by HIP events on its stream, median over >= 100 calls. Calls rewrite the
    same cache slots with the same values, so every call does identical work."""
    import ctypes

    import numpy as np

    wl = sys.modules["ortmi.workloads"]
    cfg = wl.paged_mixed_config()
    d = {k: torch.from_numpy(cfg[k]).cuda() for k in ("q", "k", "v", "kc", "vc", "cum", "past", "bt")}
    H, KV, hd, blk = cfg["H"], cfg["KV"], cfg["hd"], cfg["blk"]
    T, batch = int(cfg["cum"][-1]), len(cfg["cum"]) - 1
    nblk, maxb = d["kc"].shape[0], d["bt"].shape[1]
    lib = ortmi.load_kernels()
    wsb = lib.ortmi_paged_attention_workspace_size(T, batch, H, KV, hd, hd, maxb * blk)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    out = torch.empty((T, H * hd), dtype=torch.float16, device="cuda")
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

    def launch_one(_i=0):
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        rc = lib.ortmi_paged_attention(
            p(d["q"]), p(d["k"]), p(d["v"]), p(d["kc"]), p(d["vc"]), nblk, blk, p(d["cum"]),
            p(d["past"]), p(d["bt"]), batch, maxb, T, maxb * blk, None, None, 0, 0, 0, 0, None,
            None, None, None, 1e-6, p(out), H, KV, hd, hd, 0.0, 10, p(ws), wsb, st)
        if rc:
            raise RuntimeError(lib.ortmi_last_error().decode())

    for i in range(max(3, warmup // 200)):
        launch_one(i)
    torch.cuda.synchronize()
    reps = max(MIN_REPLAYS, steps // 20)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    t0 = time.perf_counter()
    ev[0].record()
    for i in range(reps):
        launch_one(i)
        ev[i + 1].record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / reps
    gpu_ms = float(np.median([ev[i].elapsed_time(ev[i + 1]) for i in range(reps)]))
    n = reps
    nbytes, flops = wl.paged_work(cfg)
    return dict(kernels="paged_prep + paged_tilemap + paged_tile + paged_merge",
                bytes_per_call=nbytes, flops_per_call=flops, gpu_ms=gpu_ms, wall_ms=wall_ms,
                launches=n, gbs=nbytes / (gpu_ms * 1e-3) / 1e9,
                tflops=flops / (gpu_ms * 1e-3) / 1e12, tokens=int(cfg["new"].sum()),
                total_context=int(cfg["ctx"].sum()))


def bench_copy(torch, steps, warmup):
    """Plain device copy of a known size, for calibrating rocprofv3 byte counters."""
    n = 512 << 20
    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)

    def one(_i):
        b.copy_(a)

    gpu_ms, wall_ms, k = timed_eager(torch, one, max(5, steps // 100), 2)
    return dict(bytes_read=n, bytes_written=n, gpu_ms=gpu_ms, gbs=2 * n / (gpu_ms * 1e-3) / 1e9)


def bench_decoder(torch, ortmi, prompt_len=512, gen=128):
    """Int4 decoder through the EP: prompt prefill, then greedy decode steps.

    The feeds are placed as a stock ONNX Runtime places them for an EP whose memory
    device is HBM: input ids, seqlens_k and total_sequence_length are host tensors
    that the harness copies to HBM through the EP's data transfer each run; the KV
    cache and the logits are bound to device buffers and the ArgMax output to host
    memory (IOBinding). The graph ends in ArgMax(logits), so a greedy step is one
    EP run over the whole graph for one token, its id landing in host memory for
    the application to feed next, timed on the wall clock with the device
    synchronised at both ends, as a serving loop sees it. Also reported: the graph without the ArgMax node (the application takes
    the argmax of the logits on the device), and the ids bound in HBM as well."""
    import importlib

    import numpy as np

    dec = importlib.import_module("ortmi.decoder")
    cfg = dec.DecoderConfig()
    w = dec.make_weights(cfg, seed=4)
    cap = prompt_len + gen
    # The decoder ending in an ArgMax node: the EP's decode program writes the greedy
    # id to the graph output.
    runner = dec.DecoderRunner(cfg, w, cap=cap, max_prompt=prompt_len, argmax_node=True,
                               host_feeds=True)
    # The same decoder without it: the application's argmax over the logits.
    runner_app = dec.DecoderRunner(cfg, w, cap=cap, max_prompt=prompt_len, host_feeds=True)
    # The ids bound in HBM too (the argmax output fed back in place).
    runner_dev = dec.DecoderRunner(cfg, w, cap=cap, max_prompt=prompt_len)
    del w
    prompt = np.random.default_rng(44).integers(0, cfg.vocab, size=prompt_len)
    runner.generate(prompt[:16], steps=4)  # warm-up: allocations and first launches
    tokens, ttft, times = runner.generate(prompt, steps=gen)
    dec_s = float(np.sum(times))
    # The reference's benchmark times session.run alone on fixed feeds (median;
    # bench/bench.py:68-76). Its counterpart here: the same one-token EP run
    # repeated at the final context (each run rewrites the same KV row), the device
    # synchronised around it, without the greedy argmax that feeds the next token.
    length = runner.length - 1
    runner.ids_host[0, 0] = int(runner.next_id.reshape(-1)[0].item())
    run_times = []
    for _ in range(max(20, gen // 2)):
        runner.length = length
        t1 = time.perf_counter()
        runner.run(runner.ids_host[:, :1], 1)
        torch.cuda.synchronize()
        run_times.append(time.perf_counter() - t1)
    runner.length = length + 1
    runner_app.generate(prompt[:16], steps=4)
    tokens_app, _, times_app = runner_app.generate(prompt, steps=gen)
    del runner_app
    runner_dev.generate(prompt[:16], steps=4)
    tokens_dev, _, times_dev = runner_dev.generate(prompt, steps=gen)
    del runner_dev
    tok_s = len(times) / dec_s
    wbytes = cfg.weight_bytes()
    # KV read per token at the mean decode context, K and V, all layers.
    mean_ctx = prompt_len + gen / 2
    kv = cfg.layers * 2 * cfg.kv_heads * cfg.head_dim * 2 * mean_ctx
    per_tok = wbytes + kv
    return dict(tok_s=tok_s, ms_per_token=dec_s / len(times) * 1e3, ttft_ms=ttft * 1e3,
                prefill_tok_s=prompt_len / ttft, bytes_per_token=int(per_tok),
                gbs=per_tok * tok_s / 1e9, tokens=tokens[:8], n_decode=len(times),
                p50_ms=float(np.median(times)) * 1e3,
                run_p50_ms=float(np.median(run_times)) * 1e3,
                app_tok_s=len(times_app) / float(np.sum(times_app)),
                app_p50_ms=float(np.median(times_app)) * 1e3,
                app_same_tokens=tokens_app == tokens,
                dev_tok_s=len(times_dev) / float(np.sum(times_dev)),
                dev_p50_ms=float(np.median(times_dev)) * 1e3, dev_same_tokens=tokens_dev == tokens)


def measured_traffic(profile: str):
    """HBM bytes per launch from the committed counter summary (two rocprofv3 --pmc
    passes, FETCH_SIZE and WRITE_SIZE, scaled by a copy of known size), or None."""
    import re

    path = os.path.join(ROOT, "profiles", profile)
    try:
        with open(path) as f:
            m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", f.read(), re.M)
    except OSError:
        return None
    return int(m.group(1)) if m else None


# Decoder layouts of the reference's documented models besides the headline one:
# name -> (DecoderConfig fields, description).
DECODER_LAYOUTS = {
    "qwen2.5_0.5b": (dict(layers=24, hidden=896, heads=14, kv_heads=2, head_dim=64, inter=4864,
                          vocab=151936, max_pos=4096),
                     "Qwen2.5-0.5B layout: 24 layers, hidden 896, 14/2 heads, hd 64, SwiGLU 4864, "
                     "vocab 151936"),
    "llama3.2_1b": (dict(layers=16, hidden=2048, heads=32, kv_heads=8, head_dim=64, inter=8192,
                         vocab=128256, max_pos=4096, rope_base=5e5),
                    "Llama-3.2-1B layout: 16 layers, hidden 2048, 32/8 heads, hd 64, SwiGLU 8192, "
                    "vocab 128256"),
    # The decoders behind the reference's published decode comparisons; hidden 3072
    # and 4096 are outside the decode program's envelope, so they run op by op.
    # Rotary here is the plain table over the whole head (the models' own LongRoPE
    # scaling and Phi-4-mini's partial rotary change no byte counts).
    "phi3.5_mini": (dict(layers=32, hidden=3072, heads=32, kv_heads=32, head_dim=96, inter=8192,
                         vocab=32064, max_pos=4096, rope_base=1e4),
                    "Phi-3.5-mini layout: 32 layers, hidden 3072, 32/32 heads, hd 96, SwiGLU "
                    "8192, vocab 32064"),
    "phi4_mini": (dict(layers=32, hidden=3072, heads=24, kv_heads=8, head_dim=128, inter=8192,
                       vocab=200064, max_pos=4096, rope_base=1e4),
                  "Phi-4-mini layout: 32 layers, hidden 3072, 24/8 heads, hd 128, SwiGLU 8192, "
                  "vocab 200064"),
    "mistral_7b": (dict(layers=32, hidden=4096, heads=32, kv_heads=8, head_dim=128, inter=14336,
                        vocab=32768, max_pos=4096, rope_base=1e6),
                   "Mistral-7B layout: 32 layers, hidden 4096, 32/8 heads, hd 128, SwiGLU 14336, "
                   "vocab 32768"),
}


def bench_decoder_layout(torch, name, prompt_len=512, gen=128):
    """A decoder layout of DECODER_LAYOUTS (random int4 weights) through the EP, fed
    as in bench_decoder (host ids, ArgMax node): greedy decode on the decode program
    (ORTMI_EP_PROGRAM=require; reported as not applying, with the reason, for a
    layout outside its envelope) and op by op (ORTMI_EP_PROGRAM=0)."""
    import numpy as np

    dec = importlib.import_module("ortmi.decoder")
    fields, desc = DECODER_LAYOUTS[name]
    cfg = dec.DecoderConfig(**fields)
    w = dec.make_weights(cfg, seed=4)
    prompt = np.random.default_rng(44).integers(0, cfg.vocab, size=prompt_len)
    out, toks = {}, {}
    prev = os.environ.get("ORTMI_EP_PROGRAM")
    try:
        for mode, key in (("require", "program"), ("0", "op_path")):
            os.environ["ORTMI_EP_PROGRAM"] = mode
            r = dec.DecoderRunner(cfg, w, cap=prompt_len + gen, max_prompt=prompt_len,
                                  argmax_node=True, host_feeds=True)
            try:
                r.generate(prompt[:16], steps=4)
            except RuntimeError as exc:
                if key != "program" or "decode program" not in str(exc):
                    raise
                out[key] = dict(applies=False, reason=str(exc)[:240])
                toks[key] = None
                del r
                torch.cuda.empty_cache()
                continue
            tokens, ttft, times = r.generate(prompt, steps=gen)
            toks[key] = tokens
            out[key] = dict(decode_tok_s=round(len(times) / float(np.sum(times)), 1),
                            p50_ms_per_token=round(float(np.median(times)) * 1e3, 3),
                            prefill_ms=round(ttft * 1e3, 2),
                            weights_gb_s=round(cfg.weight_bytes() * len(times) /
                                               float(np.sum(times)) / 1e9, 1))
            del r
            torch.cuda.empty_cache()
    finally:
        if prev is None:
            os.environ.pop("ORTMI_EP_PROGRAM", None)
        else:
            os.environ["ORTMI_EP_PROGRAM"] = prev
    out["config"] = (f"{desc}, int4 block 32 random weights; {prompt_len}-token prompt then "
                     f"{gen} greedy tokens, batch 1, host-fed ids, ArgMax node")
    if toks["program"] is not None:
        a, b = toks["program"], toks["op_path"]
        out["same_tokens"] = a == b
        if a != b:
            # Free-running greedy decodes part at the first near-tie of the logits and
            # then follow different prompts; the teacher-forced comparison is in the tests.
            out["first_divergence"] = next(i for i in range(min(len(a), len(b)) + 1)
                                           if i == min(len(a), len(b)) or a[i] != b[i])
    out["first_tokens"] = (toks["program"] or toks["op_path"])[:8]
    return out


def cpu_baseline_decoder(budget_s=15.0, prompt_len=512):
    """The same int4 decoder's greedy decode steps on the host cores, the way a CPU
    runs them: every MatMulNBits through the oracle's fp32 AVX2 kernel (fast.c,
    OpenMP), one-token attention and the other ops in fp32 numpy, rounding to fp16
    at op outputs as the graph stores them. The KV cache of the 512-token context is
    filled with random fp16 rows instead of a CPU prefill (a decode step's work does
    not depend on the cached values); steps run from context 513 until the budget or
    the 640-token capacity. tokens/s = 1 / median step time."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import importlib

    import numpy as np
    import oracle

    dec = importlib.import_module("ortmi.decoder")
    cfg = dec.DecoderConfig()
    w = dec.make_weights(cfg, seed=4)
    cap = prompt_len + 128
    rng = np.random.default_rng(7)
    shape = (1, cfg.kv_heads, cap, cfg.head_dim)
    kr = [rng.standard_normal(shape).astype(np.float16).astype(np.float32)
          for _ in range(cfg.layers)]
    vr = [rng.standard_normal(shape).astype(np.float16).astype(np.float32)
          for _ in range(cfg.layers)]
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    tok, length, times = 47650, prompt_len, []
    oracle.decoder_forward(w, cfg, [tok], kr, vr, length + 1, fast=True)  # warm-up
    t_start = time.perf_counter()
    while (len(times) < 3 or time.perf_counter() - t_start < budget_s) and length < cap:
        t1 = time.perf_counter()
        r = oracle.decoder_forward(w, cfg, [tok], kr, vr, length + 1, fast=True)
        tok = int(np.argmax(r[0]))
        times.append(time.perf_counter() - t1)
        length += 1
    med = float(np.median(times))
    return dict(value=round(1.0 / med, 3), unit="tokens/s", cores=threads, kind="port",
                sample=f"{len(times)} greedy decode steps of the same 28-layer int4 decoder at "
                       f"context {prompt_len + 1}-{length}: MatMulNBits in the oracle's fp32 "
                       f"AVX2 kernel (OpenMP {threads} threads), attention and the other ops in "
                       f"fp32 numpy, KV cache rows random; median {med * 1e3:.1f} ms per token")


def cpu_baseline_gemv(inputs, budget_s=12.0):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle

    A, B, s, zp = inputs
    K, N = A.shape[1], B.shape[0]
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    nbytes = B.nbytes + s.nbytes + zp.nbytes + A.nbytes + N * 4
    # Rotate over copies of the weights (>= 512 MB in all), so that every call reads
    # them from DRAM, not from the CPU's last-level cache.
    copies = [(B, s, zp)] + [(B.copy(), s.copy(), zp.copy())
                             for _ in range(max(1, (512 << 20) // nbytes))]
    times = []
    oracle.mnb_matmul_fast(A[0], B, s, zp, N, K, 32, nthreads=threads)  # warm-up
    t_start = time.perf_counter()
    while (len(times) < 3 or time.perf_counter() - t_start < budget_s) and len(times) < 2000:
        Bi, si, zi = copies[len(times) % len(copies)]
        t0 = time.perf_counter()
        oracle.mnb_matmul_fast(A[0], Bi, si, zi, N, K, 32, nthreads=threads)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return dict(value=nbytes / med / 1e9, unit="GB/s", cores=threads, kind="port",
                sample=f"{len(times)} full K=4096 N=11008 int4 GEMV calls of the oracle's fp32 "
                       f"AVX2 kernel (fast.c: block-folded zero points, OpenMP {threads} "
                       f"threads), rotating over {len(copies)} weight copies; median "
                       f"{med * 1e3:.3f} ms per call")


# ------------------------------------------------------------------------ main --

def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--workload", default="all",
                    choices=["all", "gemv", "gemm", "gqa", "gqa_growing", "gqa_shared", "paged",
                             "decoder", "decoder_layouts", "copy"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--layouts", default="",
                    help="decoder_layouts: comma-separated names (default: every layout)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: there is no multi-GPU path (the kernels are "
              "measured at one GPU's share); run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    ortmi = load_pkg()
    import importlib

    importlib.import_module("ortmi.workloads")
    dev = torch.cuda.get_device_properties(0)
    log(f"device: {dev.name} CUs={dev.multi_processor_count}")

    wl = args.workload
    if wl == "copy":
        r = bench_copy(torch, args.steps, args.warmup)
        log(json.dumps(r))
        return 0
    secondary = {}
    gemv = None
    if wl in ("all", "gemv"):
        gemv = bench_gemv(torch, ortmi, args.steps, args.warmup)
        log(f"gemv: {gemv['gbs']:.1f} GB/s ({gemv['gpu_ms'] * 1e3:.2f} us/call)")
        r = bench_gemv(torch, ortmi, args.steps, args.warmup, shard=8)
        secondary["gemv_shard_of_8"] = {
            "config": "one GPU's share of the same GEMV sharded 8 ways along N: M=1 K=4096 "
                      "N=1376, fp32",
            "gbs": round(r["gbs"], 1), "us_per_call": round(r["gpu_ms"] * 1e3, 2),
            "bytes_per_call": r["bytes_per_call"],
            "roofline": {"bound": "hbm", "achieved": round(r["gbs"], 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(r["gbs"] / HBM_PEAK_GBS, 4)}}
        log(f"gemv shard 1/8: {r['gbs']:.1f} GB/s ({r['gpu_ms'] * 1e3:.2f} us/call)")
    if wl in ("all", "gemm"):
        r = bench_gemm(torch, ortmi, args.steps, args.warmup)
        secondary["mnb_gemm_prefill"] = {
            "config": "M=512 K=4096 N=4096 bits=4 block=32 fp16, zero points U{0..15}",
            "tflops": round(r["tflops"], 2), "us_per_call": round(r["gpu_ms"] * 1e3, 2),
            "roofline": {"bound": "mfma", "achieved": round(r["tflops"], 2),
                         "peak": FP16_DENSE_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(r["mfma_frac"], 4)}}
        log(f"gemm: {r['tflops']:.1f} TFLOP/s ({r['gpu_ms'] * 1e3:.2f} us/call)")
        r = bench_gemm(torch, ortmi, args.steps, args.warmup, bf16=True)
        secondary["mnb_gemm_prefill_bf16"] = {
            "config": "the same GEMM in bf16 (activations and scales rounded to bf16)",
            "tflops": round(r["tflops"], 2), "us_per_call": round(r["gpu_ms"] * 1e3, 2),
            "roofline": {"bound": "mfma", "achieved": round(r["tflops"], 2),
                         "peak": FP16_DENSE_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(r["mfma_frac"], 4)}}
        log(f"gemm bf16: {r['tflops']:.1f} TFLOP/s ({r['gpu_ms'] * 1e3:.2f} us/call)")
    if wl in ("all", "gqa", "gqa_growing"):
        r = bench_gqa(torch, ortmi, args.steps, args.warmup)
        secondary["gqa_decode"] = {
            "config": "B=8 H=32 KV=8 hd=128 past=4096 fp16 rotary, growing contract",
            "gbs": round(r["gbs"], 1), "us_per_call": round(r["gpu_ms"] * 1e3, 2),
            "bytes_per_call": r["bytes_per_call"],
            "roofline": {"bound": "hbm", "achieved": round(r["gbs"], 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(r["gbs"] / HBM_PEAK_GBS, 4)}}
        log(f"gqa: {r['gbs']:.1f} GB/s ({r['gpu_ms'] * 1e3:.2f} us/call)")
    if wl in ("all", "gqa", "gqa_shared"):
        r = bench_gqa_shared(torch, ortmi, args.steps, args.warmup)
        secondary["gqa_decode_shared"] = {
            "config": "B=8 H=32 KV=8 hd=128 past=4096 fp16 rotary, shared (in-place) contract",
            "gbs": round(r["gbs"], 1), "us_per_call": round(r["gpu_ms"] * 1e3, 2),
            "bytes_per_call": r["bytes_per_call"],
            "roofline": {"bound": "hbm", "achieved": round(r["gbs"], 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(r["gbs"] / HBM_PEAK_GBS, 4)}}
        log(f"gqa shared: {r['gbs']:.1f} GB/s ({r['gpu_ms'] * 1e3:.2f} us/call)")
    if wl in ("all", "paged"):
        r = bench_paged(torch, ortmi, args.steps, args.warmup)
        secondary["paged_attention_mixed"] = {
            "config": "32 seqs ctx U[256,8192], 4 prefill x 256 + 28 decode, block 16, "
                      "H=32 KV=8 hd=128 fp16",
            "gbs": round(r["gbs"], 1), "tflops": round(r["tflops"], 2),
            "us_per_call": round(r["gpu_ms"] * 1e3, 2),
            "roofline": {"bound": "hbm", "achieved": round(r["gbs"], 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(r["gbs"] / HBM_PEAK_GBS, 4)}}
        log(f"paged: {r['gbs']:.1f} GB/s {r['tflops']:.1f} TFLOP/s ({r['gpu_ms'] * 1e3:.1f} us)")

    if wl in ("all", "decoder"):
        r = bench_decoder(torch, ortmi)
        secondary["int4_decoder"] = {
            "config": "28 layers, hidden 1536, 12/2 heads, hd 128, SwiGLU 8960, vocab 151936, "
                      "int4 block 32; 512-token prompt then 128 greedy tokens, batch 1",
            "decode_tok_s": round(r["tok_s"], 1), "ms_per_token": round(r["ms_per_token"], 3),
            "p50_ms_per_token": round(r["p50_ms"], 3), "prefill_ms": round(r["ttft_ms"], 2),
            # The EP run alone, as the reference's bench times session.run (median),
            # without reading the id back.
            "run_only_p50_ms": round(r["run_p50_ms"], 3),
            "run_only_tok_s": round(1e3 / r["run_p50_ms"], 1),
            # The graph without the trailing ArgMax: the application's argmax on the
            # device over the logits output.
            "app_argmax_tok_s": round(r["app_tok_s"], 1),
            "app_argmax_p50_ms": round(r["app_p50_ms"], 3),
            "app_argmax_same_tokens": r["app_same_tokens"],
            # Input ids bound in HBM as well (IOBinding of every feed but the two
            # int32 scalars), the argmax output fed back in place.
            "device_ids_tok_s": round(r["dev_tok_s"], 1),
            "device_ids_p50_ms": round(r["dev_p50_ms"], 3),
            "device_ids_same_tokens": r["dev_same_tokens"],
            "feeds": "input ids, seqlens_k, total_sequence_length in host memory, copied to "
                     "HBM by the EP's data transfer (ORT's placement rule); KV cache and "
                     "logits bound in HBM; the ArgMax output (the greedy id) bound to host "
                     "memory",
            "prefill_tok_s": round(r["prefill_tok_s"], 1),
            "bytes_per_token": r["bytes_per_token"],
            "roofline": {"bound": "hbm", "achieved": round(r["gbs"], 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(r["gbs"] / HBM_PEAK_GBS, 4)},
            "first_tokens": r["tokens"]}
        log(f"decoder: {r['tok_s']:.1f} tok/s ({r['ms_per_token']:.3f} ms/token, p50 "
            f"{r['p50_ms']:.3f}), prefill {r['ttft_ms']:.1f} ms; EP run alone p50 "
            f"{r['run_p50_ms']:.3f} ms; application argmax {r['app_tok_s']:.1f} tok/s (p50 "
            f"{r['app_p50_ms']:.3f} ms, same tokens: {r['app_same_tokens']}); ids in HBM "
            f"{r['dev_tok_s']:.1f} tok/s (same tokens: {r['dev_same_tokens']})")
        if not args.no_cpu_baseline:
            cpu_dec = cpu_baseline_decoder()
            secondary["int4_decoder"]["cpu_baseline"] = cpu_dec
            log(f"decoder cpu baseline: {cpu_dec['value']} tok/s on {cpu_dec['cores']} threads")

    if wl == "decoder_layouts":  # not part of "all": further decoder layouts on request
        names = [n for n in args.layouts.split(",") if n] or list(DECODER_LAYOUTS)
        for name in names:
            secondary[f"int4_decoder_{name}"] = r = bench_decoder_layout(torch, name)
            prog = (f"program {r['program']['decode_tok_s']} tok/s" if "decode_tok_s" in r["program"]
                    else "program does not apply")
            log(f"{name}: {prog}, op path {r['op_path']['decode_tok_s']} tok/s"
                f"{', same tokens ' + str(r['same_tokens']) if 'same_tokens' in r else ''}")

    if gemv is None:
        print(json.dumps({"workload": wl, "secondary": secondary}))
        return 0
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_gemv(gemv["inputs"])
        log(f"cpu baseline: {cpu['value']:.2f} GB/s on {cpu['cores']} threads")
    line = {
        "metric": METRIC,
        "value": round(gemv["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gemv["gpu_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "MatMulNBits decode GEMV: M=1 K=4096 N=11008 bits=4 block=32, fp32 "
                        "activations/scales, zero points all 8",
            "weights_rotated_over_bytes": gemv["bytes_per_call"] * gemv["copies"],
            "parallelism": "single GPU",
            "timing": f"median over {gemv['launches'] // gemv['copies']} HIP-graph replays of "
                      f"{gemv['copies']} launches each ({gemv['launches']} launches timed), "
                      f"HIP events on the replay stream; wall {gemv['wall_ms'] * 1e3:.2f} us "
                      f"per launch",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gemv["gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gemv["gbs"] / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic("mnb_gemv_k4096_n11008_f32.md"),
            "kernel": gemv["kernel"],
            "us_per_launch": round(gemv["gpu_ms"] * 1e3, 3),
            "bytes_per_launch": gemv["bytes_per_call"],
        },
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
