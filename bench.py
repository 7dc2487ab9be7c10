"""Headline benchmark: decode QK^T + attn.V on packed 4-bit KV at 32k context (one MI355X).

Workload H (BASELINE.json metric, configs[4] shape with 4-bit K and V, one
layer, every token quantized): B=8, 32 query heads over 8 KV heads (GQA 4),
head_dim 128, T=32768, asym groups of 32 (K along head_dim, V along tokens).
A step is one decode-attention call of the product path (QK^T GEMV, fp32
softmax -> fp16, attn.V GEMV with its split-T combine) for one new query
token per sequence.  Inputs are resident in HBM; the packed caches rotate
over --copies independent copies (>= 1 GiB) so every step reads cold data
past the 256 MiB Infinity Cache.

value = algorithmic packed-code + metadata bytes of both GEMVs / step time,
the steps timed back to back on the GPU (time_backlogged; the median of three
loops of exactly --steps steps).
roofline = the dominant kernel (the fused flash-decoding split kernel, which
reads every packed byte) alone: the split stage of the step exactly as the step
launches it (iq_decode_attention_splits_live: the same kernel and grid, live
split slots), launched back to back in the same rotation and timed the same way
with HIP events on the stream it runs on (medians of three loops of at least
100 launches, alternating with full steps over the same launch count); traffic = its HBM bytes from rocprofv3 FETCH_SIZE / WRITE_SIZE
(profiles/traffic.json).  cpu_baseline = the
reference's torch CPU path (dequantize int32 codes -> fp16 -> eager
attention) on a sample of the same workload, timed on host cores
(oracle/timing.py).

    python bench.py [--gpus 1] [--steps 100] [--warmup 10]
    python bench.py --config {H,1,2,3,4}    other BASELINE configs (not the headline line)
    python bench.py --config {base,small_preset,hybrid,hybrid_k,base_padded}
                                            the reference's presets at the config-4 shape
                                            (hybrid_k: innerq_hybrid with hybrid keys too;
                                            base_padded: innerq_base, a left-padded batch)
"""
from __future__ import annotations

import argparse
import json
import statistics
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

METRIC = "decode QK^T+attn·V µs/step and HBM GB/s (% of peak) at 32k ctx, 4-bit"
PEAK_GBS = 8000.0


def gemv_bytes(B, Hkv, T, D, G, bits, mode, axis):
    m = 4 if mode == "asymmetric" else 2
    groups = T * (D // G) if axis == "channel" else (T // G) * D
    return B * Hkv * (T * D * bits // 8 + groups * m)


def make_store(axis, B, Hkv, T, D, G, bits, mode, seed, dev, n_out=4, factor=10.0):
    import torch
    from innerq_amd import ops
    gen = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(B, Hkv, T, D, generator=gen, device=dev, dtype=torch.float32)
    ch = torch.randperm(D, generator=torch.Generator().manual_seed(seed))[:n_out].to(dev)
    x[..., ch] *= factor
    x = x.to(torch.float16)
    st = ops.PackedStore(axis, B, Hkv, D, G, bits, mode, dev, t_cap=T)
    st.append(x)
    del x
    return st


def clock_warmup(dev, ms: float = 40.0) -> None:
    """Bring the GPU out of its idle power state before anything is timed: plain
    256 MiB device copies for about ``ms`` milliseconds.  Without it the first
    ~200 decode steps after an idle period run up to ~15% slower while the
    clocks ramp (measured per launch with HIP events: 67.7 -> 60.1 us for the
    fused kernel over the first 13 ms of back-to-back steps), so a short
    warm-up of the workload itself would time the ramp."""
    import torch
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(2000):  # bounded: ~70 us per copy, stops at ``ms``
        for _ in range(20):
            dst.copy_(src)
        e1.record()
        e1.synchronize()
        if e0.elapsed_time(e1) >= ms:
            break
    del src, dst


def time_loop(fn, n, warmup):
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(n):
        fn(i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n * 1e3  # us per call


def time_graph(fn, reps, n):
    """GPU time per call: `reps` calls captured in one HIP graph and replayed n
    times, so the Python/ctypes launch cost of each call is not in the timing."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on the capture stream: its workspace exists before capture
        for i in range(reps):
            fn(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        for i in range(reps):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (n * reps) * 1e3


# host threads a one-GPU job may use on the GPU boxes (their CPU share per GPU),
# whatever os.cpu_count() reports for the whole host
CPU_SHARE = 16


def gpu_backlog(dev, ms: float = 25.0) -> None:
    """Queue about ``ms`` milliseconds of plain 256 MiB device copies on the
    current stream and return without waiting: the host then enqueues the loop
    that follows while the GPU is still busy, so that loop runs back to back on
    the GPU even where the host (or the runtime's bookkeeping of the queued
    launches) now and then falls behind the GPU."""
    import torch
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(int(ms / 0.07) + 1):  # ~70 us per copy
        dst.copy_(src)


def time_backlogged(fn, n, warmup, backlog_ms=25.0):
    """GPU time per call of n back-to-back calls: after `warmup` untimed calls
    and a synchronize, the calls are enqueued behind a GPU backlog (gpu_backlog)
    and timed with HIP events on the stream they run on, bracketed by
    synchronizes.  Host launch cost and any host-side stall of the runtime stay
    outside the timed GPU interval, as in a replayed graph."""
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    gpu_backlog(stream.device, ms=max(backlog_ms, 0.12 * n))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(n):
        fn(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n * 1e3  # us per call


def cpu_baseline(B, Hq, Hkv, T, D, G, bk, bv, step_bytes, budget_s=12.0):
    from oracle import timing
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    threads = max(1, min(CPU_SHARE, usable))
    sample_b = 1
    sec, reps = timing.time_reference(sample_b, Hq, Hkv, T, D, G, bk, bv, threads, min_seconds=budget_s)
    step_s = sec * (B / sample_b)
    return {"value": round(step_bytes / step_s / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "us_per_step": round(step_s * 1e6, 1),
            "sample": f"{reps} reference steps of 1 of the {B} sequences (Hq={Hq}, Hkv={Hkv}, T={T}, D={D}, "
                      f"int32 codes -> fp32 dequant -> fp16 -> eager attention, torch CPU, {threads} threads), "
                      f"scaled x{B // sample_b}",
            "cpu": _cpu_model(), "torch_threads": threads, "host_cpus": os.cpu_count(), "usable_cpus": usable,
            "cpu_share": CPU_SHARE}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def traffic_from_profiles(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter summary
    (FETCH_SIZE and WRITE_SIZE passes scaled by a plain-copy calibration), or None."""
    path = os.path.join(HERE, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(kernel, {}).get("bytes")
    except (OSError, ValueError, AttributeError):
        return None


def bench_headline(args):
    import torch
    from innerq_amd import ops
    dev = torch.device("cuda:0")
    B, Hq, Hkv, D, T, G, bits, mode = 8, 32, 8, 128, 32768, 32, 4, "asymmetric"
    scale = D ** -0.5
    ks = [make_store("channel", B, Hkv, T, D, G, bits, mode, 100 + c, dev) for c in range(args.copies)]
    vs = [make_store("token", B, Hkv, T, D, G, bits, mode, 200 + c, dev) for c in range(args.copies)]
    q = torch.randn(B, Hq, D, device=dev, dtype=torch.float16)
    out = torch.empty(B, Hq, D, device=dev, dtype=torch.float16)
    C = args.copies

    def step(i):
        ops.decode_attention(q, None, ks[i % C], None, None, vs[i % C], None, scale, out=out)

    def split_stage(i):  # the step's launch of the fused split kernel (every token packed, one format)
        return ops.decode_attention_splits_live(q, None, ks[i % C], None, None, vs[i % C], None, scale)

    clock_warmup(dev)
    # the step: the median of three timed loops of exactly K steps each
    us_step = statistics.median(time_backlogged(step, args.steps, args.warmup) for _ in range(3))
    # the dominant kernel: the split stage alone (one launch of the fused split
    # kernel), at least 100 back-to-back launches in the same rotation right
    # after the timed loops, timed the same way; HIP events between the two
    # kernels of each step would add ~3 us of marker latency to every bracketed
    # launch (measured), so the kernel is timed on its own.  The full step over
    # the same number of launches alternates with it (three of each, medians):
    # a step is the kernel plus the combine, so only noise can put the kernel
    # above the step, and a line where it still does says so.
    nl = max(100, args.steps)
    plan = split_stage(0)
    nsplit, grid = plan.nsplit, plan.grid
    splits, steps_nl = [], []
    for _ in range(3):
        splits.append(time_backlogged(split_stage, nl, C))
        steps_nl.append(time_backlogged(step, nl, C))
    us_split, us_step_nl = statistics.median(splits), statistics.median(steps_nl)
    inverted = us_split > min(us_step, us_step_nl)
    if inverted:
        print(f"warning: split stage {us_split:.2f} us above the step ({us_step:.2f} / {us_step_nl:.2f} us)",
              file=sys.stderr)

    qk_b = gemv_bytes(B, Hkv, T, D, G, bits, mode, "channel")
    av_b = gemv_bytes(B, Hkv, T, D, G, bits, mode, "token")
    step_b = qk_b + av_b
    value = step_b / (us_step * 1e-6) / 1e9
    ach = step_b / (us_split * 1e-6) / 1e9
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us_step / 1e3, 5), "us_per_step": round(us_step, 2),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "frac_of_hbm_peak": round(value / PEAK_GBS, 4),
        "dtype": "u4 codes, f16 operands, f32 accumulate", "data": "synthetic (seeded torch.randn K/V, 4 outlier "
                                                                      "channels x10, quantized by the product path)",
        "config": {"workload": "H: one-layer decode attention, B=8, Hq=32, Hkv=8, D=128, T=32768 all quantized, "
                               "4-bit K (groups along head_dim) and V (groups along tokens), asym, G=32",
                   "global_batch": B, "seq_len": T, "parallelism": "single GPU", "copies_rotated": C,
                   "algorithmic_bytes_per_step": step_b},
        "kernels_us": {"flash_fused_kernel": round(us_split, 2), "splits": nsplit, "workgroups": grid, "launches": nl,
                       "step_us_same_rotation": round(us_step_nl, 2), **({"kernel_above_step": True} if inverted else {})},
        "roofline": {"bound": "hbm", "kernel": "flash_fused_kernel", "achieved": round(ach, 1), "peak": PEAK_GBS,
                     "unit": "GB/s", "frac": round(ach / PEAK_GBS, 4),
                     "traffic": traffic_from_profiles("flash_fused_kernel"), "algorithmic_bytes": step_b},
    }
    if args.gemvs:
        logits = torch.empty(B, Hq, T, device=dev, dtype=torch.float32)
        p = torch.softmax(torch.randn(B, Hq, T, device=dev) * 2.0, dim=-1).to(torch.float16)
        o32 = torch.empty(B, Hq, D, device=dev, dtype=torch.float32)
        us_qk = time_loop(lambda i: ops.qk_gemv(q, ks[i % C], scale, out=logits), args.steps, args.warmup)
        us_av = time_loop(lambda i: ops.av_gemv(p, vs[i % C], out32=o32), args.steps, args.warmup)
        line["kernels_us"].update(qk_gemv=round(us_qk, 2), av_gemv_incl_records_combine=round(us_av, 2),
                                  qk_GBs=round(qk_b / us_qk / 1e3, 1), av_GBs=round(av_b / us_av / 1e3, 1))
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(B, Hq, Hkv, T, D, G, bits, bits, step_b)
    print(json.dumps(line), flush=True)


def bench_config(args):
    """Non-headline BASELINE configs, one JSON line each: us = per call through the
    Python API (host launch cost included), us_graph = the same calls replayed from
    a captured HIP graph (16 calls per graph: a replay's own launch gap, a few us,
    is spread over them), us_gpu = the same calls enqueued behind a GPU backlog
    (time_backlogged, median of three loops: back-to-back GPU time, the headline's
    timing)."""
    import torch
    from innerq_amd import ops
    dev = torch.device("cuda:0")
    C = args.copies
    cfg = args.config
    res = {"config": cfg}
    if cfg == "1":
        B, Hq, Hkv, D, T, G = 1, 32, 8, 128, 8192, 32
        ks = [make_store("channel", B, Hkv, T, D, G, 4, "asymmetric", 10 + c, dev) for c in range(C)]
        q = torch.randn(B, Hq, D, device=dev, dtype=torch.float16)
        lg = torch.empty(B, Hq, T, device=dev)
        fn = lambda i: ops.qk_gemv(q, ks[i % C], D ** -0.5, out=lg)
        clock_warmup(dev)
        us = time_loop(fn, args.steps, args.warmup)
        ug = time_graph(fn, 4 * C, max(1, args.steps // 4))
        ub = statistics.median(time_backlogged(fn, args.steps, args.warmup) for _ in range(3))
        b = gemv_bytes(B, Hkv, T, D, G, 4, "asymmetric", "channel")
        res.update(us=us, GBs=b / us / 1e3, us_graph=ug, GBs_graph=b / ug / 1e3, us_gpu=ub, GBs_gpu=b / ub / 1e3,
                   bytes=b)
    elif cfg == "2":
        B, Hq, Hkv, D, T, G = 8, 32, 8, 128, 32768, 64
        for mode in ("asymmetric", "symmetric"):
            vs = [make_store("token", B, Hkv, T, D, G, 2, mode, 20 + c, dev) for c in range(C)]
            p = torch.softmax(torch.randn(B, Hq, T, device=dev) * 2.0, dim=-1).to(torch.float16)
            out = torch.empty(B, Hq, D, device=dev, dtype=torch.float16)
            fn = lambda i: ops.av_gemv(p, vs[i % C], out=out)
            clock_warmup(dev)
            us = time_loop(fn, args.steps, args.warmup)
            ug = time_graph(fn, 4 * C, max(1, args.steps // 4))
            ub = statistics.median(time_backlogged(fn, args.steps, args.warmup) for _ in range(3))
            b = gemv_bytes(B, Hkv, T, D, G, 2, mode, "token")
            res[mode] = dict(us=us, GBs=b / us / 1e3, us_graph=ug, GBs_graph=b / ug / 1e3, us_gpu=ub,
                             GBs_gpu=b / ub / 1e3, frac_gpu=b / ub / 1e3 / PEAK_GBS, bytes=b)
            del vs
    elif cfg == "3":
        B, Hq, Hkv, D, T, G, R = 16, 32, 8, 128, 16384, 32, 128
        Tq = T - R
        ks = [make_store("channel", B, Hkv, Tq, D, G, 3, "symmetric", 30 + c, dev) for c in range(C)]
        vs = [make_store("token", B, Hkv, Tq, D, G, 3, "symmetric", 40 + c, dev) for c in range(C)]
        kr = torch.randn(B, Hkv, R, D, device=dev, dtype=torch.float16)
        vr = torch.randn(B, Hkv, R, D, device=dev, dtype=torch.float16)
        q = torch.randn(B, Hq, D, device=dev, dtype=torch.float16)
        knew = torch.randn(B, Hkv, 1, D, device=dev, dtype=torch.float16)
        out = torch.empty(B, Hq, D, device=dev, dtype=torch.float16)
        ap = [make_store("channel", B, Hkv, 64, D, G, 3, "symmetric", 50, dev) for _ in range(1)][0]

        def step(i):
            ops.decode_attention(q, None, ks[i % C], kr, None, vs[i % C], vr, D ** -0.5, out=out)
            ap.length = 0
            ap.append(knew)  # quantize-on-append of one token per sequence (K, flush 1)

        clock_warmup(dev)

        us = time_loop(step, args.steps, args.warmup)
        ug = time_graph(step, 4 * C, max(1, args.steps // 4))
        ub = statistics.median(time_backlogged(step, args.steps, args.warmup) for _ in range(3))
        b = 2 * gemv_bytes(B, Hkv, Tq, D, G, 3, "symmetric", "channel")
        res.update(us=us, GBs=b / us / 1e3, us_graph=ug, GBs_graph=b / ug / 1e3, us_gpu=ub, GBs_gpu=b / ub / 1e3,
                   frac_gpu=b / ub / 1e3 / PEAK_GBS, bytes=b)
    elif cfg == "4":
        B, Hq, Hkv, D, T, G, R, L = 8, 32, 8, 128, 32768, 32, 128, 32
        Tq = T - R
        ks = [make_store("channel", B, Hkv, Tq, D, G, 2, "asymmetric", 60 + l, dev) for l in range(L)]
        vs = [make_store("token", B, Hkv, Tq, D, G, 4, "asymmetric", 100 + l, dev) for l in range(L)]
        kr = torch.randn(B, Hkv, R, D, device=dev, dtype=torch.float16)
        vr = torch.randn(B, Hkv, R, D, device=dev, dtype=torch.float16)
        q = torch.randn(B, Hq, D, device=dev, dtype=torch.float16)
        out = torch.empty(B, Hq, D, device=dev, dtype=torch.float16)

        def step(i):
            for l in range(L):
                ops.decode_attention(q, None, ks[l], kr, None, vs[l], vr, D ** -0.5, out=out)

        clock_warmup(dev)

        us = time_loop(step, max(1, args.steps // 10), 2)
        ug = time_graph(step, 1, max(1, args.steps // 10))
        ub = statistics.median(time_backlogged(step, max(1, args.steps // 10), 2) for _ in range(3))
        b = L * (gemv_bytes(B, Hkv, Tq, D, G, 2, "asymmetric", "channel")
                 + gemv_bytes(B, Hkv, Tq - Tq % G, D, G, 4, "asymmetric", "token"))
        res.update(us=us, us_per_layer=us / L, GBs=b / us / 1e3, us_graph=ug, us_per_layer_graph=ug / L,
                   GBs_graph=b / ug / 1e3, us_gpu=ub, us_per_layer_gpu=ub / L, GBs_gpu=b / ub / 1e3,
                   frac_gpu=b / ub / 1e3 / PEAK_GBS, bytes=b)
    elif cfg in ("base", "small_preset", "hybrid", "hybrid_k", "base_padded"):
        # the reference's presets (scripts/run_lmeval.sh:94-153; innerq_amd.presets) at
        # the config-4 shape: a drop-in cache layer prefilled with 32k tokens (32 fp16
        # sinks, 32640 packed, 96 recent per role), then decode steps of the product
        # path: append() (window append, the K token's and, every 32 steps, the V
        # group's quantize-on-append) + attend() (fused kernel over the packed range,
        # the merging dense kernel over sinks and windows).  Four layers rotate, so each
        # step reads cold data; a timed loop covers whole 32-step V flush cycles of
        # every layer.  Store capacity is reserved before timing (no reallocation).
        from innerq_amd import cache as IC
        from innerq_amd import presets
        name = {"base": "innerq_base", "small_preset": "innerq_small", "hybrid": "innerq_hybrid",
                "hybrid_k": "innerq_hybrid", "base_padded": "innerq_base"}[cfg]
        over = {"key_quantize_mode": "hybrid"} if cfg == "hybrid_k" else {}  # cache.py:92-98
        # base_padded: the leading tokens a left-padding mask hides per sequence
        # (six distinct starts: six decode calls per step)
        pads = [0, 0, 64, 64, 300, 1024, 4096, 9000] if cfg == "base_padded" else None
        B, Hq, Hkv, D, T, L = 8, 32, 8, 128, 32768, 4
        gen = torch.Generator(device=dev).manual_seed(300)

        def kv(n):
            x = torch.randn(B, Hkv, n, D, generator=gen, device=dev)
            x[..., :: D // 4] *= 8.0  # outlier channels
            return x.to(torch.float16)

        layers = []
        for l in range(L):
            layer = IC.InnerqDynamicLayer(presets.preset_config(name, **over), l)
            layer.update(kv(T), kv(T))
            layer._kq.store.reserve(T + 4096)
            layer._vq.store.reserve(T + 4096)
            layers.append(layer)
        kn, vn = kv(1), kv(1)
        q = torch.randn(B, Hq, 1, D, generator=gen, device=dev).to(torch.float16)

        def step(i):
            layer = layers[i % L]
            layer.append(kn, vn)
            layer.attend(q, D ** -0.5, pads)

        clock_warmup(dev)
        cyc = 32 * L
        n = max(1, args.steps // cyc) * cyc
        us = statistics.median(time_backlogged(step, n, cyc) for _ in range(3))
        lay = layers[0]
        b = lay._kq.store.nbytes() + lay._vq.store.nbytes()  # packed bytes one step reads (layer 0, at the end)
        if pads:
            b = b * (1.0 - sum(pads) / (B * lay.attend_length()))  # the tokens the batch attends to
        res.update(preset=name + (" + hybrid K" if over else "") + (" (left-padded batch)" if pads else ""),
                   us=us, GBs=b / us / 1e3, frac=b / us / 1e3 / PEAK_GBS, bytes=b, steps=n, pads=pads,
                   k_packed=lay._kq.length, v_packed=lay._vq.length,
                   k_window=lay.keys_recent.shape[2], v_window=lay.values_recent.shape[2])
    elif cfg == "small":
        # not a BASELINE config: one sequence (B=1) decode steps and attn.V
        # calls, where a head is spread over many workgroups (a fused run per
        # workgroup, many split slots for the combine); 4-bit K and V (attn.V:
        # 2-bit G=64 V), with and without a 128-token fp16 window
        D, G = 128, 32
        clock_warmup(dev)
        for Hkv, T, R in ((8, 32768, 0), (8, 32768, 128), (8, 131072, 0), (8, 131072, 128),
                          (1, 131072, 0), (1, 131072, 128)):
            B, Hq, Tq = 1, 4 * Hkv, T - R
            ks = make_store("channel", B, Hkv, Tq, D, G, 4, "asymmetric", 70, dev)
            vs = make_store("token", B, Hkv, Tq, D, G, 4, "asymmetric", 71, dev)
            kr = torch.randn(B, Hkv, R, D, device=dev, dtype=torch.float16) if R else None
            vr = torch.randn(B, Hkv, R, D, device=dev, dtype=torch.float16) if R else None
            q = torch.randn(B, Hq, D, device=dev, dtype=torch.float16)
            out = torch.empty(B, Hq, D, device=dev, dtype=torch.float16)
            fn = lambda i: ops.decode_attention(q, None, ks, kr, None, vs, vr, D ** -0.5, out=out)
            ug = time_graph(fn, 1, max(1, 2 * args.steps))
            b = gemv_bytes(B, Hkv, Tq, D, G, 4, "asymmetric", "channel") + \
                gemv_bytes(B, Hkv, Tq, D, G, 4, "asymmetric", "token")
            res[f"decode_Hkv{Hkv}_T{T}_R{R}"] = dict(us_graph=ug, GBs_graph=b / ug / 1e3, bytes=b)
            del ks, vs
        for Hkv, T in ((8, 8192), (8, 131072), (1, 131072)):
            B, Hq, GV = 1, 4 * Hkv, 64
            vs = make_store("token", B, Hkv, T, D, GV, 2, "asymmetric", 72, dev)
            p = torch.softmax(torch.randn(B, Hq, T, device=dev) * 2.0, dim=-1).to(torch.float16)
            out = torch.empty(B, Hq, D, device=dev, dtype=torch.float16)
            fn = lambda i: ops.av_gemv(p, vs, out=out)
            ug = time_graph(fn, 1, max(1, 2 * args.steps))
            b = gemv_bytes(B, Hkv, T, D, GV, 2, "asymmetric", "token")
            res[f"av_Hkv{Hkv}_T{T}"] = dict(us_graph=ug, GBs_graph=b / ug / 1e3, bytes=b)
            del vs
    print(json.dumps(res), flush=True)


def calib_copy(args):
    """A plain device copy of known size, for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE."""
    import torch
    n = 256 << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calib_copy_bytes": n}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--copies", type=int, default=4)
    ap.add_argument("--config", default="H")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calib-copy", action="store_true")
    ap.add_argument("--gemvs", action="store_true", help="also time the standalone QK^T and attn.V GEMV API calls")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build runs on one GPU only (no collectives); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)
    if args.calib_copy:
        calib_copy(args)
    elif args.config == "H":
        bench_headline(args)
    else:
        bench_config(args)


if __name__ == "__main__":
    main()
