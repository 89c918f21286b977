"""Sparse-decode layer-step benchmark on one MI355X.

Workload: the 32K-history sparse decode of a Qwen3-4B-shaped attention stack
(32 query heads, 8 KV heads, head_dim 128), 36 independent layers with their
own seeded synthetic history (32768 tokens = 512 blocks each), Top-32 blocks
+ 64-token sink + 512-token recent window, r = 4 representatives per block.
A step is one decode token through all 36 layers: block scoring + Top-32 for
every layer (one launch pair), then in-place gather + segmented attention for
every layer (one launch), including the recent-window append.

Prints one JSON line: decode tokens/s over the 36 layers (value), us per
layer-step, achieved HBM GB/s on the algorithmic bytes of the step, the
roofline of the dominant kernel (attention) from HIP events, and the
reference algorithm timed on the host cores (cpu_baseline).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "nano-vllm-kv-optimizer_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = ("µs per sparse-decode layer-step @32K + achieved HBM GB/s; "
          "decode tokens/s (36L)")
PREFILL_METRIC = "TFLOP/s of the chunked-prefill sparse attention (causal-exact FLOPs)"
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


def step_bytes(nblocks, k, sink, recent, kv_format, hkv=8, d=128, r=4, hq=32, B=64):
    """Algorithmic HBM bytes of one decode layer-step (reps + selected + sink + recent + q/o)."""
    reps = nblocks * hkv * r * d * 2
    row = hkv * d
    if kv_format == "bf16":
        sel = k * B * row * 2 * 2
        scales = 0
    elif kv_format == "int8":
        sel = k * B * row * 2
        scales = hkv * d * 4 + k * hkv * 4
    else:
        sel = k * B * row * 2
        scales = k * B * hkv * 2 * 2
    win = (sink + recent) * row * 2 * 2
    qo = 2 * hq * d * 2
    return {"reps": reps, "selected": sel + scales, "window": win, "qo": qo,
            "total": reps + sel + scales + win + qo, "attend": sel + scales + win + qo}


class DeviceEvents:
    """HIP timing events recorded with a device-scope release.

    torch.cuda.Event records with a system-scope release, which on this
    runtime leaves the GPU idle for several microseconds per record; a
    per-step pair of them inflates the step time it brackets.  Events made
    with hipEventReleaseToDevice only order the device's own work, which is
    all a kernel timing needs.  The handles live in the same HIP runtime as
    torch's (one libamdhip64.so.7 per process).
    """

    _RELEASE_TO_DEVICE = 0x40000000

    def __init__(self, n):
        import ctypes
        import torch
        self._c = ctypes
        self._hip = ctypes.CDLL("libamdhip64.so.7")
        self._hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self._hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self._hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self._hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self._stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        self.ev = []
        for _ in range(n):
            e = ctypes.c_void_p()
            rc = self._hip.hipEventCreateWithFlags(ctypes.byref(e), self._RELEASE_TO_DEVICE)
            if rc != 0:
                raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")
            self.ev.append(e)

    def record(self, i):
        rc = self._hip.hipEventRecord(self.ev[i], self._stream)
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_ms(self, i, j):
        ms = self._c.c_float()
        rc = self._hip.hipEventElapsedTime(self._c.byref(ms), self.ev[i], self.ev[j])
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return ms.value

    def close(self):
        for e in self.ev:
            self._hip.hipEventDestroy(e)
        self.ev = []


def _cpu_model():
    """The host CPU as /proc/cpuinfo names it: the model-name string (lscpu's
    "Model name") with its family / model / stepping numbers, which identify
    the part when a virtualised host reports a generic name."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break
                key, _, val = line.partition(":")
                fields[key.strip()] = val.strip()
    except OSError:
        return None
    name = fields.get("model name")
    if name is None:
        return None
    ids = [f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields]
    vendor = fields.get("vendor_id")
    return f"{name} ({', '.join(([vendor] if vendor else []) + ids)})" if ids or vendor else name


def cpu_baseline(model, args, qs, ks, vs, seconds):
    """The reference's host-side op sequence timed on this box's cores (bounded sample)."""
    import torch

    from oracle.cpu_path import CpuLayer
    st = model.store
    nb = model.nblocks_filled
    n_sample = min(args.cpu_layers, args.layers)
    layers = []
    for i in range(n_sample):
        # reference layout: history [nb, 64, Hkv, D], sink/recent [S|R, Hkv, D]
        hk = st.hist_k[i, :, :nb].permute(1, 2, 0, 3).cpu()
        hv = st.hist_v[i, :, :nb].permute(1, 2, 0, 3).cpu()
        R = st.recent_tokens
        rs = model.core.ring_start
        order = [(rs + j) % R for j in range(R)]
        rk = st.recent_k[i][:, order].permute(1, 0, 2).cpu()
        rv = st.recent_v[i][:, order].permute(1, 0, 2).cpu()
        layers.append(CpuLayer(hk, hv, st.reps[i, :, :nb].cpu(), st.sink_k[i].permute(1, 0, 2).cpu(),
                               st.sink_v[i].permute(1, 0, 2).cpu(), rk, rv,
                               model.core.protected_blocks, top_k=args.top_k))
    qc, kc, vc = qs.cpu(), ks.cpu(), vs.cpu()
    times = []
    t_end = time.perf_counter() + seconds
    s = 0
    while time.perf_counter() < t_end or s < n_sample:
        li = s % n_sample
        step = (s // n_sample) % qc.shape[0]
        t0 = time.perf_counter()
        layers[li].decode(qc[step, li], kc[step, li], vc[step, li])
        times.append(time.perf_counter() - t0)
        s += 1
    times.sort()
    med_us = times[len(times) // 2] * 1e6
    # the reference's own CPU-gather anchor, on the ids this run selected
    from oracle.cpu_path import gather_anchor
    groups = [model.last_ids_dev[i, 0, :model.last_n_selected].to("cpu", torch.int64)
              for i in range(model.last_ids_dev.shape[0])]
    counts = sorted({1, 2, 4, 8, min(os.cpu_count() or 1, torch.get_num_threads())})
    anchor = gather_anchor(layers[0].flat_k, layers[0].flat_v, groups, threads=counts)
    mib = 2 * groups[0].numel() * 64 * layers[0].flat_k.shape[1] * layers[0].flat_k.shape[2] * 2 / 2 ** 20
    return {
        "value": round(1e6 / (args.layers * med_us), 3),
        "unit": "tokens/s",
        "us_per_layer_step": round(med_us, 1),
        "cores": torch.get_num_threads(),
        "torch_threads": torch.get_num_threads(),
        "host_cpus": os.cpu_count(),
        "cpus_in_affinity": len(os.sched_getaffinity(0)),
        "cpu_model": _cpu_model(),
        "kind": "port",
        "sample": (f"{len(times)} layer-steps of the 32K workload ({n_sample} distinct layers, "
                   f"~{seconds:.0f} s): torch-CPU einsum scorer + topk + index_select gather + "
                   f"pack + fp32 einsum attention, median per layer-step x {args.layers} layers"),
        "gather_anchor": {
            "what": (f"reference CPU gather microbenchmark form (benchmark_m20_gather.py:88-99): "
                     f"token-index index_select of {groups[0].numel()} selected blocks ({mib:.0f} MiB K+V) "
                     f"from a pageable bf16 [{layers[0].nblocks}, 64, 8, 128] history into pinned staging, "
                     f"cycling the {len(groups)} layers' ids of this run's last step; median us per gather"),
            "us_by_threads": {str(n): round(t, 1) for n, t in anchor.items()},
            "reference_us_by_threads": {"1": 871.77, "2": 632.35, "4": 378.28, "8": 315.31},
            "reference_source": "docs/m20_gather_results.md:107-112 (RTX 3080 Laptop host CPU)",
        },
    }


def prefill_flops(chunk, n_prior, hq=32, d=128):
    """Causal-exact FLOPs of one layer's chunk attention: 4 Hq D sum_t (n_prior + t + 1)."""
    return 4 * hq * d * (chunk * n_prior + chunk * (chunk + 1) // 2)


def bench_prefill(args, dev):
    """Chunked prefill: a 4096-token chunk of every layer against its 32K history.

    A step is query summaries + selection + matrix-core attention over
    [32 selected blocks | sink | recent | causal chunk] for all layers (the
    chunk's store is not part of the step, so every step sees the same state).
    """
    import torch

    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12ModelRuntime
    from nanokv_amd.store import query_summaries

    L, T0, T = args.layers, args.context, args.chunk
    quant = args.kv_format != "bf16"
    cfg = M12Config(max_model_len=T0 + T, top_k_blocks=args.top_k, quant_history=quant,
                    quant_scale_layout="token" if args.kv_format == "int8_token" else "channel_block",
                    prefill_selection=args.prefill_selection)
    model = M12ModelRuntime(L, cfg, device=dev)
    kh = torch.empty(L, T0, 8, 128, dtype=torch.bfloat16, device=dev)
    vh = torch.empty_like(kh)
    for i in range(L):
        k, v, _, _ = workload.history(T0, args.seed + i, device=dev)
        kh[i].copy_(k)
        vh[i].copy_(v)
    model.prefill(kh, vh)
    del kh, vh
    q, k, v = workload.prefill_chunk_inputs(T, args.seed, device=dev, layers=L)
    core = model.core

    tile = cfg.prefill_selection_tile

    def step(ev=None):
        if cfg.prefill_selection == "tile":
            ids, n = core.select_tiles(q, args.top_k, tile)
        else:
            qs = query_summaries(q, cfg.prefill_query_segments)
            ids, _, n = core.select(qs, args.top_k)
        if ev is not None:
            ev[0].record()
        if cfg.prefill_selection == "tile":
            out, _, _ = core.chunk_attend_tiled(q, k, v, ids, tile, n)
        else:
            out, _, _ = core.chunk_attend(q, k, v, ids, ids.shape[-1], n)
        if ev is not None:
            ev[1].record()
        return out

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(args.steps):
        step(evs[i])
    stop.record()
    torch.cuda.synchronize()
    ms_step = start.elapsed_time(stop) / args.steps
    attn_ms = sum(a.elapsed_time(b) for a, b in evs) / args.steps
    n_prior = args.top_k * 64 + cfg.sink_tokens + cfg.recent_tokens
    flops = prefill_flops(T, n_prior) * L
    tflops = flops / (ms_step * 1e-3) / 1e12
    attn_tflops = flops / (attn_ms * 1e-3) / 1e12
    return {
        "metric": PREFILL_METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)/sqrt(128) K/V history and chunk K/V, N(0,1) chunk queries)",
        "config": {
            "workload": (f"chunked prefill, {T}-token chunk vs {T0}-token history x {L} layers, "
                         f"Qwen3-4B attention shape (Hq=32, Hkv=8, D=128), top-{args.top_k} + sink "
                         f"{cfg.sink_tokens} + recent {cfg.recent_tokens} + causal chunk, "
                         f"{args.kv_format} history, selection per "
                         + ("chunk" if cfg.prefill_selection == "chunk" else f"{tile}-query tile")),
            "layers": L, "context": T0, "chunk": T, "top_k": args.top_k, "kv_format": args.kv_format,
            "prefill_selection": cfg.prefill_selection,
        },
        "tokens_per_s": round(T * 1e3 / ms_step, 1),
        "flops_per_step": flops,
        "roofline": {
            "bound": "mfma",
            "kernel": "prefill_kernel (segmented causal attention, bf16 MFMA, all layers)",
            "achieved": round(attn_tflops, 2),
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(attn_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "traffic": None,
            "avg_launch_us": round(attn_ms * 1e3, 2),
        },
    }


MODEL_METRIC = "Qwen3-4B decode tokens/s (1 / TPOT) at 32K context, sparse attention, whole model"


def bench_model(args, dev):
    """End-to-end decode of a Qwen3-4B-architecture decoder (36 layers, hidden
    2560, MLP 9728, vocab 151936, tied head; random N(0, 0.02) weights, since
    no checkpoint is reachable offline) after a prompt of --context tokens
    prefilled in --chunk-token chunks (first chunk dense within itself, later
    chunks through the sparse chunked prefill).  A step is one greedy decode
    token through the whole model: embedding, per layer RMSNorm + q/k/v
    projection + q/k RMSNorm + RoPE + the sparse decode layer-step + output
    projection + RMSNorm + SiLU MLP, final norm, LM head, argmax.  The layers
    run one after the other, so each layer-step is its own select + attend
    launches (not the batched 36-layer launches of the decode line)."""
    import torch

    from nanokv_amd.qwen3 import Qwen3Config, Qwen3ForCausalLM, init_random_
    from nanokv_amd.sparse import M12Config

    T = args.context
    cfg = Qwen3Config(num_hidden_layers=args.layers)
    quant = args.kv_format != "bf16"
    m12 = M12Config(max_model_len=T, top_k_blocks=args.top_k, quant_history=quant,
                    quant_scale_layout="token" if args.kv_format == "int8_token" else "channel_block")
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            model = Qwen3ForCausalLM(cfg, T + 2 * args.warmup + 2 * args.steps + 16)
    finally:
        torch.set_default_dtype(prev)
    init_random_(model, args.seed)
    model.attach(m12, dev)
    prompt = torch.randint(0, cfg.vocab_size, (T,), device=dev,
                           generator=torch.Generator(device=dev).manual_seed(args.seed))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits = model.prefill(prompt, chunk=args.chunk)
    torch.cuda.synchronize()
    prefill_ms = (time.perf_counter() - t0) * 1e3
    pos = T
    tok = logits.argmax().view(1)

    def run(fn, n):
        """n greedy decode steps through fn; returns (ms per token, host enqueue ms per token)."""
        nonlocal tok, pos
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record()
        for _ in range(n):
            tok = fn(tok, pos).argmax().view(1)
            pos += 1
        stop.record()
        host = (time.perf_counter() - t0) * 1e3 / n
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / n, host

    # eager steps (every op launched from Python), then the captured token step
    run(model.decode, max(2, args.warmup // 4))
    eager_ms, eager_host = run(model.decode, max(4, args.steps // 4))
    run(model.decode_graph, args.warmup + 2)   # eager device-ring step, capture, replays
    tpot, host_ms = run(model.decode_graph, args.steps)
    params = sum(p.numel() for p in model.parameters())
    return {
        "metric": MODEL_METRIC,
        "value": round(1e3 / tpot, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(tpot, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random N(0, 0.02) weights, seeded random prompt tokens, greedy decode)",
        "config": {
            "workload": (f"Qwen3-4B architecture ({args.layers} layers, {params / 1e9:.2f} B parameters), "
                         f"{T}-token prompt prefilled in {args.chunk}-token chunks, then greedy decode; "
                         f"sparse attention top-{args.top_k} + sink {m12.sink_tokens} + recent "
                         f"{m12.recent_tokens}, {args.kv_format} history"),
            "layers": args.layers, "context": T, "chunk": args.chunk, "top_k": args.top_k,
            "kv_format": args.kv_format,
        },
        "tpot_ms": round(tpot, 4),
        "host_enqueue_ms_per_token": round(host_ms, 4),
        "decode_mode": "HIP graph of the whole token step (decode_graph), replayed per token",
        "eager_tpot_ms": round(eager_ms, 4),
        "eager_host_enqueue_ms_per_token": round(eager_host, 4),
        "prefill_ms": round(prefill_ms, 1),
        "reference_published": {"tpot_ms": 141.84, "prefill_32k_ms": 12718,
                                "hardware": "RTX 3080 Laptop, host-offloaded history"},
    }


def verify_bytes(u_mean, nblocks, tq, kv_format, hkv=8, d=128, r=4, hq=32, B=64, sink=64, recent=512):
    """Algorithmic bytes of one lossless verify layer-step: reps + the union's
    blocks (K+V) + sink + recent + the chunk's K/V + q and o."""
    elem = 1 if kv_format != "bf16" else 2
    reps = nblocks * hkv * r * d * 2
    union = u_mean * hkv * B * d * 2 * elem
    scales = 0 if kv_format == "bf16" else (u_mean * hkv * 4 if kv_format == "int8" else u_mean * hkv * B * 2 * 2)
    ring = (sink + recent) * hkv * d * 2 * 2
    chunk = tq * hkv * d * 2 * 2
    qo = tq * hq * d * 2 * 2
    return reps + union + scales + ring + chunk + qo


def bench_verify(args, dev):
    """Speculative verify: Tq = 6 draft + target tokens of every layer against its history.

    A round is one lossless verification pass for all layers (M12ModelRuntime.verify:
    per-query Top-K, device-side union + per-query mask, causal attention over
    [union | sink | recent | the Tq tokens]) followed by a rollback, so every
    round sees the same state.
    """
    import torch

    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12ModelRuntime

    L, T0, tq = args.layers, args.context, args.verify_tokens
    quant = args.kv_format != "bf16"
    extra = {} if args.mfma_chunk_min is None else {"mfma_chunk_min_tokens": args.mfma_chunk_min}
    if args.splits is not None:
        extra["attend_splits"] = args.splits
    cfg = M12Config(max_model_len=T0 + 64, top_k_blocks=args.top_k, quant_history=quant,
                    quant_scale_layout="token" if args.kv_format == "int8_token" else "channel_block",
                    **extra)
    model = M12ModelRuntime(L, cfg, device=dev)
    kh = torch.empty(L, T0, 8, 128, dtype=torch.bfloat16, device=dev)
    vh = torch.empty_like(kh)
    for i in range(L):
        k, v, _, _ = workload.history(T0, args.seed + i, device=dev)
        kh[i].copy_(k)
        vh[i].copy_(v)
    model.prefill(kh, vh)
    del kh, vh
    g = torch.Generator(device=dev).manual_seed(args.seed + 31)
    nrounds = args.warmup + args.steps
    qs = torch.randn(nrounds, L, tq, 32, 128, generator=g, device=dev).to(torch.bfloat16)
    ks = (torch.randn(nrounds, L, tq, 8, 128, generator=g, device=dev) * 128 ** -0.5).to(torch.bfloat16)
    vs = (torch.randn(nrounds, L, tq, 8, 128, generator=g, device=dev) * 128 ** -0.5).to(torch.bfloat16)
    for i in range(args.warmup):
        model.verify(qs[i], ks[i], vs[i], lossless=True)
        model.rollback_verified()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(args.steps):
        model.verify(qs[args.warmup + i], ks[args.warmup + i], vs[args.warmup + i], lossless=True)
        model.rollback_verified()
    stop.record()
    torch.cuda.synchronize()
    ms_round = start.elapsed_time(stop) / args.steps
    u_mean = float(model.last_union_count_dev.float().mean())  # the last round's unions
    by = verify_bytes(u_mean, model.nblocks_filled, tq, args.kv_format) * L

    # region B: the same rounds again with events the library records right
    # before and right after the attention kernel (nkv_set_attend_marks) ->
    # the kernel's average launch duration for the roofline
    from nanokv_amd import _lib
    ev = DeviceEvents(2 * args.steps)
    try:
        for i in range(args.steps):
            _lib.set_attend_marks(ev.ev[2 * i].value, ev.ev[2 * i + 1].value)
            model.verify(qs[args.warmup + i], ks[args.warmup + i], vs[args.warmup + i], lossless=True)
            model.rollback_verified()
    finally:
        _lib.set_attend_marks(None, None)
    torch.cuda.synchronize()
    attend_us = sum(ev.elapsed_ms(2 * i, 2 * i + 1) for i in range(args.steps)) / args.steps * 1e3
    ev.close()
    reps_b = model.nblocks_filled * 8 * 4 * 128 * 2   # read by the scorer, not the attention
    by_att = (verify_bytes(u_mean, model.nblocks_filled, tq, args.kv_format) - reps_b) * L
    att_gbps = by_att / (attend_us * 1e-6) / 1e9
    return {
        "metric": "µs per lossless speculative-verify round (all layers)",
        "value": round(ms_round * 1e3, 2),
        "unit": "µs",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_round, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if args.kv_format == "bf16" else "int8",
        "data": "synthetic (seeded N(0,1)/sqrt(128) K/V history and draft K/V, N(0,1) queries)",
        "config": {
            "workload": (f"lossless speculative verify, {tq} tokens vs {T0}-token history x {L} layers, "
                         f"per-query top-{args.top_k}, union + per-query mask, sink {cfg.sink_tokens} + "
                         f"recent {cfg.recent_tokens}, {args.kv_format} history"),
            "layers": L, "context": T0, "verify_tokens": tq, "top_k": args.top_k,
            "kv_format": args.kv_format,
        },
        "us_per_layer_round": round(ms_round * 1e3 / L, 4),
        "union_blocks_mean": round(u_mean, 1),
        "hbm_gbps": round(by / (ms_round * 1e-3) / 1e9, 1),
        "step_roofline_frac": round(by / (ms_round * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
        "roofline": {
            "bound": "hbm",
            "kernel": "attend_wide_kernel (union blocks + sink + recent + draft tokens, all layers)",
            "achieved": round(att_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(att_gbps / HBM_PEAK_GBPS, 4),
            "traffic": None,
            "bytes_per_launch": int(by_att),
            "avg_launch_us": round(attend_us, 2),
        },
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--context", type=int, default=32768)
    ap.add_argument("--top-k", type=int, default=32)
    ap.add_argument("--kv-format", choices=["bf16", "int8", "int8_token"], default="bf16")
    ap.add_argument("--splits", type=int, default=None)
    ap.add_argument("--history", choices=["hbm", "host"], default="hbm",
                    help="decode: history in HBM (default) or in pinned host memory read in place")
    ap.add_argument("--seed", type=int, default=2024)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--cpu-layers", type=int, default=8)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--layer-streams", type=int, default=1,
                    help="streams the decode step's layer ranges are spread over")
    ap.add_argument("--step-events", choices=["device", "torch"], default="device",
                    help="timing events: device-scope release (default) or torch.cuda.Event")
    ap.add_argument("--verify-tokens", type=int, default=6, help="verify: queries per round")
    ap.add_argument("--mfma-chunk-min", type=int, default=None,
                    help="verify: M12Config.mfma_chunk_min_tokens (chunks this long use the MFMA kernel)")
    ap.add_argument("--workload", choices=["decode", "prefill", "verify", "model"], default="decode",
                    help="decode (the headline line), the chunked-prefill attention, "
                         "lossless speculative verify (use --context 16384), or whole-model "
                         "Qwen3-4B decode (tokens/s = 1 / TPOT)")
    ap.add_argument("--chunk", type=int, default=4096, help="prefill chunk length")
    ap.add_argument("--prefill-selection", choices=["chunk", "tile"], default="chunk",
                    help="prefill: one selection per chunk (the reference's routing) or per 64-query tile")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (counter calibration)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: measures one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); the sparse layer-step is not run across GPUs here.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from nanokv_amd import workload
    from nanokv_amd.sparse import M12Config, M12ModelRuntime

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_probe_mib:
        n = args.copy_probe_mib << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(8):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n, "launches": 8}), flush=True)
        return
    if args.workload == "prefill":
        print(json.dumps(bench_prefill(args, dev)), flush=True)
        return
    if args.workload == "verify":
        print(json.dumps(bench_verify(args, dev)), flush=True)
        return
    if args.workload == "model":
        print(json.dumps(bench_model(args, dev)), flush=True)
        return
    L, T = args.layers, args.context
    quant = args.kv_format != "bf16"
    cfg = M12Config(max_model_len=T, top_k_blocks=args.top_k, quant_history=quant,
                    quant_scale_layout="token" if args.kv_format == "int8_token" else "channel_block",
                    attend_splits=args.splits, history_tier=args.history)
    model = M12ModelRuntime(L, cfg, device=dev, layer_streams=args.layer_streams)

    t0 = time.perf_counter()
    kh = torch.empty(L, T, 8, 128, dtype=torch.bfloat16, device=dev)
    vh = torch.empty_like(kh)
    for i in range(L):
        k, v, _, _ = workload.history(T, args.seed + i, device=dev)
        kh[i].copy_(k)
        vh[i].copy_(v)
    model.prefill(kh, vh)
    del kh, vh
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t0

    nsteps = args.warmup + 2 * args.steps
    qs, ks, vs = workload.decode_inputs(nsteps, args.seed, device=dev, layers=L)

    for s in range(args.warmup):
        model.decode(qs[s], ks[s], vs[s])
    torch.cuda.synchronize()

    # Two timed regions over the same workload.  A: K steps bracketed by one
    # event pair -> the step time and `value` (model.decode: the layers split
    # over --layer-streams streams).  B: K more steps, all layers on one
    # stream, with events the library records right before and right after
    # each step's attention kernel (nkv_set_attend_marks) and one after the
    # split merge -> the attention kernel's average launch duration for the
    # roofline, and the merge's.  A record leaves the GPU idle briefly, so
    # these durations include part of that idle time (conservative).
    K = args.steps
    if args.step_events == "torch":
        tev = [torch.cuda.Event(enable_timing=True) for _ in range(3 * K + 2)]
        for e in tev:
            e.record()   # the HIP event exists from its first record on
        rec = lambda i: tev[i].record()
        elapsed = lambda i, j: tev[i].elapsed_time(tev[j])
        handle = lambda i: tev[i].cuda_event
    else:
        dev_ev = DeviceEvents(3 * K + 2)
        rec = dev_ev.record
        elapsed = dev_ev.elapsed_ms
        handle = lambda i: dev_ev.ev[i].value
    torch.cuda.synchronize()
    host_t0 = time.perf_counter()
    rec(3 * K)
    for i in range(K):
        s = args.warmup + i
        model.decode(qs[s], ks[s], vs[s])
    rec(3 * K + 1)
    host_us = (time.perf_counter() - host_t0) / K * 1e6  # launch-side time per step
    torch.cuda.synchronize()
    ms_step = elapsed(3 * K, 3 * K + 1) / K

    from nanokv_amd import _lib
    splits = model.core._splits(args.top_k + 9, 1) if args.splits is None else args.splits
    try:
        for i in range(K):
            s = args.warmup + K + i
            ids, _, n = model.select(qs[s])
            _lib.set_attend_marks(handle(3 * i), handle(3 * i + 1))
            model.core.decode_attend(qs[s], ks[s], vs[s], ids, ids.shape[-1], n)
            rec(3 * i + 2)
    finally:
        _lib.set_attend_marks(None, None)
    torch.cuda.synchronize()
    attend_us = sum(elapsed(3 * i, 3 * i + 1) for i in range(K)) / K * 1e3
    merge_us = sum(elapsed(3 * i + 1, 3 * i + 2) for i in range(K)) / K * 1e3 if splits != 1 else 0.0
    if args.step_events != "torch":
        dev_ev.close()

    nb = model.nblocks_filled
    by = step_bytes(nb, args.top_k, cfg.sink_tokens, cfg.recent_tokens, args.kv_format)
    traffic = None
    prof = os.path.join(ROOT, "profiles", "decode32k_bf16_traffic.json")
    if (args.kv_format, L, T, args.top_k) == ("bf16", 36, 32768, 32) and os.path.exists(prof):
        with open(prof) as f:
            traffic = json.load(f)["traffic_bytes_per_launch"]["attend_kernel<0, 4, false, true>"]
    us_layer = ms_step * 1e3 / L
    step_gbps = by["total"] * L / (ms_step * 1e-3) / 1e9
    attend_gbps = by["attend"] * L / (attend_us * 1e-6) / 1e9
    result = {
        "metric": METRIC,
        "value": round(1000.0 / ms_step, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if args.kv_format == "bf16" else "int8",
        "data": "synthetic (seeded N(0,1)/sqrt(128) K/V, N(0,1) q, 3 planted blocks per layer)",
        "config": {
            "workload": (f"sparse decode layer-step, {T}-token history ({nb} blocks) x {L} "
                         f"independent layers, Qwen3-4B attention shape (Hq=32, Hkv=8, D=128), "
                         f"top-{args.top_k} + sink {cfg.sink_tokens} + recent {cfg.recent_tokens}, "
                         f"r=4, {args.kv_format} history"
                         + (" in pinned host memory, read in place over the host link"
                            if args.history == "host" else "")),
            "layers": L, "context": T, "top_k": args.top_k, "kv_format": args.kv_format,
            "layer_streams": args.layer_streams, "history_tier": args.history,
        },
        "us_per_layer_step": round(us_layer, 4),
        "hbm_gbps": round(step_gbps, 1),
        "bytes_per_layer_step": by["total"],
        "attend_splits": splits,
        "roofline": {
            "bound": "hbm",
            "kernel": "attend_kernel (in-place gather + segmented attention, all layers; one launch per step)",
            "achieved": round(attend_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(attend_gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": ("profiles/decode32k_bf16_traffic.json (calibrated FETCH_SIZE+WRITE_SIZE "
                               "of attend_kernel)") if traffic else None,
            "bytes_per_launch": by["attend"] * L,
            "avg_launch_us": round(attend_us, 2),
            "merge_us": round(merge_us, 2),
            "op_frac": round(by["attend"] * L / ((attend_us + merge_us) * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
        },
        "step_roofline_frac": round(step_gbps / HBM_PEAK_GBPS, 4),
        "host_launch_us_per_step": round(host_us, 1),
        "setup_s": round(setup_s, 1),
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(model, args, qs, ks, vs, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
