"""Benchmark of SemBlend's KV-reuse path on one MI355X at the Qwen2.5-7B shape.

One step is one pass of the path over synthetic inputs resident in HBM:

  rope       RoPE delta correction of donor K in place: K [28, 4, 8192, 128] bf16, theta 1e6,
             delta constant per 256-token chunk, uniform in [-2048, 2048]
             (rope_correct_k semantics; four rotating copies so the 256 MB Infinity Cache
             cannot hold the 235 MB tensor between visits);
  scatter    donor-KV scatter into paged caches for 28 layers in one launch: per layer cache
             [2048, 2, 4, 16, 128] bf16, donor [2, 4, 16384, 128]; 64 donor 256-token chunks
             reused in shuffled order, minus 2458 recomputed positions -> 13926 pairs;
  attention  GQA partial-prefill attention, 28 q heads / 4 KV heads, head_dim 128, bf16, over a
             16384-token paged context; 2458 recompute rows (first 256 tokens, two random
             256-token chunks, the rest scattered).

The reported ``value`` is the attention phase's throughput in TFLOP/s (useful causal FLOPs
4 * D * Hq * sum(p + 1)); the scatter and RoPE phases are reported in GB/s of useful bytes
(each moved row read once and written once). The timed steps are K whole steps, each one HIP
graph replay (RoPE, scatter and attention launches back to back inside it, as a serving loop
would launch them), enqueued back to back between one pair of HIP events: ``ms_per_step``.
Phase durations come from the eager pass that precedes the graphs, in which the library
brackets each of its kernel launches with HIP events that the runtime stamps with the
kernel's own start and end (``kernels``); a phase is its kernels (attention: the MFMA kernel
and the split-key merge). ``launch_inclusive_ms`` times each phase as its own graph with
events around every replay, which adds one graph launch (about 8 us on this GPU) per phase.
The RoPE and scatter phases stream 2 GB through the 256 MB Infinity Cache before every
attention launch, so no timed kernel finds its inputs cached from the previous step.
``roofline`` prices the MFMA attention kernel's average launch against the bf16 peak.
``phases.copy_ceiling`` is a plain 1 GiB device copy through the library's flat copy kernel,
the achievable HBM rate; every HBM phase also reports ``frac_of_copy`` against it.
``rope_scatter`` times the scatter workload again with K rotated on the way (one donor, and
a composite from four donors); ``chunk_load`` streams the same donor from pinned host memory
in 256-token chunks with the RoPE scatter overlapped. The CPU
baseline times the oracle (a restatement of the reference's CPU path, with its per-pair
loops) on the whole workload on the host's cores.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu-baseline] [--no-llama-batch]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np
import torch

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2516.6   # MI355X dense bf16 MFMA, TFLOP/s

L, HKV, HQ, D, BS = 28, 4, 28, 128, 16
CTX, N_RECOMPUTE, CHUNK = 16384, 2458, 256
ROPE_TOKENS, ROPE_BASE = 8192, 1e6
POOL_BLOCKS = 2048

# Library kernels whose launches are timed with HIP events over the timed region.
KERNELS = ("attn_mfma", "attn_merge", "move_rows", "rope_rows", "rope_index", "fill_i32")
# (the projection section times its own kernel, qkv_mfma)

# HBM bytes per launch on this workload, from rocprofv3 FETCH_SIZE and WRITE_SIZE passes over
# this script, scaled by what the same counters read for the 1 GiB copy of copy_ceiling()
# (FETCH_SIZE x 2.0, WRITE_SIZE x 1.0); kernel changes call for a new measurement. Attention:
# the planned launch that the step times.
MEASURED_TRAFFIC_BYTES = {
    "attn_mfma": (2 * 92677 + 63581) * 1024,
    "move_rows": (2 * 391155 + 779861) * 1024,
    "rope_rows": (2 * 114793 + 229376) * 1024,
}
MEASURED_TRAFFIC_SOURCE = ("rocprofv3 FETCH_SIZE / WRITE_SIZE passes at commit 0817005, "
                           "profiles/kv_reuse_7b_16k_hbm_traffic.md")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def recompute_positions(g: torch.Generator, ctx: int = CTX,
                        n_recompute: int = N_RECOMPUTE) -> torch.Tensor:
    """First 256 tokens + two random whole chunks + uniform scatter, n_recompute in total
    (chunks only while they fit the budget)."""
    n_chunks = ctx // CHUNK
    mask = torch.zeros(ctx, dtype=torch.bool)
    mask[:min(CHUNK, n_recompute)] = True
    for c in (torch.randperm(n_chunks - 1, generator=g)[:2] + 1).tolist():
        if int(mask.sum()) + CHUNK <= n_recompute:
            mask[c * CHUNK:(c + 1) * CHUNK] = True
    rest = (~mask).nonzero().flatten()
    mask[rest[torch.randperm(rest.numel(), generator=g)[:n_recompute - int(mask.sum())]]] = True
    return mask.nonzero().flatten().to(torch.int32)


# Qwen2.5-0.5B one-layer pipeline (the reference's CPU-runnable case).
QWEN05B = {"hq": 14, "hkv": 2, "d": 64, "theta": 1e6, "ctx": 1024, "pool_blocks": 128,
           "max_delta": 64, "rows": 154}


def qwen05b_pipeline_inputs(seed: int = 0) -> dict:
    """Inputs of the one-layer KV-reuse pipeline at the Qwen2.5-0.5B shape (14 q heads, 2 KV
    heads, head_dim 64, fp32, theta 1e6, 1024 tokens), drawn in this order from one CPU
    generator: donor K/V [2, 2, 1024, 64] ~ N(0, 1); a block table of 64 entries from a random
    permutation of the 128-block pool; one RoPE delta per token, uniform over the integers in
    [-64, 64]; 154 recompute positions (15%) drawn uniformly without replacement (sorted);
    their queries [154, 14, 64] ~ N(0, 1). The cache [128, 2, 2, 16, 64] starts zeroed and
    donor row t goes to position t. CPU tensors."""
    c = QWEN05B
    g = torch.Generator("cpu").manual_seed(seed)
    donor = torch.randn((2, c["hkv"], c["ctx"], c["d"]), generator=g)
    bt = torch.randperm(c["pool_blocks"], generator=g)[:c["ctx"] // BS].to(torch.int32)
    deltas = torch.randint(-c["max_delta"], c["max_delta"] + 1, (c["ctx"],), generator=g)
    rows = torch.randperm(c["ctx"], generator=g)[:c["rows"]].sort().values.to(torch.int32)
    q = torch.randn((c["rows"], c["hq"], c["d"]), generator=g)
    return {"donor": donor, "block_table": bt, "deltas": deltas, "rows": rows, "q": q,
            "cache": torch.zeros((c["pool_blocks"], 2, c["hkv"], BS, c["d"])),
            "positions": torch.arange(c["ctx"], dtype=torch.int32)}


def delta_groups(deltas: torch.Tensor) -> list[tuple[int, list[int]]]:
    """(delta, positions) for every distinct nonzero per-token delta, in ascending delta
    order: one in-place RoPE call per group."""
    d = deltas.numpy()
    order = np.argsort(d, kind="stable")  # positions stay ascending within a group
    sd = d[order]
    bounds = (np.flatnonzero(np.diff(sd)) + 1).tolist()
    pos, val = order.tolist(), sd.tolist()
    return [(int(val[s]), pos[s:e]) for s, e in zip([0] + bounds, bounds + [len(pos)])
            if val[s] != 0]


def qwen05b_pipeline(mod_tk, mod_rc, inp: dict, device=None, one_call: bool = False):
    """The pipeline through the drop-in entry points (``mod_tk`` / ``mod_rc`` are the
    triton_kernels / rope_correction modules, or the oracle for both): scatter the donor into
    the paged cache, rotate every token's K in place by its delta (one
    ``apply_rope_delta_inplace`` call per distinct delta, or with ``one_call`` a single
    ``apply_rope_deltas_inplace_layers`` call with the per-token deltas), then causal GQA
    attention of the recompute rows over that cache. Returns (cache, attention output)."""
    c = QWEN05B
    to = (lambda t: t.to(device)) if device is not None else (lambda t: t.clone())
    kv = to(inp["cache"])
    bt = to(inp["block_table"])
    pos = to(inp["positions"])
    mod_tk.scatter_donor_kv_paged(kv, to(inp["donor"]), bt, pos, pos)
    if one_call:
        mod_rc.apply_rope_deltas_inplace_layers([kv], bt, inp["positions"], inp["deltas"],
                                                rope_base=c["theta"])
    else:
        for dl, where in delta_groups(inp["deltas"]):
            mod_rc.apply_rope_delta_inplace(kv, bt, where, dl, rope_base=c["theta"])
    if device is not None:
        out = mod_tk.partial_prefill_attention_paged(to(inp["q"]), kv, bt, to(inp["rows"]))
    else:
        out = mod_tk.partial_attention_paged(inp["q"], kv, bt, inp["rows"])
    return kv, out


# Llama-3-8B batch (four requests sharing one paged pool, all layers).
LLAMA = {"layers": 32, "hq": 32, "hkv": 8, "d": 128, "theta": 5e5,
         "ctx": (8192, 16384, 24576, 32768), "frac": (0.10, 0.15, 0.20, 0.30),
         "pool_blocks": 8192, "delta": 4096}


def llama_batch(dev: torch.device, layers: int = LLAMA["layers"], ctx=LLAMA["ctx"],
                frac=LLAMA["frac"], pool_blocks: int = LLAMA["pool_blocks"],
                max_delta: int = LLAMA["delta"], seed: int = 4):
    """Synthetic Llama-3-8B KV-reuse batch: per-layer caches [pool, 2, 8, 16, 128] bf16 filled
    with N(0, 1) (the recompute rows' fresh K/V), per-request donor buffers [2, 8, ctx, 128],
    reuse pairs t -> d = t - delta with delta constant per 256-token chunk (uniform in
    [-max_delta, max_delta], redrawn until the chunk's donor rows lie in the donor buffer),
    recompute sets built like the 7B workload, and block tables drawn from one random
    permutation of the pool. Returns (caches, requests, theta)."""
    from semblend_amd.batch import ReuseRequest

    g = torch.Generator("cpu").manual_seed(seed)
    gd = torch.Generator(dev).manual_seed(seed)
    hkv, d = LLAMA["hkv"], LLAMA["d"]
    caches = [torch.randn((pool_blocks, 2, hkv, BS, d), generator=gd, device=dev,
                          dtype=torch.bfloat16) for _ in range(layers)]
    perm = torch.randperm(pool_blocks, generator=g)
    requests, at = [], 0
    for c, f in zip(ctx, frac):
        nblk = (c + BS - 1) // BS
        if at + nblk > pool_blocks:
            raise ValueError("pool too small for the batch")
        bt = perm[at:at + nblk].to(torch.int32)
        at += nblk
        pos_r = recompute_positions(g, c, int(round(c * f)))
        keep = torch.ones(c, dtype=torch.bool)
        keep[pos_r.long()] = False
        t = torch.arange(c)[keep]
        delta = torch.empty(c // CHUNK + 1, dtype=torch.int64)
        for k in range(delta.numel()):
            lo, hi = max(-max_delta, k * CHUNK + CHUNK - c), min(max_delta, k * CHUNK)
            delta[k] = torch.randint(lo, hi + 1, (1,), generator=g)
        dpos = t - delta[t // CHUNK]
        donors = [torch.randn((2, hkv, c, d), generator=gd, device=dev, dtype=torch.bfloat16)
                  for _ in range(layers)]
        requests.append(ReuseRequest(block_table=bt.to(dev), donor_kvs=donors,
                                     donor_positions=dpos.to(torch.int32).to(dev),
                                     target_positions=t.to(torch.int32).to(dev),
                                     compute_positions=pos_r.to(dev)))
    return caches, requests, LLAMA["theta"]


def build_inputs(dev: torch.device):
    g = torch.Generator("cpu").manual_seed(0)
    gd = torch.Generator(dev).manual_seed(0)
    inp = {}
    # rope: four rotating copies of K
    inp["rope_k"] = [torch.randn((L, HKV, ROPE_TOKENS, D), generator=gd, device=dev,
                                 dtype=torch.bfloat16) for _ in range(4)]
    deltas = torch.randint(-2048, 2049, (ROPE_TOKENS // CHUNK,), generator=g)
    d = torch.arange(ROPE_TOKENS)
    inp["rope_d"] = d.to(torch.int32).to(dev)
    inp["rope_t"] = (d + deltas[d // CHUNK]).to(torch.int32).to(dev)
    # scatter: 28 layers
    pos_r = recompute_positions(g)
    perm = torch.randperm(CTX // CHUNK, generator=g)
    t = torch.arange(CTX)
    dpos = perm[t // CHUNK] * CHUNK + t % CHUNK
    keep = torch.ones(CTX, dtype=torch.bool)
    keep[pos_r.long()] = False
    inp["sc_d"] = dpos[keep].to(torch.int32).to(dev)
    inp["sc_t"] = t[keep].to(torch.int32).to(dev)
    inp["block_table"] = torch.randperm(POOL_BLOCKS, generator=g)[:CTX // BS].to(torch.int32).to(dev)
    inp["caches"] = [torch.zeros((POOL_BLOCKS, 2, HKV, BS, D), dtype=torch.bfloat16, device=dev)
                     for _ in range(L)]
    inp["donors"] = [torch.randn((2, HKV, CTX, D), generator=gd, device=dev, dtype=torch.bfloat16)
                     for _ in range(L)]
    # attention over the first layer's cache, fully populated
    kv = inp["caches"][0]
    kv.normal_(generator=gd)
    inp["attn_kv"] = kv
    inp["attn_pos"] = pos_r.to(dev)
    inp["attn_q"] = torch.randn((pos_r.shape[0], HQ, D), generator=gd, device=dev,
                                dtype=torch.bfloat16)
    inp["pos_cpu"] = pos_r
    return inp


def copy_ceiling(dev: torch.device, nbytes: int = 1 << 30, reps: int = 10) -> dict:
    """Achievable HBM bandwidth of a plain 1 GiB device copy (read + write), GB/s: the
    library's flat copy (one 16-byte vector per thread, nontemporal; the ceiling the movers'
    ``frac_of_copy`` refers to) and torch's ``copy_`` beside it."""
    from semblend_amd import _lib

    a = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    out = {}
    for name, fn in (("library", lambda: _lib.device_copy(b, a)), ("torch", lambda: b.copy_(a))):
        fn()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[name] = 2.0 * nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del a, b
    return out


def gemm_ceiling(dev: torch.device, n: int = 8192, reps: int = 10) -> float:
    """Achievable dense bf16 matrix-core rate of a large square library GEMM (torch matmul,
    hipBLASLt), TFLOP/s: the practical ceiling next to the 2516.6 TFLOP/s spec figure."""
    g = torch.Generator(dev).manual_seed(9)
    a = torch.randn((n, n), generator=g, device=dev, dtype=torch.bfloat16)
    b = torch.randn((n, n), generator=g, device=dev, dtype=torch.bfloat16)
    c = torch.matmul(a, b)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        torch.matmul(a, b, out=c)
    e1.record()
    torch.cuda.synchronize()
    tflops = 2.0 * n ** 3 * reps / (e0.elapsed_time(e1) * 1e-3) / 1e12
    del a, b, c
    return tflops


def cpu_model() -> dict:
    """Host CPU description: lscpu's model name, family/model/stepping, sockets and threads
    per core (what /proc/cpuinfo says when lscpu is absent)."""
    info = {}
    try:
        import subprocess

        res = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10)
        for line in res.stdout.splitlines():
            key, _, val = line.partition(":")
            key = key.strip()
            if key in ("Model name", "Vendor ID", "CPU family", "Model", "Stepping",
                       "Socket(s)", "Thread(s) per core", "Core(s) per socket", "CPU(s)",
                       "CPU max MHz"):
                info[key] = val.strip()
    except (OSError, ValueError):
        pass
    # /proc/cpuinfo's own string too: a virtual machine may report a shortened model name
    # to lscpu, and the family / model numbers above then identify the part.
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    info["cpuinfo model name"] = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    info.setdefault("Model name", info.get("cpuinfo model name", "unknown"))
    return info


def median_time(fn, reps: int = 3) -> float:
    """Median wall time of ``reps`` calls of fn (time.perf_counter), seconds."""
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def cpu_baseline(inp) -> dict:
    """Oracle (reference CPU path restated) on the whole workload, on the host's cores;
    each leg's time is the median of three runs."""
    from oracle import ref_cpu as ref

    torch.set_num_threads(max(1, os.cpu_count() or 1))
    cores = torch.get_num_threads()
    kv = inp["attn_kv"].cpu()
    bt = inp["block_table"].cpu()
    pos = inp["pos_cpu"]
    q = inp["attn_q"].cpu()
    flops = 4.0 * D * HQ * float((pos.double() + 1).sum())
    dt = median_time(lambda: ref.partial_attention_paged(q, kv, bt, pos))
    out = {
        "value": flops / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "host": {"cpu_count": os.cpu_count(), "torch_threads": cores, "cpu": cpu_model()},
        "timing": "median of 3 (time.perf_counter)",
        "sample": f"whole workload: partial attention, all {pos.shape[0]} recompute rows, "
                  f"28q/4kv x 128, 16384-token paged context, bf16 in / fp32 math {dt:.2f} s",
    }
    # scatter (all pairs, all layers) and RoPE (the whole K) reported alongside
    d_pos, t_pos = inp["sc_d"].cpu(), inp["sc_t"].cpu()
    donors = [x.cpu() for x in inp["donors"]]
    caches = [torch.zeros((POOL_BLOCKS, 2, HKV, BS, D), dtype=torch.bfloat16)
              for _ in range(L)]

    def scatter_all():
        for layer in range(L):
            ref.scatter_donor_kv_paged(caches[layer], donors[layer], bt, d_pos, t_pos)

    dt_s = median_time(scatter_all)
    out["scatter_gbps"] = float(d_pos.shape[0]) * L * 2 * HKV * D * 2 * 2 / dt_s / 1e9
    del caches, donors
    k = inp["rope_k"][0].cpu()
    dt_r = median_time(lambda: ref.rope_correct_k(k, inp["rope_d"].cpu(), inp["rope_t"].cpu(),
                                                  head_dim=D, rope_base=ROPE_BASE))
    out["rope_gbps"] = k.numel() * 2 * 2 / dt_r / 1e9
    out["sample"] += (f"; scatter {d_pos.shape[0]} pairs x {L} layers {dt_s:.2f} s; "
                      f"rope {ROPE_TOKENS} tokens x {L} layers x {HKV} heads {dt_r:.2f} s")
    return out


def qwen05b_section(dev: torch.device, steps: int, cpu: bool) -> dict:
    """The one-layer Qwen2.5-0.5B pipeline (fp32, 1024 tokens): scatter, per-token RoPE in
    place (one call per distinct delta), 154-row GQA attention. GPU: the drop-in calls as a
    caller makes them, host work included (wall time around the synchronised pipeline,
    median over ``steps``); CPU: the oracle, median of 3."""
    from semblend_amd import rope_correction as rc
    from semblend_amd import triton_kernels as tk

    inp = qwen05b_pipeline_inputs(seed=0)
    c = QWEN05B
    rows = inp["rows"].double()
    flops = 4.0 * c["d"] * c["hq"] * float((rows + 1).sum())
    moved = float(c["ctx"]) * 2 * c["hkv"] * c["d"] * 4 * 2
    def timed(one_call: bool) -> float:
        qwen05b_pipeline(tk, rc, inp, device=dev, one_call=one_call)
        torch.cuda.synchronize()
        ts = []
        for _ in range(max(steps, 3)):
            t0 = time.perf_counter()
            qwen05b_pipeline(tk, rc, inp, device=dev, one_call=one_call)
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        return 1e3 * sorted(ts)[len(ts) // 2]

    gpu_ms = timed(False)
    one_ms = timed(True)
    res = {
        "workload": "Qwen2.5-0.5B one layer: 14q/2kv x 64, fp32, theta 1e6, 1024 tokens; "
                    "scatter into [128, 2, 2, 16, 64] (permuted block table), per-token "
                    "deltas in [-64, 64] applied in place (one call per distinct delta), "
                    "154 recompute rows",
        "rope_calls": len(delta_groups(inp["deltas"])),
        "attention_flops": flops, "scatter_bytes": moved,
        "gpu": {"ms": round(gpu_ms, 3), "what": "drop-in calls incl. host work, median"},
        "gpu_one_rope_call": {
            "ms": round(one_ms, 3),
            "what": "the same pipeline with the per-token deltas in one "
                    "apply_rope_deltas_inplace_layers call (same bits), incl. host work"},
    }
    if cpu:
        from oracle import ref_cpu as ref

        cpu_s = median_time(lambda: qwen05b_pipeline(ref, ref, inp))
        res["cpu_baseline"] = {"ms": round(1e3 * cpu_s, 1), "cores": torch.get_num_threads(),
                               "kind": "port", "timing": "median of 3",
                               "sample": "the whole pipeline (it is small)"}
    return res


def llama_batch_section(dev: torch.device, steps: int, cpu: bool) -> dict:
    """The Llama-3-8B batch (four requests, 8K-32K contexts, 10-30% recompute, 32 layers):
    RoPE scatter of every request into every layer's cache, then batched attention of all
    requests layer by layer. Reported beside the headline workload."""
    from semblend_amd import _lib
    from semblend_amd.batch import KVReuseBatch

    caches, reqs, theta = llama_batch(dev)
    batch = KVReuseBatch(caches, reqs, rope_base=theta)
    layers, hq, hkv, d = LLAMA["layers"], LLAMA["hq"], LLAMA["hkv"], LLAMA["d"]
    gd = torch.Generator(dev).manual_seed(5)
    q = torch.randn((batch.num_rows, hq, d), generator=gd, device=dev, dtype=torch.bfloat16)
    out = torch.empty_like(q)
    pairs = sum(int(r.donor_positions.shape[0]) for r in reqs)
    moved = float(pairs) * layers * 2 * hkv * d * 2 * 2
    sum_p1 = sum(float((r.compute_positions.double() + 1).sum().cpu()) for r in reqs)
    flops = 4.0 * d * hq * sum_p1 * layers

    def step():
        batch.scatter_rope()
        for layer in range(layers):
            batch.attention(layer, q, out=out)

    step()
    torch.cuda.synchronize()
    _lib.kernel_timing(True)
    e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    t_sr, t_at = [], []
    for _ in range(steps):
        e[0].record()
        batch.scatter_rope()
        e[1].record()
        for layer in range(layers):
            batch.attention(layer, q, out=out)
        e[2].record()
        torch.cuda.synchronize()
        t_sr.append(e[0].elapsed_time(e[1]))
        t_at.append(e[1].elapsed_time(e[2]))
    _lib.kernel_timing(False)
    mfma_ms, n = _lib.kernel_time("attn_mfma")
    sr_ms = sum(t_sr) / len(t_sr)
    at_ms = sum(t_at) / len(t_at)
    res = {
        "workload": "Llama-3-8B KV reuse batch: 32 layers, 32q/8kv x 128, bf16, theta 5e5; "
                    "requests of 8192/16384/24576/32768 tokens with 10/15/20/30% recompute "
                    "(chunk-constant deltas in [-4096, 4096]); shared pool of 8192 blocks of 16",
        "requests": len(reqs),
        "rows": batch.num_rows,
        "pairs": pairs,
        "steps": steps,
        "scatter_rope": {"ms": round(sr_ms, 4), "bytes": moved,
                         "gbps": round(moved / (sr_ms * 1e-3) / 1e9, 1),
                         "frac_of_peak": round(moved / (sr_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "attention": {"ms": round(at_ms, 4), "flops": flops,
                      "tflops": round(flops / (at_ms * 1e-3) / 1e12, 2),
                      "frac_of_peak": round(flops / (at_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                      "mfma_kernel_ms": round(mfma_ms / max(steps, 1), 4)},
        "ms_per_step": round(sr_ms + at_ms, 4),
    }
    if cpu:
        # Oracle on layer 0, extrapolated to 32 layers: the RoPE scatter of every pair of
        # every request into layer 0, and attention for one in 16 recompute rows of every
        # request (rows spread evenly over each request's positions) scaled by the FLOP
        # share of the sample. Median of 3 each.
        from oracle import ref_cpu as ref

        kv0 = caches[0].cpu()
        donors0 = [r.donor_kvs[0].cpu() for r in reqs]
        tables = [r.block_table.cpu() for r in reqs]
        dps = [r.donor_positions.cpu() for r in reqs]
        tps = [r.target_positions.cpu() for r in reqs]

        def scatter_layer0():
            for i in range(len(reqs)):
                ref.rope_correct_scatter_paged(kv0, donors0[i], tables[i], dps[i], tps[i],
                                               rope_base=theta)

        dt_s = median_time(scatter_layer0)
        qs, poss, sample_p1 = [], [], 0.0
        for i, r in enumerate(reqs):
            a0 = batch.row_offsets[i]
            sel = torch.arange(0, r.compute_positions.shape[0], 16)
            qs.append(q[a0:a0 + r.compute_positions.shape[0]].cpu()[sel])
            poss.append(r.compute_positions.cpu()[sel])
            sample_p1 += float((poss[-1].double() + 1).sum())

        def attn_sample():
            for i in range(len(reqs)):
                ref.partial_attention_paged(qs[i], kv0, tables[i], poss[i])

        dt_a = median_time(attn_sample)
        sample_flops = 4.0 * d * hq * sample_p1
        attn_s = dt_a * flops / sample_flops
        sr_s = dt_s * layers
        res["cpu_baseline"] = {
            "extrapolated": True,
            "scatter_rope_ms": round(1e3 * sr_s, 1),
            "scatter_rope_gbps": moved / sr_s / 1e9,
            "attention_ms": round(1e3 * attn_s, 1),
            "attention_tflops": flops / attn_s / 1e12,
            "cores": torch.get_num_threads(), "kind": "port", "timing": "median of 3",
            "sample": f"layer 0: RoPE scatter of all {pairs} pairs ({dt_s:.2f} s, x{layers} "
                      f"layers) and attention of every 16th recompute row of each request "
                      f"({sum(x.shape[0] for x in poss)} rows, {dt_a:.2f} s, scaled by "
                      f"{flops / sample_flops:.1f}x = total / sampled FLOPs)"}
    del caches, reqs, batch
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


def rope_scatter_section(dev: torch.device, inp, steps: int) -> dict:
    """Fused RoPE scatter of the 28-layer scatter workload (same 13926 pairs and bytes), from
    one donor (``rope_correct_scatter_paged_layers``) and as a composite from four donors
    (each 256-token target chunk owned by a random one of four 16384-token donors,
    ``prepare_composite_scatter_paged_layers``, pairs grouped by donor; and, as
    ``four_donors_indexed``, the per-call form with a per-pair donor index), K rotated by a
    per-chunk delta. Graph replays timed with HIP events, each after a RoPE pass (as in a step)
    and back to back."""
    from semblend_amd import rope_correction as rc
    from semblend_amd.multi_donor import (composite_scatter_paged_layers,
                                          prepare_composite_scatter_paged_layers)

    g = torch.Generator("cpu").manual_seed(3)
    gd = torch.Generator(dev).manual_seed(3)
    n_donors = 4
    donors = [inp["donors"]] + [
        [torch.randn((2, HKV, CTX, D), generator=gd, device=dev, dtype=torch.bfloat16)
         for _ in range(L)] for _ in range(n_donors - 1)]
    owner = torch.randint(0, n_donors, (CTX // CHUNK,), generator=g)
    didx = owner[inp["sc_t"].cpu().long() // CHUNK].to(torch.int32).to(dev)
    n_pairs = inp["sc_d"].shape[0]
    nbytes = float(n_pairs) * L * 2 * HKV * D * 2 * 2

    def one_donor():
        rc.rope_correct_scatter_paged_layers(inp["caches"], inp["donors"], inp["block_table"],
                                             inp["sc_d"], inp["sc_t"], rope_base=ROPE_BASE)

    def four_donors_indexed():
        composite_scatter_paged_layers(inp["caches"], donors, inp["block_table"], didx,
                                       inp["sc_d"], inp["sc_t"], rope=True, rope_base=ROPE_BASE)

    # bound once per request, pairs grouped by donor (each workgroup's pairs share a donor)
    four_donors = prepare_composite_scatter_paged_layers(
        inp["caches"], donors, inp["block_table"], didx.cpu(), inp["sc_d"].cpu(),
        inp["sc_t"].cpu(), rope=True, rope_base=ROPE_BASE)

    # Each replay is timed after a RoPE pass over K[28,4,8192,128] (470 MB through the
    # Infinity Cache, as in a step: the donor rows come from HBM) and, as ``back_to_back``,
    # right after the previous replay (part of the donor rows then still sit in the Infinity
    # Cache, as when a donor chunk was uploaded or computed just before).
    rope_gr = capture(lambda: rc.rope_correct_k_inplace(
        inp["rope_k"][0], inp["rope_d"], inp["rope_t"], head_dim=D, rope_base=ROPE_BASE,
        distinct_donors=True))
    out = {"pairs": int(n_pairs), "bytes": nbytes}
    for name, fn in (("one_donor", one_donor), ("four_donors", four_donors),
                     ("four_donors_indexed", four_donors_indexed)):
        gr = capture(fn)
        gr.replay()
        torch.cuda.synchronize()
        times = {}
        for ctx in ("after_rope", "back_to_back"):
            evs = []
            for _ in range(steps):
                if ctx == "after_rope":
                    rope_gr.replay()
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record()
                gr.replay()
                e1.record()
                evs.append((e0, e1))
            torch.cuda.synchronize()
            times[ctx] = [a.elapsed_time(b) for a, b in evs]
        t = times["after_rope"]
        avg = sum(t) / len(t)
        t2 = times["back_to_back"]
        avg2 = sum(t2) / len(t2)
        out[name] = {"ms": round(avg, 4), "ms_median": round(sorted(t)[len(t) // 2], 4),
                     "gbps": round(nbytes / (avg * 1e-3) / 1e9, 1),
                     "frac_of_peak": round(nbytes / (avg * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "back_to_back": {
                         "ms": round(avg2, 4),
                         "gbps": round(nbytes / (avg2 * 1e-3) / 1e9, 1),
                         "frac_of_peak": round(nbytes / (avg2 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}}
        del gr
    del rope_gr
    return out


def chunk_load_section(dev: torch.device, inp, steps: int) -> dict:
    """The donor of the scatter workload (16384 tokens x 28 layers, 939.5 MB) held in host
    memory as 64 LMCache chunks [2, 28, 256, 512] (pinned), loaded into the paged caches
    with RoPE on the way (13926 pairs, per-chunk delta). Three schedules, each timed with
    HIP events on the current stream: the copies alone (the PCIe ceiling), copy-then-scatter
    on one stream (no overlap), and ChunkedKVLoader (8 staging slots; scatters on their own
    stream, overlapped with the copies)."""
    from semblend_amd.loader import ChunkedKVLoader, group_pairs_by_chunk
    from semblend_amd.multi_donor import composite_scatter_paged_layers

    T = CHUNK
    n_chunks = CTX // T
    chunks = []
    for c in range(n_chunks):
        x = torch.stack([dn[:, :, c * T:(c + 1) * T].permute(0, 2, 1, 3) for dn in inp["donors"]],
                        dim=1).reshape(2, L, T, HKV * D)
        h = torch.empty(x.shape, dtype=x.dtype, pin_memory=True)
        h.copy_(x)
        chunks.append(h)
    host_bytes = float(sum(h.numel() * h.element_size() for h in chunks))
    dpos = inp["sc_d"].cpu().numpy()
    tpos = inp["sc_t"].cpu().numpy()
    loader = ChunkedKVLoader(inp["caches"], inp["block_table"], chunk_tokens=T, slots=8,
                             rope_base=ROPE_BASE)
    arr, offs = group_pairs_by_chunk(dpos, tpos, T, n_chunks)
    pairs = torch.from_numpy(arr).to(dev)
    staging = torch.empty((2, L, T, HKV, D), dtype=torch.bfloat16, device=dev)

    def copies_only():
        for h in chunks:
            staging.copy_(h.view(2, L, T, HKV, D), non_blocking=True)

    def serial():
        for c, h in enumerate(chunks):
            staging.copy_(h.view(2, L, T, HKV, D), non_blocking=True)
            lo, hi = int(offs[c]), int(offs[c + 1])
            composite_scatter_paged_layers(
                inp["caches"], [[staging[:, l].permute(0, 2, 1, 3) for l in range(L)]],
                inp["block_table"], pairs[2, lo:hi], pairs[0, lo:hi], pairs[1, lo:hi],
                rope=True, rope_base=ROPE_BASE, donor_first_positions=[c * T])

    def streamed():
        loader.load(chunks, dpos, tpos, rope=True)

    out = {"chunks": n_chunks, "chunk_shape": [2, L, T, HKV * D], "host_bytes": host_bytes,
           "pairs": int(len(dpos))}
    for name, fn in (("copies_only", copies_only), ("serial", serial), ("streamed", streamed)):
        fn()
        torch.cuda.synchronize()
        t = []
        for _ in range(steps):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            t.append(e0.elapsed_time(e1))
        avg = sum(t) / len(t)
        out[name] = {"ms": round(avg, 3), "host_gbps": round(host_bytes / (avg * 1e-3) / 1e9, 1)}
    out["overlap_efficiency"] = round(out["copies_only"]["ms"] / out["streamed"]["ms"], 4)
    del loader, chunks
    return out


QWEN7B_HIDDEN = 3584


def projection_section(dev: torch.device, inp, steps: int) -> dict:
    """Compacted QKV projection of the attention workload's recompute rows (Qwen2.5-7B:
    hidden 3584 -> 28 q + 2 x 4 KV heads x 128 = 4608 features, QKV bias), RoPE theta 1e6 at
    the new positions, K/V written into the paged cache: ``qkv_projection_paged`` with the
    fused MFMA kernel (graph replays and per launch) and with the library GEMM plus the
    epilogue kernel (graph replays). For comparison, torch on the same rows: gather + addmm
    (hipBLASLt), without RoPE and without the K/V write."""
    from semblend_amd import _lib
    from semblend_amd import triton_kernels as tk

    hidden = QWEN7B_HIDDEN
    feats = (HQ + 2 * HKV) * D
    gd = torch.Generator(dev).manual_seed(5)
    x = torch.randn((CTX, hidden), generator=gd, device=dev, dtype=torch.bfloat16)
    w = (torch.randn((feats, hidden), generator=gd, device=dev) * hidden ** -0.5).to(torch.bfloat16)
    b = torch.randn((feats,), generator=gd, device=dev, dtype=torch.bfloat16)
    pos = inp["attn_pos"]
    rows = int(pos.shape[0])
    q = torch.empty((rows, HQ, D), dtype=torch.bfloat16, device=dev)
    flops = 2.0 * rows * hidden * feats

    def fused():
        tk.qkv_projection_paged(x, w, pos, inp["attn_kv"], inp["block_table"], HQ, HKV, D,
                                qkv_bias=b, rope_base=ROPE_BASE, out=q, backend="fused")

    def library_epilogue():
        tk.qkv_projection_paged(x, w, pos, inp["attn_kv"], inp["block_table"], HQ, HKV, D,
                                qkv_bias=b, rope_base=ROPE_BASE, out=q, backend="library")

    pos_l = pos.long()

    def library():
        torch.addmm(b, x[pos_l], w.t())

    def timed(fn, graph: bool):
        fn()
        torch.cuda.synchronize()
        gr = capture(fn) if graph else None
        evs = []
        for _ in range(steps):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            gr.replay() if graph else fn()
            e1.record()
            evs.append((e0, e1))
        torch.cuda.synchronize()
        t = [a.elapsed_time(c) for a, c in evs]
        return sum(t) / len(t)

    ms_fused = timed(fused, True)
    _lib.kernel_timing(True)
    for _ in range(steps):
        fused()
    torch.cuda.synchronize()
    _lib.kernel_timing(False)
    total, n = _lib.kernel_time("qkv_mfma")
    kern_us = 1e3 * total / n
    ms_lib = timed(library, False)
    ms_lib_epi = timed(library_epilogue, True)
    wo = (torch.randn((hidden, HQ * D), generator=gd, device=dev) * (HQ * D) ** -0.5).to(
        torch.bfloat16)

    def layer():
        tk.partial_prefill_layer_paged(x, w, wo, pos, inp["attn_kv"], inp["block_table"], HQ,
                                       HKV, D, qkv_bias=b, rope_base=ROPE_BASE)

    ms_layer = timed(layer, False)
    # the same layer with the request's attention plan, made once (as for every layer of it)
    layer_plan = tk.plan_partial_attention_paged(inp["pos_cpu"], HQ, HKV, D, BS,
                                                 inp["block_table"].shape[0], torch.bfloat16,
                                                 dev)

    def layer_planned():
        tk.partial_prefill_layer_paged(x, w, wo, pos, inp["attn_kv"], inp["block_table"], HQ,
                                       HKV, D, qkv_bias=b, rope_base=ROPE_BASE, plan=layer_plan)

    ms_layer_planned = timed(layer_planned, False)
    return {
        "rows": rows, "hidden": hidden, "features": feats, "flops": flops,
        "fused": {"ms": round(ms_fused, 4), "tflops": round(flops / (ms_fused * 1e-3) / 1e12, 1)},
        "kernel": {"avg_us": round(kern_us, 2),
                   "tflops": round(flops / (kern_us * 1e-6) / 1e12, 1),
                   "frac_of_peak": round(flops / (kern_us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4)},
        "library_with_epilogue": {
            "ms": round(ms_lib_epi, 4), "tflops": round(flops / (ms_lib_epi * 1e-3) / 1e12, 1),
            "what": "qkv_projection_paged(backend='library'): row gather + hipBLASLt GEMM "
                    "(fp32 out) + the epilogue kernel (bias, RoPE, Q and paged K/V write)"},
        "torch_gather_addmm": {"ms": round(ms_lib, 4),
                               "tflops": round(flops / (ms_lib * 1e-3) / 1e12, 1),
                               "what": "x[pos] @ W^T + b via torch (hipBLASLt), no RoPE, no K/V write"},
        "layer": {"ms": round(ms_layer, 4),
                  "planned_ms": round(ms_layer_planned, 4),
                  "what": "partial_prefill_layer_paged: projection + K/V write + RoPE, paged "
                          "GQA attention, output projection (3584 x 3584) of the 2458 rows; "
                          "planned_ms with the request's attention plan"},
    }


def capture(fn) -> "torch.cuda.CUDAGraph":
    """One launch sequence of fn captured as a HIP graph (after an eager run on the capture
    stream, so that every cached device table already exists)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-llama-batch", action="store_true",
                    help="skip the Llama-3-8B multi-request batch section")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the library has no multi-GPU path "
              "(each GPU would own its own layers or KV heads with no exchange). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    from semblend_amd import _lib
    from semblend_amd import rope_correction as rc
    from semblend_amd import triton_kernels as tk

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log("building inputs")
    inp = build_inputs(dev)
    torch.cuda.synchronize()

    pos = inp["pos_cpu"].double()
    attn_flops = 4.0 * D * HQ * float((pos + 1).sum())
    n_pairs = inp["sc_d"].shape[0]
    scatter_bytes = float(n_pairs) * L * 2 * HKV * D * 2 * 2
    rope_bytes = float(L * HKV * ROPE_TOKENS * D * 2 * 2)

    def phase_rope(i):
        # every position is named once (d = 0..8191): the one-launch distinct-donor form
        rc.rope_correct_k_inplace(inp["rope_k"][i % 4], inp["rope_d"], inp["rope_t"],
                                  head_dim=D, rope_base=ROPE_BASE, distinct_donors=True)

    def rope_indexed(i):
        # the general form (per-position pair index built on the device, then the rotation)
        rc.rope_correct_k_inplace(inp["rope_k"][i % 4], inp["rope_d"], inp["rope_t"],
                                  head_dim=D, rope_base=ROPE_BASE)

    def phase_scatter(i):
        tk.scatter_donor_kv_paged_layers(inp["caches"], inp["donors"], inp["block_table"],
                                         inp["sc_d"], inp["sc_t"])

    # The attention launch is planned once from the host positions (as a serving loop plans a
    # request once and reuses the plan for every layer): key split and longest-first order.
    attn_plan = tk.plan_partial_attention_paged(inp["pos_cpu"], HQ, HKV, D, BS,
                                                inp["block_table"].shape[0], torch.bfloat16,
                                                dev)

    def phase_attn(i):
        tk.partial_prefill_attention_paged(inp["attn_q"], inp["attn_kv"], inp["block_table"],
                                           inp["attn_pos"], out=inp.setdefault(
                                               "attn_out", torch.empty_like(inp["attn_q"])),
                                           plan=attn_plan)

    def attn_unplanned(i):
        tk.partial_prefill_attention_paged(inp["attn_q"], inp["attn_kv"], inp["block_table"],
                                           inp["attn_pos"], out=inp["attn_out"])

    phases = [("rope", phase_rope), ("scatter", phase_scatter), ("attention", phase_attn)]
    log(f"warmup {args.warmup}")
    for i in range(max(1, args.warmup)):
        for _, fn in phases:
            fn(i)
    torch.cuda.synchronize()

    # Per-kernel durations: eager passes with HIP events attached to each library launch, in
    # three rounds that alternate a pass of whole steps (RoPE, scatter, planned attention)
    # with a pass of the unplanned attention (after the scatter, as in a step); each kernel's
    # figure is the median of its three round averages (so that neither form always runs
    # first after the warm-up).
    log(f"kernel timing passes (3 rounds of {args.steps} eager steps, two forms each)")

    def timed_pass(fns) -> dict:
        _lib.kernel_timing(True)
        for i in range(args.steps):
            for fn in fns:
                fn(i)
        torch.cuda.synchronize()
        _lib.kernel_timing(False)
        return {name: _lib.kernel_time(name) for name in KERNELS}

    main_fns = [fn for _, fn in phases]
    unplanned_fns = [phase_scatter, attn_unplanned]
    rounds = {"main": [], "unplanned": []}
    for r in range(3):
        order = ["main", "unplanned"] if r % 2 == 0 else ["unplanned", "main"]
        for tag in order:
            rounds[tag].append(timed_pass(main_fns if tag == "main" else unplanned_fns))

    def median_avg_us(tag: str, name: str) -> tuple[float, int]:
        avgs = sorted(1e3 * t / n for t, n in (rd[name] for rd in rounds[tag]) if n)
        n_total = sum(rd[name][1] for rd in rounds[tag])
        return (avgs[len(avgs) // 2] if avgs else 0.0), n_total

    kernels = {}
    for name in KERNELS:
        avg_us, n = median_avg_us("main", name)
        if n:
            kernels[name] = {"launches": n, "avg_us": round(avg_us, 2)}
    unplanned = {name: round(median_avg_us("unplanned", name)[0], 2)
                 for name in ("attn_mfma", "attn_merge")}

    log("capturing one HIP graph per step (RoPE, scatter, attention) and one per phase")

    def one_step(c):
        phase_rope(c)
        phase_scatter(c)
        phase_attn(c)

    step_graphs = [capture(lambda c=c: one_step(c)) for c in range(4)]
    graphs = {
        "rope": [capture(lambda c=c: phase_rope(c)) for c in range(4)],
        "scatter": [capture(lambda: phase_scatter(0))],
        "attention": [capture(lambda: phase_attn(0))],
    }
    for g in step_graphs:
        g.replay()
    torch.cuda.synchronize()

    # The timed region: K whole steps, each one graph replay (the step's kernels run back to
    # back inside it), all enqueued back to back between one pair of HIP events.
    log(f"timing {args.steps} steps (whole-step graph replays)")
    torch.cuda.synchronize()
    t_wall0 = time.perf_counter()
    e_step0 = torch.cuda.Event(enable_timing=True)
    e_step1 = torch.cuda.Event(enable_timing=True)
    e_step0.record()
    for i in range(args.steps):
        step_graphs[i % 4].replay()
    e_step1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall0
    ms_per_step = e_step0.elapsed_time(e_step1) / args.steps

    # Launch-inclusive phase times: each phase as its own graph, events around every replay,
    # phases interleaved as in a step (each includes one graph launch, ~8 us on this GPU).
    ev = {name: [] for name, _ in phases}
    for i in range(args.steps):
        for name, _ in phases:
            gs = graphs[name]
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            gs[i % len(gs)].replay()
            e1.record()
            ev[name].append((e0, e1))
    torch.cuda.synchronize()
    launch_ms = {name: sum(a.elapsed_time(b) for a, b in v) / len(v) for name, v in ev.items()}
    idx_graphs = [capture(lambda c=c: rope_indexed(c)) for c in range(4)]
    idx_ev = []
    for i in range(args.steps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        idx_graphs[i % 4].replay()
        e1.record()
        idx_ev.append((e0, e1))
        phase_scatter(0)  # keep the interleaving: K must not stay in the Infinity Cache
    torch.cuda.synchronize()
    rope_idx_ms = sum(a.elapsed_time(b) for a, b in idx_ev) / len(idx_ev)
    del idx_graphs, step_graphs
    copy_rates = copy_ceiling(dev)
    copy_gbps = copy_rates["library"]
    gemm_tflops = gemm_ceiling(dev)
    log("kernels (avg us): " + ", ".join(f"{k} {v['avg_us']}" for k, v in kernels.items())
        + f"; copy ceiling {copy_gbps:.0f} GB/s (torch copy_ {copy_rates['torch']:.0f})")
    # Phase durations on the GPU: the phase's kernels, each bracketed by HIP events that the
    # runtime stamps with the kernel's start and end, in the interleaved eager pass above.
    avg = {"rope": kernels["rope_rows"]["avg_us"] * 1e-3,
           "scatter": kernels["move_rows"]["avg_us"] * 1e-3,
           "attention": (kernels["attn_mfma"]["avg_us"] + kernels["attn_merge"]["avg_us"]) * 1e-3}

    attn_tflops = attn_flops / (avg["attention"] * 1e-3) / 1e12
    # Dominant kernel: the MFMA attention kernel, one launch per step.
    mfma_us = kernels["attn_mfma"]["avg_us"]
    mfma_tflops = attn_flops / (mfma_us * 1e-6) / 1e12
    scatter_gbps = scatter_bytes / (avg["scatter"] * 1e-3) / 1e9
    rope_gbps = rope_bytes / (avg["rope"] * 1e-3) / 1e9
    log(f"attention {avg['attention']:.3f} ms ({attn_tflops:.1f} TFLOP/s), "
        f"scatter {avg['scatter']:.3f} ms ({scatter_gbps:.0f} GB/s), "
        f"rope {avg['rope']:.3f} ms ({rope_gbps:.0f} GB/s), wall {wall:.3f} s")

    result = {
        "metric": "partial-attn TFLOP/s + scatter/RoPE GB/s @7B GQA 16K ctx; % of roofline",
        "value": round(attn_tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "Qwen2.5-7B KV reuse, 16K context: partial attention 28q/4kv x 128 "
                        "over 16384 paged tokens, |R|=2458; scatter 28 layers x 13926 pairs; "
                        "RoPE K[28,4,8192,128] theta 1e6",
            "attention_rows": int(inp["pos_cpu"].shape[0]),
            "attention_flops": attn_flops,
            "scatter_pairs": int(n_pairs),
            "scatter_bytes": scatter_bytes,
            "rope_bytes": rope_bytes,
            "block_size": BS,
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "attn_mfma_kernel",
            "achieved": round(mfma_tflops, 2),
            "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(mfma_tflops / BF16_PEAK_TFLOPS, 4),
            "traffic": MEASURED_TRAFFIC_BYTES["attn_mfma"],
            "traffic_source": MEASURED_TRAFFIC_SOURCE,
        },
        "phases": {
            "attention": {"ms": round(avg["attention"], 4),
                          "launch_inclusive_ms": round(launch_ms["attention"], 4),
                          "tflops": round(attn_tflops, 2),
                          "frac_of_peak": round(attn_tflops / BF16_PEAK_TFLOPS, 4),
                          "plan": {"ks_first": attn_plan.ks_first,
                                   "ks_rest": attn_plan.ks_rest,
                                   "max_chunks": attn_plan.max_chunks,
                                   "what": "host plan from the recompute positions: key split "
                                           "and longest-first dispatch order"},
                          "unplanned": {
                              "attn_mfma_us": unplanned["attn_mfma"],
                              "attn_merge_us": unplanned["attn_merge"],
                              "tflops": round(attn_flops / ((unplanned["attn_mfma"]
                                                             + unplanned["attn_merge"])
                                                            * 1e-6) / 1e12, 2),
                              "what": "the same call without a plan (default split, "
                                      "workgroup order)"}},
            "scatter": {"ms": round(avg["scatter"], 4),
                        "launch_inclusive_ms": round(launch_ms["scatter"], 4),
                        "gbps": round(scatter_gbps, 1),
                        "kernel_gbps": round(scatter_bytes / (kernels["move_rows"]["avg_us"] * 1e-6) / 1e9, 1),
                        "traffic_bytes": MEASURED_TRAFFIC_BYTES["move_rows"],
                        "frac_of_peak": round(scatter_gbps / HBM_PEAK_GBS, 4),
                        "frac_of_copy": round(scatter_gbps / copy_gbps, 4)},
            "rope": {"ms": round(avg["rope"], 4),
                     "launch_inclusive_ms": round(launch_ms["rope"], 4),
                     "gbps": round(rope_gbps, 1),
                     "kernel_gbps": round(rope_bytes / (kernels["rope_rows"]["avg_us"] * 1e-6) / 1e9, 1),
                     "traffic_bytes": MEASURED_TRAFFIC_BYTES["rope_rows"],
                     "frac_of_peak": round(rope_gbps / HBM_PEAK_GBS, 4),
                     "frac_of_copy": round(rope_gbps / copy_gbps, 4),
                     "what": "one launch per step (donor positions distinct: d = 0..8191)",
                     "indexed": {"ms": round(rope_idx_ms, 4),
                                 "gbps": round(rope_bytes / (rope_idx_ms * 1e-3) / 1e9, 1),
                                 "what": "general form: pair index on the device, then the "
                                         "rotation (two launches)"}},
            "gemm_ceiling": {"tflops": round(gemm_tflops, 1),
                             "frac_of_peak": round(gemm_tflops / BF16_PEAK_TFLOPS, 4),
                             "what": "8192^3 bf16 torch matmul (hipBLASLt), 10 repeats"},
            "copy_ceiling": {"gbps": round(copy_gbps, 1),
                             "frac_of_peak": round(copy_gbps / HBM_PEAK_GBS, 4),
                             "torch_copy_gbps": round(copy_rates["torch"], 1),
                             "what": "1 GiB device-to-device copy through the library's flat "
                                     "copy kernel (one 16-byte vector per thread, "
                                     "nontemporal), 10 repeats; torch copy_ beside it"},
        },
        "kernels": kernels,
    }
    log("fused RoPE scatter: one donor and four-donor composite")
    result["rope_scatter"] = rope_scatter_section(dev, inp, args.steps)
    rs = result["rope_scatter"]
    for k in ("one_donor", "four_donors", "four_donors_indexed"):
        rs[k]["frac_of_copy"] = round(rs[k]["gbps"] / copy_gbps, 4)
        rs[k]["back_to_back"]["frac_of_copy"] = round(rs[k]["back_to_back"]["gbps"] / copy_gbps, 4)
    log(f"rope scatter: one donor {rs['one_donor']['ms']:.3f} ms ({rs['one_donor']['gbps']:.0f} GB/s), "
        f"four donors {rs['four_donors']['ms']:.3f} ms ({rs['four_donors']['gbps']:.0f} GB/s)")
    log("compacted QKV projection with the K/V write")
    result["projection"] = projection_section(dev, inp, args.steps)
    pj = result["projection"]
    log(f"projection: library+epilogue {pj['library_with_epilogue']['ms']:.4f} ms; "
        f"fused {pj['fused']['ms']:.4f} ms ({pj['fused']['tflops']} TFLOP/s), kernel "
        f"{pj['kernel']['avg_us']} us ({pj['kernel']['tflops']} TFLOP/s), torch gather+addmm "
        f"{pj['torch_gather_addmm']['ms']:.4f} ms ({pj['torch_gather_addmm']['tflops']} TFLOP/s); "
        f"whole layer {pj['layer']['ms']:.3f} ms")
    log("chunked host-to-device donor load with RoPE on the way")
    result["chunk_load"] = chunk_load_section(dev, inp, 5)
    cl = result["chunk_load"]
    log(f"chunk load: copies only {cl['copies_only']['ms']:.2f} ms "
        f"({cl['copies_only']['host_gbps']:.1f} GB/s), serial {cl['serial']['ms']:.2f} ms, "
        f"streamed {cl['streamed']['ms']:.2f} ms (overlap {cl['overlap_efficiency']:.3f})")
    log("Qwen2.5-0.5B one-layer pipeline (fp32)")
    result["qwen05b_pipeline"] = qwen05b_section(dev, args.steps, not args.no_cpu_baseline)
    qp = result["qwen05b_pipeline"]
    log(f"qwen0.5b pipeline: gpu {qp['gpu']['ms']:.3f} ms"
        + (f", cpu {qp['cpu_baseline']['ms']:.1f} ms" if "cpu_baseline" in qp else ""))
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle on host cores)")
        result["cpu_baseline"] = cpu_baseline(inp)
    if not args.no_llama_batch:
        log("Llama-3-8B batch section")
        del inp, graphs
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        result["llama3_8b_batch"] = llama_batch_section(dev, 3, not args.no_cpu_baseline)
        lb = result["llama3_8b_batch"]
        lb["scatter_rope"]["frac_of_copy"] = round(lb["scatter_rope"]["gbps"] / copy_gbps, 4)
        log(f"llama batch: scatter+rope {lb['scatter_rope']['ms']:.2f} ms "
            f"({lb['scatter_rope']['gbps']:.0f} GB/s), attention {lb['attention']['ms']:.2f} ms "
            f"({lb['attention']['tflops']:.1f} TFLOP/s)")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
