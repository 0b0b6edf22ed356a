"""Benchmark of the paged-KV attention path on one MI355X.

Headline (the JSON line's `value`): paged decode attention at the
Llama-2-7B shape — 32 layers, 32/32 heads, head_dim 128, fp16 KV in a
16384-page pool of 16-token pages, batch 64 with contexts
lognormal(median 700) clipped to [16, 4096]. One step is one decode sweep
over the 32 layers (one launch per layer, each layer with its own q).
`value` is algorithmic KV bytes moved per second (K and V of every cached
token once, plus q, out and page ids) with all inputs resident in HBM.

Also measured: `prefill` — chunked-prefill attention with K/V append (16
sequences, prompts U[512, 4096], prefixes U[0, 2048], chunk 512) as MFMA
utilisation of the fp16 dense peak (and `prefill_page256`, the same
workload on 256-token pages, the reference's default block size, and
`bf16_prefill_page256` on a bf16 pool of 256-token pages, both reference
defaults; `prefill_head_dim64` and `prefill_head_dim256`, the same rows and
heads at head_dim 64 and 256, and `prefill_gqa8`, the same rows with
Llama-3-8B's 32 query / 8 KV heads, attention only), beside `mfma_ceiling`, the
rate the part sustains on fp16 MFMAs with random and with constant operands;
`gqa_decode` — Llama-3-8B GQA decode (32/8 heads, batch 128, contexts
U[1024, 8192]) as HBM bandwidth; `bf16_decode` — the headline decode on a
bf16 pool (the reference's default dtype), and `bf16_decode_page256` on a
bf16 pool of 256-token pages (both reference defaults); `remap` — the 8192-block remap
copy as HBM bandwidth and a Llama-2-70B layer decode
(64/8 heads, batch 256) on the remapped tables, bit-exact against the
original tables; `pmm` — the Llama-2-7B decode on a pool whose last 784
pages are 16 dropped Llama-2-7B weight layers (pmm_drop), with the drop and
restore time per layer; `swap` — 512 random blocks swapped out to pinned
host memory and back, against a contiguous copy over the same link.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3]
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

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
FP16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 (and bf16) MFMA, TFLOP/s
METRIC = "paged decode attn KV GB/s & % HBM peak at Llama-7B shape; prefill MFMA util"
PROFILE_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def fill_random_(t: torch.Tensor, gen: torch.Generator, slab_dim: int = 1) -> None:
    """N(0,1) fp16 fill, one slice along slab_dim at a time (bounded temp)."""
    for i in range(t.shape[slab_dim]):
        s = t.select(slab_dim, i)
        s.copy_(torch.randn(s.shape, generator=gen, device=t.device, dtype=torch.float32))


def region_ms(fn, device) -> float:
    """Milliseconds of GPU time of `fn()` (which enqueues work on the
    current stream): HIP events on that stream before and after it. One
    event pair around a whole pass leaves out the packets that events
    around every launch add (about 5 us per launch)."""
    stream = torch.cuda.current_stream(device)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    fn()
    ev1.record(stream)
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1)


def power_during(fn, device, seconds: float = 4.0):
    """Socket power and GFX clock (amd-smi, sampled from a thread about every
    0.3 s) while `fn()` runs back to back for `seconds`; None without
    amd-smi. The part holds its power limit by lowering the clock, so a
    kernel's clock under load says how much of the part's clock it keeps."""
    import re
    import shutil
    import subprocess
    import threading

    if not shutil.which("amd-smi"):
        return None
    samples = []
    stop = threading.Event()

    def sampler():
        while not stop.is_set():
            try:
                out = subprocess.run(["amd-smi", "metric", "-g", "0", "-p", "-c"],
                                     capture_output=True, text=True, timeout=10).stdout
            except (OSError, subprocess.SubprocessError):
                return
            pw = re.search(r"SOCKET_POWER:\s*(\d+)", out)
            clk = [int(x) for x in re.findall(r"GFX_\d+:\s+CLK:\s*(\d+) MHz", out)]
            if pw and clk and not stop.is_set():   # read while the loop still ran
                samples.append((int(pw.group(1)), float(np.median(clk))))
            stop.wait(0.3)

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 1.0:   # reach the steady clock before sampling
        fn()
        torch.cuda.synchronize()
    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        fn()
        torch.cuda.synchronize()
    stop.set()
    th.join(timeout=15)
    if not samples:
        return None
    pw = [p for p, _ in samples]
    ck = [c for _, c in samples]
    return {"socket_power_w": [min(pw), float(np.median(pw)), max(pw)],
            "gfx_clock_mhz": [min(ck), float(np.median(ck)), max(ck)], "samples": len(samples)}


class LaunchTimer:
    """HIP events around each launch on the current stream."""

    def __init__(self):
        self.pairs = []

    def start(self):
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        return e

    def stop(self, start):
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        self.pairs.append((start, e))

    def mean_ms(self) -> float:
        torch.cuda.synchronize()
        return float(np.mean([a.elapsed_time(b) for a, b in self.pairs]))


# ------------------------------------------------------------------ decode


def measure_decode(w, pool, layers, args, device, indices_override=None, q_scale=1.0):
    """Times paged_decode over `layers` of `pool` for workload `w`: one step
    is one launch per layer. Returns the timing and the objects used."""
    import kunserve_amd as ks

    gen = torch.Generator(device=device)
    gen.manual_seed(w.seed + 7)
    indptr, indices = w.csr()
    if indices_override is not None:
        indices = indices_override
    table = ks.PageTable(indptr, indices, w.kv_len, device)
    plan = ks.DecodePlan(w.kv_len, w.num_qo_heads, w.num_kv_heads, device,
                         part_tokens=args.part_tokens)
    ws = torch.zeros(max(plan.workspace_bytes(w.head_dim), 1), dtype=torch.uint8, device=device)
    qs = [(torch.randn((w.batch, w.num_qo_heads, w.head_dim), generator=gen, device=device
                       ) * q_scale).to(pool.k.dtype) for _ in layers]
    out = torch.empty_like(qs[0])

    def step():
        for i, layer in enumerate(layers):
            ks.paged_decode(pool, layer, table, qs[i], plan, out=out, workspace=ws)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    # Per-launch duration from HIP events on the launch stream around a
    # second pass over the same steps, divided by the launches in it.
    # Events around every launch would add their own packets (about 5 us
    # per launch) to what they measure.
    def timed_pass():
        for _ in range(args.steps):
            step()

    launch_ms = region_ms(timed_pass, device) / (args.steps * len(layers))
    bytes_per_layer = w.kv_bytes_per_layer()
    return {
        "value": bytes_per_layer * len(layers) * args.steps / elapsed / 1e9,
        "ms_per_step": elapsed / args.steps * 1e3,
        "launch_ms": launch_ms,
        "achieved": bytes_per_layer / (launch_ms * 1e-3) / 1e9,
        "bytes_per_layer": bytes_per_layer,
        "workload": w, "plan": plan, "pool": pool, "table": table, "qs": qs,
    }


def bench_decode(args, device):
    import kunserve_amd as ks
    from kunserve_amd import workloads

    w = workloads.llama2_7b_decode()
    log(f"decode workload: {w.name}; tokens {int(w.kv_len.sum())}, "
        f"{w.kv_bytes_per_layer() / 2**30:.3f} GiB per layer")
    gen = torch.Generator(device=device)
    gen.manual_seed(w.seed)
    pool = ks.KVPool.allocate(w.num_pages, w.num_layers, w.num_kv_heads, w.page_size, w.head_dim,
                              device)
    fill_random_(pool.k, gen)
    fill_random_(pool.v, gen)
    res = measure_decode(w, pool, list(range(w.num_layers)), args, device)
    res["access_pattern"] = slab_ceiling(w, pool, res["plan"], device, res["launch_ms"])
    plan = res["plan"]
    log(f"plan: {plan.num_items} work items x {w.num_qo_heads // plan.info.group_size} "
        f"head groups, part_tokens {plan.info.part_tokens}, {plan.info.num_merge} merged rows")
    log(f"decode: {res['ms_per_step']:.3f} ms/step, {res['value']:.1f} GB/s whole-step; "
        f"per launch {res['launch_ms'] * 1e3:.1f} us = {res['achieved']:.1f} GB/s "
        f"({res['achieved'] / HBM_PEAK_GBS * 100:.1f}% of HBM peak)")
    return res


def slab_ceiling(w, pool, plan, device, launch_ms, reps=5):
    """The decode's own access pattern, timed alone: kunserve_decode_slab_probe
    reads every K/V slab (one page's tokens of one KV head) the launch reads,
    in the partition kernel's workgroup shape, with the offsets precomputed
    and no arithmetic, over the same layers. A launch near this time is
    bound by how its slabs are served, not by its lookups or arithmetic."""
    from kunserve_amd import _lib

    indptr, indices = w.csr()
    rec = plan.plan_host[: 4 * plan.info.num_work].reshape(-1, 4)   # padding: seq -1
    shift = int(w.page_size).bit_length() - 1
    max_slabs = max(1, plan.info.part_tokens // w.page_size + 1)
    es = pool.k.element_size()
    base = np.zeros((len(rec), max_slabs), dtype=np.int64)
    counts = np.zeros(len(rec), dtype=np.int32)
    for i, (seq, tb, te, _) in enumerate(rec):
        if seq >= 0 and te > tb:
            pages = indices[indptr[seq] + (tb >> shift): indptr[seq] + ((te - 1) >> shift) + 1]
            base[i, : len(pages)] = pages.astype(np.int64) * pool.k.stride(0) * es
            counts[i] = len(pages)
    slab_bytes = w.page_size * w.head_dim * es
    offs = [torch.from_numpy(base + layer * pool.k.stride(1) * es).to(device)
            for layer in range(w.num_layers)]
    cnt = torch.from_numpy(counts).to(device)
    sink = torch.empty(len(rec) * w.num_kv_heads, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream

    def sweep():
        for o in offs:
            _lib.call("kunserve_decode_slab_probe", pool.k.data_ptr(), pool.v.data_ptr(),
                      o.data_ptr(), cnt.data_ptr(), len(rec), max_slabs,
                      pool.k.stride(2) * es, w.num_kv_heads, slab_bytes, sink.data_ptr(), stream)
    sweep()
    ms = region_ms(lambda: [sweep() for _ in range(reps)], device) / (reps * w.num_layers)
    nbytes = 2 * slab_bytes * int(counts.sum()) * w.num_kv_heads
    log(f"decode access pattern alone (slab probe): {ms * 1e3:.1f} us per layer = "
        f"{nbytes / (ms * 1e-3) / 1e9:.0f} GB/s over {nbytes / 1e6:.0f} MB of slabs; the decode "
        f"launch takes {launch_ms / ms:.3f}x that")
    return {"probe_us_per_layer": ms * 1e3, "slab_bytes_per_layer": nbytes,
            "probe_gbs": nbytes / (ms * 1e-3) / 1e9, "launch_over_probe": launch_ms / ms}


def bench_single_layer(args, device):
    """Single-layer decode (batch 8, 32/32 heads, contexts U[128, 512],
    tables from a permutation of a 512-page pool, Q/K/V ~ N(0,1)/sqrt(128)):
    the shape the reference's CPU path runs whole. Times many back-to-back
    launches (one launch moves about 34 MB, so launch overhead is a large
    share), checks the output against the numpy oracle, and times the
    PyTorch-CPU restatement of the whole layer and the one-thread numpy
    oracle beside it."""
    import copy

    import kunserve_amd as ks
    from kunserve_amd import workloads
    from oracle import paged_attention_ref as ref
    from oracle import torch_cpu
    from threadpoolctl import threadpool_limits

    w = workloads.single_layer_decode()
    scale = 1 / math.sqrt(w.head_dim)
    gen = torch.Generator(device=device)
    gen.manual_seed(w.seed)
    pool = ks.KVPool.allocate(w.num_pages, 1, w.num_kv_heads, w.page_size, w.head_dim, device)
    for t in (pool.k, pool.v):
        t.copy_(torch.randn(t.shape, generator=gen, device=device) * scale)
    a = copy.copy(args)
    a.steps = max(args.steps, 200)
    res = measure_decode(w, pool, [0], a, device, q_scale=scale)
    indptr, indices = w.csr()
    q = res["qs"][0]
    out = ks.paged_decode(pool, 0, res["table"], q, res["plan"])
    kh, vh, qh = pool.k.cpu(), pool.v.cpu(), q.cpu()
    want = ref.decode_attention(qh.numpy(), kh.numpy(), vh.numpy(), 0, indptr, indices,
                                w.kv_len, scale)
    err = float(np.max(np.abs(out.float().cpu().numpy() - want)))
    log(f"single-layer decode: {w.name}: per launch {res['launch_ms'] * 1e3:.2f} us = "
        f"{res['achieved']:.1f} GB/s ({res['achieved'] / HBM_PEAK_GBS * 100:.1f}% of HBM peak); "
        f"max-abs vs the oracle {err:.2e}")
    if err > 2e-3:
        print(f"single-layer decode check failed: max-abs {err}", file=sys.stderr)
        sys.exit(1)
    cpu = None
    if not args.no_cpu_baseline:
        threads = cpu_threads()
        prev = torch.get_num_threads()
        torch.set_num_threads(threads)
        try:
            med, times = cpu_timed(lambda: torch_cpu.decode_attention(
                qh, kh, vh, 0, indptr, indices, w.kv_len, scale), args.cpu_budget / 8)
        finally:
            torch.set_num_threads(prev)
        with threadpool_limits(limits=1):
            np_med, _ = cpu_timed(lambda: ref.decode_attention(
                qh.numpy(), kh.numpy(), vh.numpy(), 0, indptr, indices, w.kv_len, scale,
                dtype=np.float32), 0.5)
        nb = res["bytes_per_layer"]
        cpu = {"value": nb / med / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"PyTorch-CPU restatement (oracle/torch_cpu.py), fp32 on fp16 pages, "
                         f"{threads} threads: the whole workload ({w.batch} rows, one layer, "
                         f"{nb / 1e6:.1f} MB); median of {len(times)} runs after one warm-up; "
                         f"{med * 1e3:.2f} ms per run",
               "runs_s": [round(t, 5) for t in times],
               "numpy_one_thread_gbs": nb / np_med / 1e9}
        log(f"single-layer decode cpu baseline: {cpu['value']:.3f} GB/s ({cpu['sample']})")
    return {"workload": w.name, "launch_us": res["launch_ms"] * 1e3, "gbs": res["achieved"],
            "hbm_frac": res["achieved"] / HBM_PEAK_GBS, "bytes_per_launch": res["bytes_per_layer"],
            "launches_timed": a.steps, "max_abs_vs_oracle": err, "cpu_baseline": cpu}


def bench_mixed(args, device, layers=4):
    """One pforward attention step that mixes the chunked-prefill workload's
    first step (16 chunks of up to 512 tokens on prefixes U[0, 2048]) with
    the Llama-2-7B decode workload's 64 decode rows, as the reference's
    scheduler batches running decodes with prefill chunks
    (kunserve/flash_backend.py:1870-1950; row arguments of
    kunserve/request.py:654-670). AttentionStep runs it per layer: append,
    then decode and chunked-prefill attention, each reading q and writing
    out in place through its row -> token map. Timed per layer against the
    same two row sets run as steps of their own, with and without the
    append."""
    import kunserve_amd as ks
    from kunserve_amd import workloads

    pw, dw = workloads.chunked_prefill(), workloads.llama2_7b_decode()
    rows, ql, kv = pw.steps()[0]
    ps, half = pw.page_size, pw.num_pages
    rng = np.random.default_rng(1006)
    # prefill rows keep their pages in [0, 8192); decode rows get disjoint ones above
    dec_pages = [half + p for p in workloads._tables(rng, dw.kv_len, ps, half)]
    pool = ks.KVPool.allocate(2 * half, layers, pw.num_kv_heads, ps, pw.head_dim, device)
    gen = torch.Generator(device=device)
    gen.manual_seed(1006)
    fill_random_(pool.k, gen)
    fill_random_(pool.v, gen)
    need = (kv + ps - 1) // ps
    pre = dict(q_lens=ql.tolist(), first=(kv - ql).tolist(), flags=[1] * len(rows),
               pages=[pw.pages[r][:n].tolist() for r, n in zip(rows, need)])
    dec = dict(q_lens=[1] * dw.batch, first=dw.kv_len.tolist(), flags=[0] * dw.batch,
               pages=[p.tolist() for p in dec_pages])
    mixed = {k: dec[k] + pre[k] for k in dec}
    hq, hkv, d = pw.num_qo_heads, pw.num_kv_heads, pw.head_dim

    def make(spec):
        step = ks.AttentionStep(pool, hq, spec["q_lens"], spec["first"], spec["flags"],
                                spec["pages"])
        T = step.num_tokens
        t = [torch.randn((T, h, d), generator=gen, device=device).half() for h in (hq, hkv, hkv)]
        return step, t, torch.empty_like(t[0])

    def attention(step, q, out, layer):
        # AttentionStep.run without its append
        if step.decode is not None:
            sd = step.decode
            ks.paged_decode(pool, layer, sd.table, q, sd.plan, step.scale, out=out,
                            workspace=step.workspace, q_token=sd.tokens)
        if step.prefill is not None:
            sp = step.prefill
            ks.paged_prefill(pool, layer, sp.table, sp.q_indptr, q, sp.plan, step.scale,
                             out=out, workspace=step.workspace, q_start=sp.tokens)

    # The three steps are timed in alternation, one pass over the layers
    # each, and the medians reported: prefill attention runs at the part's
    # power limit, and its clock drifts over a run by several percent.
    built = {name: make(spec) for name, spec in (("mixed", mixed), ("decode", dec),
                                                   ("prefill", pre))}
    full = {n: (lambda st=st, t=t, o=o: [st.run(l, *t, out=o) for l in range(layers)])
            for n, (st, t, o) in built.items()}
    attn = {n: (lambda st=st, t=t, o=o: [attention(st, t[0], o, l) for l in range(layers)])
            for n, (st, t, o) in built.items()}
    for n in built:
        full[n]()
    torch.cuda.synchronize()
    samples = {n: {"full": [], "attn": []} for n in built}
    for _ in range(max(5, args.steps // 2)):
        for n in built:
            samples[n]["full"].append(region_ms(full[n], device) / layers)
            samples[n]["attn"].append(region_ms(attn[n], device) / layers)
    res = {n: {"tokens": built[n][0].num_tokens,
               "ms_per_layer": float(np.median(samples[n]["full"])),
               "attention_ms_per_layer": float(np.median(samples[n]["attn"])),
               "passes": len(samples[n]["attn"])} for n in built}
    del built, full, attn
    sep = res["decode"]["attention_ms_per_layer"] + res["prefill"]["attention_ms_per_layer"]
    sep_full = res["decode"]["ms_per_layer"] + res["prefill"]["ms_per_layer"]
    out = {"workload": f"{pw.name} first step (16 chunks) + {dw.name.split(' x')[0]} "
                       f"(64 decode rows), one step, {layers} layers",
           "layers": layers, "steps": res,
           "attention_ratio_vs_separate": res["mixed"]["attention_ms_per_layer"] / sep,
           "ratio_vs_separate_with_append": res["mixed"]["ms_per_layer"] / sep_full}
    log(f"mixed step: attention {res['mixed']['attention_ms_per_layer'] * 1e3:.1f} us/layer "
        f"against decode {res['decode']['attention_ms_per_layer'] * 1e3:.1f} + prefill "
        f"{res['prefill']['attention_ms_per_layer'] * 1e3:.1f} us/layer run apart "
        f"(ratio {out['attention_ratio_vs_separate']:.3f}); with append "
        f"{res['mixed']['ms_per_layer'] * 1e3:.1f} us/layer (ratio "
        f"{out['ratio_vs_separate_with_append']:.3f})")
    del pool
    return out


def bench_gqa(args, device):
    """Llama-3-8B GQA decode (32 Q / 8 KV heads, batch 128, contexts
    U[1024, 8192]), one layer per launch."""
    import kunserve_amd as ks
    from kunserve_amd import workloads

    w = workloads.llama3_8b_gqa_decode()
    gen = torch.Generator(device=device)
    gen.manual_seed(w.seed)
    pool = ks.KVPool.allocate(w.num_pages, 1, w.num_kv_heads, w.page_size, w.head_dim, device)
    fill_random_(pool.k, gen)
    fill_random_(pool.v, gen)
    res = measure_decode(w, pool, [0], args, device)
    log(f"gqa decode: {w.name}: per launch {res['launch_ms'] * 1e3:.1f} us = "
        f"{res['achieved']:.1f} GB/s ({res['achieved'] / HBM_PEAK_GBS * 100:.1f}% of HBM peak), "
        f"part_tokens {res['plan'].info.part_tokens}, group {res['plan'].info.group_size}")
    pattern = slab_ceiling(w, pool, res["plan"], device, res["launch_ms"], reps=20)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_decode_sample(w, pool, 0, res["qs"][0], np.arange(0, w.batch, 8),
                                args.cpu_budget / 4)
        log(f"gqa decode cpu baseline: {cpu['value']:.3f} GB/s ({cpu['sample']})")
    return {"workload": w.name, "launch_us": res["launch_ms"] * 1e3, "gbs": res["achieved"],
            "hbm_frac": res["achieved"] / HBM_PEAK_GBS, "bytes_per_launch": res["bytes_per_layer"],
            "access_pattern": pattern, "cpu_baseline": cpu}


def bench_bf16_decode(args, device, page_size=16):
    """The Llama-2-7B decode workload on a bf16 pool (the reference's default
    --dtype), 4 layers of the pool swept one launch per layer; page_size 256
    is the reference's default block size as well."""
    import kunserve_amd as ks
    from kunserve_amd import workloads

    w = workloads.llama2_7b_decode(page_size=page_size)
    gen = torch.Generator(device=device)
    gen.manual_seed(w.seed)
    layers = 4
    pool = ks.KVPool.allocate(w.num_pages, layers, w.num_kv_heads, w.page_size, w.head_dim,
                              device, dtype=torch.bfloat16)
    fill_random_(pool.k, gen)
    fill_random_(pool.v, gen)
    res = measure_decode(w, pool, list(range(layers)), args, device)
    log(f"bf16 decode: {w.name} on a {layers}-layer bf16 pool: per launch "
        f"{res['launch_ms'] * 1e3:.1f} us = {res['achieved']:.1f} GB/s "
        f"({res['achieved'] / HBM_PEAK_GBS * 100:.1f}% of HBM peak)")
    out = {"workload": w.name + " (bf16 pool, 4 layers)", "launch_us": res["launch_ms"] * 1e3,
           "gbs": res["achieved"], "hbm_frac": res["achieved"] / HBM_PEAK_GBS}
    del pool, res
    return out


def bench_remap(args, device):
    """Block remap under memory pressure: 8192 random 2 MiB blocks (32
    layers x 8 heads x 16 x 128, K+V) copied between disjoint pool regions,
    then a Llama-2-70B layer decode (64 Q / 8 KV heads, batch 256) on tables
    that point at the copies; its output must equal, bit for bit, the
    decode on the original tables."""
    import kunserve_amd as ks
    from kunserve_amd import workloads

    r = workloads.kv_remap()
    gen = torch.Generator(device=device)
    gen.manual_seed(r.seed)
    pool = ks.KVPool.allocate(r.num_pages, r.num_layers, r.num_kv_heads, r.page_size,
                              r.head_dim, device)
    reps = max(2, args.steps // 4)
    ceiling = copy_ceiling(pool, r, reps, device)
    fill_random_(pool.k, gen)
    fill_random_(pool.v, gen)
    src = torch.from_numpy(r.src).to(device)
    dst = torch.from_numpy(r.dst).to(device)
    ks.copy_blocks(pool, src, dst)
    torch.cuda.synchronize()
    copy_ms = region_ms(lambda: [ks.copy_blocks(pool, src, dst) for _ in range(reps)],
                        device) / reps
    copy_gbs = r.copy_bytes() / (copy_ms * 1e-3) / 1e9
    log(f"block copy: {len(r.src)} blocks of {r.copy_bytes() / 4 / len(r.src) / 2**20:.0f} MiB "
        f"(K and V), {copy_ms:.3f} ms = {copy_gbs:.1f} GB/s "
        f"({copy_gbs / HBM_PEAK_GBS * 100:.1f}% of HBM peak)")
    w, w2 = r.decode, r.decode_remapped
    dec = measure_decode(w2, pool, [0], args, device)
    out_remapped = ks.paged_decode(pool, 0, dec["table"], dec["qs"][0], dec["plan"])
    indptr, indices = w.csr()
    table0 = ks.PageTable(indptr, indices, w.kv_len, device)
    out_orig = ks.paged_decode(pool, 0, table0, dec["qs"][0], dec["plan"])
    torch.cuda.synchronize()
    same = bool(torch.equal(out_orig.view(torch.int16), out_remapped.view(torch.int16)))
    log(f"70b decode on remapped tables: per launch {dec['launch_ms'] * 1e3:.1f} us = "
        f"{dec['achieved']:.1f} GB/s ({dec['achieved'] / HBM_PEAK_GBS * 100:.1f}% of HBM peak); "
        f"bit-exact vs original tables: {same}")
    if not same:
        print("remapped decode differs from the original tables", file=sys.stderr)
        sys.exit(1)
    cpu_copy = cpu_dec = None
    if not args.no_cpu_baseline:
        cpu_dec = cpu_decode_sample(w2, pool, 0, dec["qs"][0], np.arange(0, w2.batch, 16),
                                    args.cpu_budget / 4)
        log(f"70b decode cpu baseline: {cpu_dec['value']:.3f} GB/s ({cpu_dec['sample']})")
        cpu_copy = cpu_copy_sample(r, args.cpu_budget / 4)
        log(f"block copy cpu baseline: {cpu_copy['value']:.3f} GB/s ({cpu_copy['sample']})")
    return {"copy": {"workload": f"remap copy {len(r.src)} blocks x 2 MiB (K+V)",
                     "ms": copy_ms, "gbs": copy_gbs, "hbm_frac": copy_gbs / HBM_PEAK_GBS,
                     "frac_of_best_ceiling_copy": copy_gbs / max(
                         ceiling["copy_gbs"], ceiling["memcpy_d2d_gbs"]),
                     "cpu_baseline": cpu_copy},
            "copy_ceiling": ceiling,
            "decode": {"workload": w.name, "launch_us": dec["launch_ms"] * 1e3,
                       "gbs": dec["achieved"], "hbm_frac": dec["achieved"] / HBM_PEAK_GBS,
                       "bit_exact_vs_original_tables": same, "cpu_baseline": cpu_dec}}


def cpu_copy_sample(r, budget_s: float, n: int = 256) -> dict:
    """The PyTorch-CPU restatement of the remap copy (oracle/torch_cpu.py
    copy_blocks: index_select then index_copy_ of whole blocks) on host
    pools of 2n blocks of the remap shape: n random blocks of the first half
    copied into a random permutation of the second half."""
    from oracle import torch_cpu

    shape = (2 * n, r.num_layers, r.num_kv_heads, r.page_size, r.head_dim)
    k = torch.randn(shape, dtype=torch.float32).half()
    v = torch.randn(shape, dtype=torch.float32).half()
    rng = np.random.default_rng(r.seed)
    src, dst = rng.permutation(n), n + rng.permutation(n)
    nbytes = 2 * 2 * n * k[0].numel() * 2
    threads = cpu_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        med, times = cpu_timed(lambda: torch_cpu.copy_blocks(k, v, src, dst), budget_s)
    finally:
        torch.set_num_threads(prev)
    return {"value": nbytes / med / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"PyTorch-CPU restatement (oracle/torch_cpu.py copy_blocks), {threads} "
                      f"threads: {n} random blocks of 2 MiB (K+V) between the halves of a "
                      f"{2 * n}-block host pool, {nbytes / 2**30:.1f} GiB read + written; median "
                      f"of {len(times)} runs after one warm-up; {med * 1e3:.1f} ms per run",
            "runs_s": [round(t, 4) for t in times]}


def copy_ceiling(pool, r, reps, device):
    """What this part's HBM gives the access mixes of a copy, over the bytes
    of the remap copy: read-only and write-only streams of 32 GiB (the K and
    V pools' first 2 x 8192 blocks), a plain copy and hipMemcpyAsync of the
    first 8192 blocks of K and V into the next 8192 (16 GiB read + 16 GiB
    written, as the remap copy). kunserve_hbm_probe has the block copy's
    launch shape; the memcpy goes through torch's copy_ of contiguous
    same-device tensors, which is one hipMemcpyAsync. Leaves the
    pool's bytes overwritten: run it before the pool is filled."""
    from kunserve_amd import _lib

    n = len(r.src)
    halves = []
    for t in (pool.k, pool.v):
        flat = t.view(torch.uint8).reshape(t.shape[0], -1)
        halves.append((flat[:n], flat[n:2 * n]))
    nbytes = halves[0][0].numel()                 # one half of one pool
    sink = torch.empty(16, dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream

    def probe(mode):
        for a, b in halves:
            if mode == 0:
                for part in (a, b):
                    _lib.call("kunserve_hbm_probe", 0, part.data_ptr(), sink.data_ptr(), nbytes,
                              stream)
            elif mode == 1:
                for part in (a, b):
                    _lib.call("kunserve_hbm_probe", 1, None, part.data_ptr(), nbytes, stream)
            else:
                _lib.call("kunserve_hbm_probe", 2, a.data_ptr(), b.data_ptr(), nbytes, stream)

    def memcpy():
        for a, b in halves:
            b.copy_(a)

    total = 4 * nbytes                            # bytes each measurement moves
    out = {"bytes": total}
    for name, fn in (("read", lambda: probe(0)), ("write", lambda: probe(1)),
                     ("copy", lambda: probe(2)), ("memcpy_d2d", memcpy)):
        fn()
        torch.cuda.synchronize()
        ms = region_ms(lambda: [fn() for _ in range(reps)], device) / reps
        out[name + "_gbs"] = total / (ms * 1e-3) / 1e9
    log("copy ceiling over 32 GiB: read-only {read_gbs:.0f}, write-only {write_gbs:.0f}, "
        "plain copy {copy_gbs:.0f}, hipMemcpyAsync D2D {memcpy_d2d_gbs:.0f} GB/s".format(**out))
    return out


# Llama-2-7B layer weights: q/k/v/o 4 x 4096^2, gate/up/down 3 x 4096 x 11008,
# two RMSNorm vectors, fp16.
LLAMA2_7B_LAYER_BYTES = 2 * (4 * 4096 * 4096 + 3 * 4096 * 11008 + 2 * 4096)


def bench_pmm(args, device):
    """The Llama-2-7B decode workload on a pool that pmm_drop grew: the last
    pages of the 16384-page pool come from 16 dropped Llama-2-7B layers
    (49 pages each), so tables address base and extend pages alike. Times
    drop and restore per layer and the decode sweep over the grown pool."""
    import kunserve_amd as ks
    from kunserve_amd import workloads

    w = workloads.llama2_7b_decode()
    page_bytes = w.num_layers * w.num_kv_heads * w.page_size * w.head_dim * 2
    per_layer = -(-LLAMA2_7B_LAYER_BYTES // (2 * page_bytes))
    dropped_layers = 16
    extend = per_layer * dropped_layers
    pm = ks.PmmPool(w.num_pages - extend, w.num_layers, w.num_kv_heads, w.page_size,
                    w.head_dim, extend, device)
    try:
        segs = [pm.add_segment(LLAMA2_7B_LAYER_BYTES) for _ in range(dropped_layers)]
        drop_ms = []
        for sid in segs:
            t0 = time.perf_counter()
            pm.drop(sid)
            drop_ms.append((time.perf_counter() - t0) * 1e3)
        assert pm.num_pages == w.num_pages
        gen = torch.Generator(device=device)
        gen.manual_seed(w.seed)
        fill_random_(pm.pool.k, gen)
        fill_random_(pm.pool.v, gen)
        res = measure_decode(w, pm.pool, list(range(w.num_layers)), args, device)
        err = check_decode(res, device)
        indptr, indices = w.csr()
        on_extend = int((indices >= w.num_pages - extend).sum())
        del res["pool"], res["qs"], res["table"]
        torch.cuda.synchronize()
        restore_ms = []
        for _ in segs:
            t0 = time.perf_counter()
            pm.restore()
            restore_ms.append((time.perf_counter() - t0) * 1e3)
    finally:
        pm.close()
    log(f"pmm: {dropped_layers} Llama-2-7B layers dropped into {extend} extend pages; drop "
        f"{np.mean(drop_ms):.2f} ms/layer, restore {np.mean(restore_ms):.2f} ms/layer; decode "
        f"over the grown pool ({on_extend} of {len(indices)} table pages on extend pages): "
        f"per launch {res['launch_ms'] * 1e3:.1f} us = {res['achieved']:.1f} GB/s "
        f"({res['achieved'] / HBM_PEAK_GBS * 100:.1f}% of HBM peak), max-abs {err:.1e}")
    if err > 2e-3:
        print(f"decode on the grown pool failed its check: max-abs {err}", file=sys.stderr)
        sys.exit(1)
    return {"workload": f"{w.name} on a pool grown by {dropped_layers} dropped Llama-2-7B layers",
            "extend_pages": extend, "table_pages_on_extend": on_extend,
            "drop_ms_per_layer": float(np.mean(drop_ms)),
            "restore_ms_per_layer": float(np.mean(restore_ms)),
            "decode_launch_us": res["launch_ms"] * 1e3, "decode_gbs": res["achieved"],
            "hbm_frac": res["achieved"] / HBM_PEAK_GBS, "decode_max_abs": err}


def check_decode(res, device, layers=(0, 31)) -> float:
    """Max-abs error of every row of two layers of the measured decode
    against softmax(q K^T / sqrt(D)) V computed in fp32 with plain torch ops
    on the device (gather through the page table, then bmm and softmax)."""
    import kunserve_amd as ks

    w, pool = res["workload"], res["pool"]
    indptr, indices = w.csr()
    idx = torch.from_numpy(indices.astype(np.int64)).to(device)
    hkv, ps, d = w.num_kv_heads, w.page_size, w.head_dim
    g = w.num_qo_heads // hkv
    worst = 0.0
    for layer in layers:
        q = res["qs"][layer]
        out = ks.paged_decode(pool, layer, res["table"], q, res["plan"]).float()
        for b in range(w.batch):
            n = int(w.kv_len[b])
            pages = idx[int(indptr[b]):int(indptr[b]) + (n + ps - 1) // ps]
            k = pool.k[pages, layer].float().transpose(0, 1).reshape(hkv, -1, d)[:, :n]
            v = pool.v[pages, layer].float().transpose(0, 1).reshape(hkv, -1, d)[:, :n]
            s = torch.bmm(q[b].float().reshape(hkv, g, d), k.transpose(1, 2).contiguous())
            p = torch.softmax(s / math.sqrt(d), dim=-1)
            want = torch.bmm(p, v.contiguous()).reshape(-1, d)
            worst = max(worst, float((out[b] - want).abs().max()))
    return worst


def _layer_pages_on_host(res, layer, used):
    pool = res["pool"]
    sel = torch.from_numpy(used.astype(np.int64)).to(pool.device)
    k = pool.k[:, layer].index_select(0, sel)[:, None].cpu()
    v = pool.v[:, layer].index_select(0, sel)[:, None].cpu()
    return k, v


def cpu_threads() -> int:
    """Threads of the CPU baseline: the process's CPU share (OMP_NUM_THREADS,
    which the GPU host sets to the cores one GPU's jobs get), else every
    core os.cpu_count() reports."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    return int(env) if env.isdigit() and int(env) > 0 else (os.cpu_count() or 1)


def cpu_baseline(res, budget_s: float) -> dict:
    """The decode workload's PyTorch-CPU restatement (oracle.torch_cpu: fp32
    compute on fp16 pages, torch intra-op threads on the host cores), one
    whole layer (all rows) per run: one warm-up run, then at least 3 timed
    runs on further layers until budget_s has passed; the value is the
    median. The single-thread numpy oracle over one layer is reported
    beside it."""
    from threadpoolctl import threadpool_limits

    from oracle import paged_attention_ref as ref
    from oracle import torch_cpu

    w = res["workload"]
    indptr, indices = w.csr()
    used = np.unique(indices)
    remap = np.zeros(w.num_pages, dtype=np.int64)
    remap[used] = np.arange(used.size)
    local = remap[indices]
    scale = 1 / math.sqrt(w.head_dim)
    threads = cpu_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    times = []
    try:
        for layer in range(w.num_layers):
            k, v = _layer_pages_on_host(res, layer, used)
            q = res["qs"][layer].cpu()
            t0 = time.perf_counter()
            torch_cpu.decode_attention(q, k, v, 0, indptr, local, w.kv_len, scale)
            dt = time.perf_counter() - t0
            if layer > 0:                 # layer 0 is the warm-up
                times.append(dt)
            if len(times) >= 3 and sum(times) >= budget_s:
                break
    finally:
        torch.set_num_threads(prev)
    median = float(np.median(times))
    # numpy oracle, one thread, one layer
    k, v = _layer_pages_on_host(res, 0, used)
    with threadpool_limits(limits=1):
        t0 = time.perf_counter()
        ref.decode_attention(res["qs"][0].cpu().numpy(), k.numpy(), v.numpy(), 0, indptr, local,
                             w.kv_len, scale, dtype=np.float32)
        np_s = time.perf_counter() - t0
    return {"value": res["bytes_per_layer"] / median / 1e9, "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"PyTorch-CPU restatement (oracle/torch_cpu.py), fp32 on fp16 pages, "
                      f"{threads} threads (host reports {os.cpu_count()} cores): median of "
                      f"{len(times)} runs, each one whole layer of the same decode workload "
                      f"(all {w.batch} rows, {res['bytes_per_layer'] / 1e9:.3f} GB), after one "
                      f"warm-up layer; {median:.2f} s per layer",
            "runs_s": [round(t, 3) for t in times],
            "numpy_one_thread_gbs": res["bytes_per_layer"] / np_s / 1e9}


def cpu_timed(fn, budget_s: float, min_runs: int = 3, max_runs: int = 50):
    """One warm-up call of fn, then timed calls until at least min_runs ran
    and budget_s passed (at most max_runs). Returns (median s, runs)."""
    fn()
    times = []
    while len(times) < min_runs or (sum(times) < budget_s and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), times


def cpu_decode_sample(w, pool, layer, q, rows, budget_s: float) -> dict:
    """The PyTorch-CPU restatement (oracle/torch_cpu.py) of decode workload
    w on the given rows of one layer: their pages are copied to the host,
    then the restatement runs on all host threads. The rate is the sampled
    rows' algorithmic bytes (K and V of their tokens once per KV head, q,
    out and page ids) over the median run."""
    from oracle import torch_cpu

    rows = np.asarray(rows)
    indptr, indices = w.csr()
    lo, hi = indptr[rows], indptr[rows + 1]
    sub_indptr = np.concatenate([[0], np.cumsum(hi - lo)]).astype(np.int32)
    ids = np.concatenate([indices[a:b] for a, b in zip(lo, hi)]).astype(np.int64)
    sel = torch.from_numpy(ids).to(pool.device)
    k = pool.k[:, layer].index_select(0, sel)[:, None].cpu()
    v = pool.v[:, layer].index_select(0, sel)[:, None].cpu()
    qh = q[torch.from_numpy(rows.astype(np.int64)).to(q.device)].cpu()
    kv = w.kv_len[rows]
    local = np.arange(ids.size, dtype=np.int32)
    nbytes = (int(kv.astype(np.int64).sum()) * w.num_kv_heads * w.head_dim * 4
              + 2 * rows.size * w.num_qo_heads * w.head_dim * 2 + ids.size * 4)
    threads = cpu_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        med, times = cpu_timed(lambda: torch_cpu.decode_attention(
            qh, k, v, 0, sub_indptr, local, kv, 1 / math.sqrt(w.head_dim)), budget_s)
    finally:
        torch.set_num_threads(prev)
    return {"value": nbytes / med / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"PyTorch-CPU restatement (oracle/torch_cpu.py), fp32 on fp16 pages, "
                      f"{threads} threads: {rows.size} of the workload's {w.batch} rows (every "
                      f"{max(1, w.batch // rows.size)}th), one layer, {nbytes / 1e9:.3f} GB; median "
                      f"of {len(times)} runs after one warm-up; {med * 1e3:.1f} ms per run",
            "runs_s": [round(t, 4) for t in times]}


# ----------------------------------------------------------------- prefill


def bench_prefill(args, device, page_size=16, dtype=torch.float16, head_dim=None,
                  num_kv_heads=None):
    """The chunked-prefill workload's 8 steps. head_dim (64 or 256) runs the
    same rows, pages and heads at another head size, and num_kv_heads (8:
    Llama-3-8B's 32 query / 8 KV heads) the same rows with grouped KV
    heads: attention only."""
    import dataclasses

    import kunserve_amd as ks
    from kunserve_amd import workloads

    w = workloads.chunked_prefill(page_size=page_size)
    full = head_dim is None and num_kv_heads is None
    if head_dim is not None:
        w = dataclasses.replace(w, head_dim=head_dim, name=f"{w.name} head_dim{head_dim}")
    if num_kv_heads is not None:
        w = dataclasses.replace(w, num_kv_heads=num_kv_heads,
                                name=f"{w.name} {w.num_qo_heads}q/{num_kv_heads}kv heads")
    gen = torch.Generator(device=device)
    gen.manual_seed(w.seed)
    pool = ks.KVPool.allocate(w.num_pages, 1, w.num_kv_heads, w.page_size, w.head_dim, device,
                              dtype=dtype)
    fill_random_(pool.k, gen)
    fill_random_(pool.v, gen)
    steps = []
    for rows, ql, kv in w.steps():
        need = (kv + w.page_size - 1) // w.page_size
        indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
        indices = np.concatenate([w.pages[r][:n] for r, n in zip(rows, need)]).astype(np.int32)
        q_indptr = np.concatenate([[0], np.cumsum(ql)]).astype(np.int32)
        T = int(q_indptr[-1])
        table = ks.PageTable(indptr, indices, kv, device)
        qi = torch.from_numpy(q_indptr).to(device)
        plan = ks.PrefillPlan(q_indptr, kv, w.num_qo_heads, w.num_kv_heads, device,
                              head_dim=w.head_dim)
        mk = lambda h: torch.randn((T, h, w.head_dim), generator=gen, device=device).to(dtype)
        steps.append((table, qi, plan, mk(w.num_qo_heads), mk(w.num_kv_heads),
                      mk(w.num_kv_heads), torch.empty((T, w.num_qo_heads, w.head_dim),
                                                      dtype=dtype, device=device)))

    def run(timer=None):
        for table, qi, plan, q, k, v, out in steps:
            ks.append_kv(pool, 0, table, qi, k, v)
            s = timer.start() if timer else None
            ks.paged_prefill(pool, 0, table, qi, q, plan, out=out)
            if timer:
                timer.stop(s)

    # The fused RoPE + append prologue over the same steps: HBM-bound, bytes =
    # q read and written, k and v read, rotated k and v written.
    inv_freq = ks.rope_inv_freq(w.head_dim, 10000.0, device)
    rope_bytes = 0
    for table, qi, plan, q, k, v, out in steps:
        T = q.shape[0]
        rope_bytes += 2 * T * w.num_qo_heads * w.head_dim * 2 + 4 * T * w.num_kv_heads * w.head_dim * 2

    def run_rope():
        for table, qi, plan, q, k, v, out in steps:
            ks.rope_append_kv(pool, 0, table, qi, q, k, v, inv_freq)

    # The append alone over the same steps: k and v read, then written.
    append_bytes = sum(4 * q.shape[0] * w.num_kv_heads * w.head_dim * 2
                       for table, qi, plan, q, k, v, out in steps)

    def run_append():
        for table, qi, plan, q, k, v, out in steps:
            ks.append_kv(pool, 0, table, qi, k, v)

    rope = append = None
    if page_size == 16 and dtype == torch.float16 and full:
        run_rope()
        run_append()
        reps_bw = 8
        rope_ms = region_ms(lambda: [run_rope() for _ in range(reps_bw)], device) / reps_bw
        append_ms = region_ms(lambda: [run_append() for _ in range(reps_bw)], device) / reps_bw
        gbs = lambda b, ms: b / (ms * 1e-3) / 1e9
        # Reference for launches of this size: a plain device copy of each
        # step's k and v (the same bytes read and written, one launch per
        # step and tensor, torch's copy kernel).
        dsts = [(torch.empty_like(k), torch.empty_like(v)) for _, _, _, _, k, v, _ in steps]

        def run_copy():
            for (table, qi, plan, q, k, v, out), (dk, dv) in zip(steps, dsts):
                dk.copy_(k)
                dv.copy_(v)
        run_copy()
        copy_ms = region_ms(lambda: [run_copy() for _ in range(reps_bw)], device) / reps_bw
        del dsts
        # And this library's copy kernel (the block copy's launch shape), one
        # launch per step over the step's k and v bytes (rounded down to the
        # kernel's 256 KiB unit), as the append.
        from kunserve_amd import _lib
        step_bytes = [(2 * k.numel() * k.element_size()) // 262144 * 262144
                      for _, _, _, _, k, v, _ in steps]
        lib_bytes = 2 * sum(step_bytes)           # read and written
        src = torch.empty(max(step_bytes), dtype=torch.uint8, device=device)
        dst = torch.empty_like(src)
        stream = torch.cuda.current_stream(device).cuda_stream

        def run_lib_copy():
            for nb in step_bytes:
                _lib.call("kunserve_hbm_probe", 2, src.data_ptr(), dst.data_ptr(), nb, stream)
        run_lib_copy()
        lib_copy_ms = region_ms(lambda: [run_lib_copy() for _ in range(reps_bw)], device) / reps_bw
        del src, dst
        log(f"rope + append prologue: {rope_ms:.3f} ms for the 8 steps = "
            f"{gbs(rope_bytes, rope_ms):.1f} GB/s; append alone {append_ms:.3f} ms = "
            f"{gbs(append_bytes, append_ms):.1f} GB/s; a plain copy of the steps' k and v "
            f"{copy_ms:.3f} ms = {gbs(append_bytes, copy_ms):.1f} GB/s (torch), "
            f"{lib_copy_ms:.3f} ms = {gbs(lib_bytes, lib_copy_ms):.1f} GB/s (this library's copy "
            f"kernel, one launch per step)")
        rope = {"ms": rope_ms, "bytes": rope_bytes, "gbs": gbs(rope_bytes, rope_ms),
                "hbm_frac": gbs(rope_bytes, rope_ms) / HBM_PEAK_GBS,
                "launches": len(steps) * reps_bw}
        append = {"ms": append_ms, "bytes": append_bytes, "gbs": gbs(append_bytes, append_ms),
                  "hbm_frac": gbs(append_bytes, append_ms) / HBM_PEAK_GBS,
                  "launches": len(steps) * reps_bw,
                  "plain_copy_same_bytes_gbs": gbs(append_bytes, copy_ms),
                  "frac_of_plain_copy": copy_ms / append_ms,
                  "library_copy_same_bytes_gbs": gbs(lib_bytes, lib_copy_ms),
                  "frac_of_library_copy": gbs(append_bytes, append_ms) / gbs(lib_bytes, lib_copy_ms)}

    reps = max(1, args.steps // 4)
    for _ in range(max(1, args.warmup)):
        run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        run()
    torch.cuda.synchronize()
    elapsed = (time.perf_counter() - t0) / reps

    def run_attention():
        for table, qi, plan, q, k, v, out in steps:
            ks.paged_prefill(pool, 0, table, qi, q, plan, out=out)

    # Attention alone (the steps' K/V are in the pages from the runs above).
    attn_ms = region_ms(lambda: [run_attention() for _ in range(reps)], device) / reps
    power = None
    if full and page_size == 16 and dtype == torch.float16:
        power = power_during(run_attention, device)
        if power:
            log(f"prefill attention back to back: socket power {power['socket_power_w'][1]:.0f} W "
                f"(median of {power['samples']} samples), GFX clock {power['gfx_clock_mhz'][1]:.0f} MHz")
    timer = LaunchTimer()   # per-step breakdown (these events add about 5 us a step)
    run(timer)
    torch.cuda.synchronize()
    per_step = [a.elapsed_time(b) for a, b in timer.pairs]
    log("prefill per-step attention ms: " + ", ".join(f"{t:.3f}" for t in per_step))
    flops = w.causal_flops()
    tflops = flops / (attn_ms * 1e-3) / 1e12
    name = "fp16" if dtype == torch.float16 else "bf16"
    # Algorithmic bytes of the pass: each step reads every row's K and V
    # once per KV head, its q and its page ids, and writes its out. Against
    # them, the arithmetic intensity and the roofline time (the larger of
    # the MFMA-bound and HBM-bound times at the peaks).
    elem = 2
    nbytes = 0
    for rows, ql, kv in w.steps():
        T = int(ql.sum())
        nbytes += int(kv.sum()) * w.num_kv_heads * w.head_dim * 2 * elem
        nbytes += 2 * T * w.num_qo_heads * w.head_dim * elem
        nbytes += int(((kv + w.page_size - 1) // w.page_size).sum()) * 4
    roof_ms = max(flops / (FP16_MFMA_PEAK_TFLOPS * 1e12), nbytes / (HBM_PEAK_GBS * 1e9)) * 1e3
    log(f"prefill ({name}, page {page_size}, head_dim {w.head_dim}, heads {w.num_qo_heads}/"
        f"{w.num_kv_heads}): {len(steps)} chunk steps, "
        f"{elapsed * 1e3:.3f} ms with "
        f"append; attention {attn_ms:.3f} ms = {tflops:.1f} TFLOP/s "
        f"({tflops / FP16_MFMA_PEAK_TFLOPS * 100:.1f}% of the {name} MFMA peak)")
    cpu = None
    if page_size == 16 and dtype == torch.float16 and full and not args.no_cpu_baseline:
        cpu = cpu_prefill_sample(w, pool, steps[0], args.cpu_budget / 4)
        log(f"prefill cpu baseline: {cpu['value']:.4f} TFLOP/s ({cpu['sample']})")
    log(f"prefill ({name}, page {page_size}): {nbytes / 1e9:.2f} GB algorithmic, "
        f"{flops / nbytes:.0f} flop/B against a ridge of "
        f"{FP16_MFMA_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9):.0f}; roofline time "
        f"{roof_ms:.3f} ms = {roof_ms / attn_ms * 100:.1f}% of the measured")
    return {"workload": w.name, "dtype": name, "head_dim": w.head_dim,
            "num_qo_heads": w.num_qo_heads, "num_kv_heads": w.num_kv_heads,
            "causal_tflop": flops / 1e12, "steps": len(steps),
            "ms_with_append": elapsed * 1e3, "attention_ms": attn_ms, "tflops": tflops,
            "mfma_util": tflops / FP16_MFMA_PEAK_TFLOPS, "page_size": page_size,
            "algorithmic_bytes": nbytes, "flop_per_byte": flops / nbytes,
            "roofline_ms": roof_ms, "roofline_frac": roof_ms / attn_ms, "power": power,
            "rope_append": rope,
            "append": append, "cpu_baseline": cpu}


def cpu_prefill_sample(w, pool, step, budget_s: float, every: int = 4) -> dict:
    """The PyTorch-CPU restatement (oracle/torch_cpu.py prefill_attention) of
    the chunked-prefill workload's first step on every `every`-th row: the
    rows' pages and q are copied to the host and the restatement runs on all
    host threads. The rate is the sampled rows' exact causal flops over the
    median run."""
    from oracle import torch_cpu

    rows0, ql0, kv0 = w.steps()[0]
    table, qi, plan, q, k, v, out = step
    sel_rows = np.arange(0, len(rows0), every)
    need = (kv0 + w.page_size - 1) // w.page_size
    ids = np.concatenate([w.pages[rows0[i]][:need[i]] for i in sel_rows]).astype(np.int64)
    sub_indptr = np.concatenate([[0], np.cumsum(need[sel_rows])]).astype(np.int32)
    q_indptr = np.concatenate([[0], np.cumsum(ql0)]).astype(np.int64)
    q_rows = np.concatenate([np.arange(q_indptr[i], q_indptr[i + 1]) for i in sel_rows])
    sub_qi = np.concatenate([[0], np.cumsum(ql0[sel_rows])]).astype(np.int32)
    sel = torch.from_numpy(ids).to(pool.device)
    kh = pool.k.index_select(0, sel).cpu()
    vh = pool.v.index_select(0, sel).cpu()
    qh = q[torch.from_numpy(q_rows).to(q.device)].cpu()
    kv = kv0[sel_rows]
    flops = 0
    for n_q, n_kv in zip(ql0[sel_rows].tolist(), kv.tolist()):
        flops += n_q * (n_kv - n_q) + n_q * (n_q + 1) // 2
    flops *= 4 * w.num_qo_heads * w.head_dim
    threads = cpu_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        med, times = cpu_timed(lambda: torch_cpu.prefill_attention(
            qh, sub_qi, kh, vh, 0, sub_indptr, np.arange(ids.size, dtype=np.int32), kv,
            1 / math.sqrt(w.head_dim)), budget_s)
    finally:
        torch.set_num_threads(prev)
    return {"value": flops / med / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"PyTorch-CPU restatement (oracle/torch_cpu.py), fp32 on fp16 pages, "
                      f"{threads} threads: {sel_rows.size} of the first step's {len(rows0)} rows "
                      f"(every {every}th; {int(ql0[sel_rows].sum())} q rows, "
                      f"{flops / 1e12:.4f} TFLOP exact causal); median of {len(times)} runs after "
                      f"one warm-up; {med * 1e3:.1f} ms per run",
            "runs_s": [round(t, 4) for t in times]}


def mfma_ceiling(device, settle_s=0.5, reps=64):
    """The rate this part sustains on the prefill kernels' 32x32x16 fp16
    MFMA (kunserve_mfma_probe: two waves per SIMD of independent MFMAs on
    every CU), with random N(0,1) operands and with constant ones. The
    operands' bits set the power the matrix cores draw and so the clock the
    part holds under its power limit; random operands draw what attention
    operands draw. Each variant first runs for settle_s so that the clock
    settles, then reps launches are timed."""
    from kunserve_amd import _lib

    wg = torch.cuda.get_device_properties(device).multi_processor_count
    n = wg * 512 * 16
    gen = torch.Generator(device=device)
    gen.manual_seed(1008)
    operands = {"constant": torch.full((n,), 0.01, dtype=torch.float16, device=device),
                "random": torch.randn(n, generator=gen, device=device).half()}
    sink = torch.empty(wg * 512, dtype=torch.float32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    iters = 1 << 14
    flop = wg * 16 * iters * 32768
    out = {"workgroups": wg, "flop_per_launch": flop}
    for name, ops in operands.items():
        def launch():
            _lib.call("kunserve_mfma_probe", 0, ops.data_ptr(), sink.data_ptr(), wg, iters, stream)
        t_end = time.perf_counter() + settle_s
        while time.perf_counter() < t_end:
            for _ in range(8):
                launch()
            torch.cuda.synchronize()
        ms = region_ms(lambda: [launch() for _ in range(reps)], device) / reps
        out[name + "_tflops"] = flop / (ms * 1e-3) / 1e12
    log("fp16 MFMA ceiling (32x32x16, two waves per SIMD, every CU): constant operands "
        "{constant_tflops:.0f}, random operands {random_tflops:.0f} TFLOP/s".format(**out))
    return out


# -------------------------------------------------------------------- swap


def bench_swap(args, device):
    """Block swap (torch.ops.swapping_ops.swap) between the GPU pool and a
    pinned host pool, both directions, on blocks of the remap workload's
    shape ([32 layers, 8 KV heads, 16, 128] fp16 = 1 MiB per K or V block).
    The copies run on the DMA engines over the host link, so the roofline is
    the link: one contiguous pinned copy of the same byte count, timed the
    same way, is the reference rate."""
    import kunserve_amd as ks

    shape = (32, 8, 16, 128)
    n_gpu, n_cpu, n = 2048, 1024, 512
    rng = np.random.default_rng(1007)
    gen = torch.Generator(device=device)
    gen.manual_seed(1007)
    kc = torch.empty((n_gpu, *shape), dtype=torch.float16, device=device)
    vc = torch.empty_like(kc)
    fill_random_(kc, gen, 0)
    fill_random_(vc, gen, 0)
    ksw = torch.empty((n_cpu, *shape), dtype=torch.float16, pin_memory=True)
    vsw = torch.empty_like(ksw, pin_memory=True)
    gpu_src = rng.permutation(n_gpu // 2)[:n].tolist()               # from the first half
    cpu_slot = rng.permutation(n_cpu)[:n].tolist()
    gpu_dst = (n_gpu // 2 + rng.permutation(n_gpu // 2)[:n]).tolist()  # into the second half
    nbytes = 2 * n * kc[0].numel() * 2

    def timed(fn, reps=3):
        best = None
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            t = a.elapsed_time(b)
            best = t if best is None else min(best, t)
        return best

    out_ms = timed(lambda: ks.swap(gpu_src, cpu_slot, False, kc, vc, ksw, vsw))
    in_ms = timed(lambda: ks.swap(cpu_slot, gpu_dst, True, kc, vc, ksw, vsw))
    ok = bool(torch.equal(kc[gpu_dst].view(torch.int16), kc[gpu_src].view(torch.int16)) and
              torch.equal(vc[gpu_dst].view(torch.int16), vc[gpu_src].view(torch.int16)))
    # Link reference: one contiguous pinned copy of the same byte count.
    dev_buf = kc[:2 * n].reshape(-1)
    host_buf = torch.empty(dev_buf.numel(), dtype=torch.float16, pin_memory=True)
    d2h_ms = timed(lambda: host_buf.copy_(dev_buf, non_blocking=True))
    h2d_ms = timed(lambda: dev_buf.copy_(host_buf, non_blocking=True))
    gbs = lambda ms: nbytes / (ms * 1e-3) / 1e9
    res = {"workload": f"swap {n} blocks of 2 x 1 MiB (K and V) GPU<->pinned host",
           "out_gbs": gbs(out_ms), "in_gbs": gbs(in_ms),
           "link_d2h_gbs": gbs(d2h_ms), "link_h2d_gbs": gbs(h2d_ms),
           "out_frac_of_link": d2h_ms / out_ms, "in_frac_of_link": h2d_ms / in_ms,
           "bit_exact_round_trip": ok}
    log(f"swap: out {res['out_gbs']:.1f} GB/s ({res['out_frac_of_link'] * 100:.0f}% of a "
        f"contiguous D2H copy, {res['link_d2h_gbs']:.1f} GB/s); in {res['in_gbs']:.1f} GB/s "
        f"({res['in_frac_of_link'] * 100:.0f}% of H2D, {res['link_h2d_gbs']:.1f} GB/s); "
        f"round trip bit-exact: {ok}")
    del kc, vc, ksw, vsw, host_buf
    return res


def load_traffic():
    """HBM bytes per decode launch measured by rocprofv3 (FETCH_SIZE and
    WRITE_SIZE passes, scaled by a known-size copy); None if not recorded."""
    import re

    path = os.path.join(PROFILE_DIR, "paged_decode_llama2_7b_traffic.md")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        m = re.search(r"^hbm_bytes_per_launch = (\d+)$", f.read(), re.M)
    return int(m.group(1)) if m else None


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--part-tokens", type=int, default=0, help="decode partition (0 = auto)")
    ap.add_argument("--only", choices=["decode", "prefill", "prefill256", "gqa", "bf16",
                                       "bf16p256", "bf16prefill", "remap", "pmm", "swap",
                                       "mfma", "single", "mixed", "prefillhd"],
                    default=None)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0,
                    help="seconds of timed CPU baseline runs (at least 3 runs)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(2)
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    import kunserve_amd

    log(f"library {kunserve_amd.library_path()}; device "
        f"{torch.cuda.get_device_properties(device).name}")

    if args.only == "prefill":
        print(json.dumps({"prefill": bench_prefill(args, device)}))
        return
    if args.only == "bf16prefill":
        print(json.dumps({"bf16_prefill_page256": bench_prefill(args, device, page_size=256,
                                                                dtype=torch.bfloat16)}))
        return
    if args.only == "single":
        print(json.dumps({"single_layer_decode": bench_single_layer(args, device)}))
        return
    if args.only == "mixed":
        print(json.dumps({"mixed_step": bench_mixed(args, device)}))
        return
    if args.only == "mfma":
        print(json.dumps({"mfma_ceiling": mfma_ceiling(device)}))
        return
    if args.only == "prefillhd":
        legs = {f"prefill_head_dim{hd}": bench_prefill(args, device, head_dim=hd) for hd in (64, 256)}
        legs["prefill_gqa8"] = bench_prefill(args, device, num_kv_heads=8)
        print(json.dumps(legs))
        return
    if args.only == "prefill256":
        print(json.dumps({"prefill_page256": bench_prefill(args, device, page_size=256)}))
        return
    if args.only == "gqa":
        print(json.dumps({"gqa_decode": bench_gqa(args, device)}))
        return
    if args.only == "bf16":
        print(json.dumps({"bf16_decode": bench_bf16_decode(args, device)}))
        return
    if args.only == "bf16p256":
        print(json.dumps({"bf16_decode_page256": bench_bf16_decode(args, device, page_size=256)}))
        return
    if args.only == "remap":
        print(json.dumps({"remap": bench_remap(args, device)}))
        return
    if args.only == "pmm":
        print(json.dumps({"pmm": bench_pmm(args, device)}))
        return
    if args.only == "swap":
        print(json.dumps({"swap": bench_swap(args, device)}))
        return

    dec = bench_decode(args, device)
    err = check_decode(dec, device)
    log(f"decode max-abs error over every row of layers 0 and 31 vs an fp32 torch "
        f"reference: {err:.2e}")
    if err > 2e-3:
        print(f"decode result check failed: max-abs {err}", file=sys.stderr)
        sys.exit(1)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(dec, args.cpu_budget)
        log(f"cpu baseline: {cpu['value']:.3f} GB/s ({cpu['sample']})")
    w = dec["workload"]
    del dec["pool"], dec["qs"]
    torch.cuda.empty_cache()
    prefill = prefill256 = prefill_bf16 = gqa = bf16 = bf16_256 = remap = pmm = swp = None
    ceiling = single = mixed = None
    prefill_hd = {"prefill_head_dim64": None, "prefill_head_dim256": None, "prefill_gqa8": None}
    if args.only is None:
        single = bench_single_layer(args, device)
        torch.cuda.empty_cache()
        mixed = bench_mixed(args, device)
        torch.cuda.empty_cache()
        ceiling = mfma_ceiling(device)
        prefill = bench_prefill(args, device)
        prefill["frac_of_random_operand_ceiling"] = prefill["tflops"] / ceiling["random_tflops"]
        torch.cuda.empty_cache()
        prefill256 = bench_prefill(args, device, page_size=256)
        prefill256["frac_of_random_operand_ceiling"] = prefill256["tflops"] / ceiling["random_tflops"]
        torch.cuda.empty_cache()
        prefill_bf16 = bench_prefill(args, device, page_size=256, dtype=torch.bfloat16)
        torch.cuda.empty_cache()
        prefill_hd = {}
        for hd in (64, 256):
            r = bench_prefill(args, device, head_dim=hd)
            prefill_hd[f"prefill_head_dim{hd}"] = {
                k: r[k] for k in ("workload", "head_dim", "causal_tflop", "attention_ms", "tflops",
                                  "mfma_util")}
            torch.cuda.empty_cache()
        r = bench_prefill(args, device, num_kv_heads=8)
        prefill_hd["prefill_gqa8"] = {
            k: r[k] for k in ("workload", "num_qo_heads", "num_kv_heads", "causal_tflop",
                              "attention_ms", "tflops", "mfma_util", "flop_per_byte")}
        torch.cuda.empty_cache()
        gqa = bench_gqa(args, device)
        torch.cuda.empty_cache()
        bf16 = bench_bf16_decode(args, device)
        torch.cuda.empty_cache()
        bf16_256 = bench_bf16_decode(args, device, page_size=256)
        torch.cuda.empty_cache()
        remap = bench_remap(args, device)
        torch.cuda.empty_cache()
        pmm = bench_pmm(args, device)
        torch.cuda.empty_cache()
        swp = bench_swap(args, device)
        torch.cuda.empty_cache()

    line = {
        "metric": METRIC,
        "value": round(dec["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": w.name,
            "layers": w.num_layers, "batch": w.batch, "num_qo_heads": w.num_qo_heads,
            "num_kv_heads": w.num_kv_heads, "head_dim": w.head_dim, "page_size": w.page_size,
            "num_pages": w.num_pages, "total_kv_tokens": int(w.kv_len.sum()),
            "part_tokens": dec["plan"].info.part_tokens,
            "hbm_frac": round(dec["value"] / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(dec["achieved"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dec["achieved"] / HBM_PEAK_GBS, 4),
            "traffic": load_traffic(),
            "kernel": "paged_decode_kernel<f16, 128, 1> + decode_merge_kernel<f16, 128> (one launch per layer)",
            "access_pattern_ceiling": dec.get("access_pattern"),
            "algorithmic_bytes_per_launch": dec["bytes_per_layer"],
            "launch_us": round(dec["launch_ms"] * 1e3, 2),
        },
        "cpu_baseline": cpu,
        "single_layer_decode": single,
        "mixed_step": mixed,
        "prefill": prefill,
        "mfma_ceiling": ceiling,
        "prefill_page256": prefill256,
        **prefill_hd,
        "gqa_decode": gqa,
        "bf16_decode": bf16,
        "bf16_decode_page256": bf16_256,
        "bf16_prefill_page256": prefill_bf16,
        "remap": remap,
        "pmm": pmm,
        "swap": swp,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
