#!/usr/bin/env python3
"""BeamAttention decode benchmark on one MI355X.

Workload: one decode step of 8 requests x 128 beams over a 2048-token shared
prefix (per-request suffix length uniform in [1, 8]), 32 query / 8 KV heads,
head_dim 128, block 16, bf16 -- synthetic seeded inputs already resident in
HBM.  A "step" is one gr_beam_attn_decode launch over the whole batch.

Prints one JSON line: value = algorithmic GB/s (each request's prefix K/V
counted once + suffix K/V + Q + O + tables) over the average step time;
roofline for the decode kernel against 8 TB/s; cpu_baseline = the torch
float32 cascade restatement of the reference (oracle/cpu_baseline.py) on the
host cores for the same step.

--workload fork | prune measure the fork+append and pruning kernels the same
way; --workload e2e runs the end-to-end semantic-ID beam decode (4 prompts x
2048 tokens, 128 beams, 3 tokens, 28-layer decoder) and reports the p99
request latency.
"""

from __future__ import annotations

import argparse
import gc
import json
import math
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "vllm-gr-ehaleva_amd")]

METRIC = "BeamAttention decode µs/step + HBM GB/s (% peak) at 128 beams, 2K prefix"
METRIC_SID = ("BeamAttention decode (split prefix) µs/step + HBM GB/s (% peak) at the semantic-ID decode "
              "step's shape: 4 requests x 128 beams, 2K prefix")
HBM_PEAK_GBPS = 8000.0
PMC_SUMMARY = {w: os.path.join(ROOT, "profiles", f"{w}_beam128_hbm_traffic.txt") for w in ("decode", "fork", "prune")}
PMC_SUMMARY["decode_sid"] = os.path.join(ROOT, "profiles", "decode_sid_step_hbm_traffic.txt")


def _log(*a):
    print(*a, file=sys.stderr, flush=True)


def _traffic_from_profile(workload: str = "decode"):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    calibrated against a copy kernel), when that summary has been committed."""
    try:
        with open(PMC_SUMMARY[workload]) as f:
            m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", f.read())
        return float(m.group(1)) if m else None
    except OSError:
        return None


def cpu_baseline(wl, budget_s: float = 20.0):
    import torch
    from oracle.cpu_baseline import cascade_decode_fp32

    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    args = (wl.q, wl.k_cache, wl.v_cache, wl.prefix_bt, wl.prefix_len, wl.beam_start, wl.suffix_bt,
            wl.suffix_len)
    kw = dict(scale=wl.scale, block_size=wl.block_size)
    R = len(wl.prefix_len)
    # bounded sample: whole requests, as many as fit the budget after one timed probe
    t0 = time.perf_counter()
    cascade_decode_fp32(*args, **kw, requests=[0])
    per_req = time.perf_counter() - t0
    reqs = list(range(min(R, max(1, int(budget_s / 12 / max(per_req, 1e-6))))))
    times = []
    for i in range(12):  # 2 warm-ups + 10 timed
        t0 = time.perf_counter()
        cascade_decode_fp32(*args, **kw, requests=reqs)
        if i >= 2:
            times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    us_step = med / len(reqs) * R * 1e6
    gbps = wl.algorithmic_bytes() / (us_step * 1e-6) / 1e9
    return {"value": round(gbps, 3), "unit": "GB/s", "cores": n, "kind": "port",
            "us_per_step": round(us_step, 1),
            "sample": f"{len(reqs)} of {R} requests (x128 beams, prefix 2048) per run, median of 10 "
                      f"after 2 warm-ups, scaled to the full step; torch float32 cascade "
                      f"(prefix pass + suffix pass + LSE merge)"}


# Copies of a workload that one timed loop rotates over: their inputs total
# well over the MI355X's 256 MB Infinity Cache (MALL), so a launch finds the
# bytes the previous launches touched evicted and reads its own from HBM --
# as a served decode step does, whose 28 layers each read distinct KV.
COLD_COPIES = 5
MALL_BYTES = 256 << 20


TIMING_NOTE = ("device time of back-to-back launches between two HIP events; every timed launch is queued "
               "behind a spin kernel before the start event, so host enqueue time is outside the window")
HOST_US: dict = {}  # host microseconds per enqueue of the last timed loop, by label


def _time_launches(steps_fns, steps: int, warmup: int, label: str | None = None) -> float:
    """Average microseconds per launch over ``steps`` back-to-back launches on
    the current stream (HIP events), after ``warmup`` untimed launches.
    ``steps_fns``: one launch closure, or a list of them (one per workload
    copy) taken in turn.

    The host's enqueue time stays out of the window: a spin kernel
    (``torch.cuda._sleep``) sized to several times the measured host time of
    the whole loop is queued ahead of the start event, so every timed launch
    is already queued when the window opens and the events time the device
    alone.  The host microseconds per enqueue go to ``HOST_US[label]``."""
    import torch
    fns = steps_fns if isinstance(steps_fns, list) else [steps_fns]
    t0 = time.perf_counter()
    for i in range(max(warmup, 1)):
        fns[i % len(fns)]()
    host_est = (time.perf_counter() - t0) / max(warmup, 1)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    # ~2.4 GHz shader clock: cover 4x the estimated enqueue time plus 2 ms
    torch.cuda._sleep(int((4.0 * host_est * steps + 2e-3) * 2.4e9))
    start.record(stream)
    t0 = time.perf_counter()
    for i in range(steps):
        fns[i % len(fns)]()
    host = time.perf_counter() - t0
    end.record(stream)
    torch.cuda.synchronize()
    if label is not None:
        HOST_US[label] = round(host * 1e6 / steps, 2)
    return start.elapsed_time(end) * 1000.0 / steps


def _device_copy(t, gen):
    """A fresh device tensor shaped like ``t``: float tensors redrawn from
    ``gen`` (N(0,1) scaled to t's std), integer tensors cloned."""
    import torch
    if t.is_floating_point():
        std = float(t[:1].float().std()) if t.numel() > 1 else 1.0
        return (torch.randn(t.shape, generator=gen, device=t.device, dtype=torch.float32) * std).to(t.dtype)
    return t.clone()


def bench_other(args) -> int:
    """Fork+append (16 requests x 128 beams, old suffix U[1,15], 8 KV heads x
    128 bf16) or pruning (64 requests x 128 beams x vocab 8192 fp32)."""
    import numpy as np
    import torch
    from vllm_gr_amd import ops, workloads

    dev = torch.device("cuda:0")
    n_cpu = len(os.sched_getaffinity(0))
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    if args.workload == "fork":
        host = workloads.fork_beam128(seed=0)
        wl = host.to(dev)
        bt_out = torch.empty_like(wl.suffix_bt)
        len_out = torch.empty_like(wl.suffix_len)

        def make_step(kv, k_new, v_new):
            def step():  # out-of-place tables; copies and appends rewrite the same bytes each time
                ops.beam_kv_fork(wl.parent, wl.suffix_bt, wl.suffix_len, kv[0], kv[1], k_new, v_new,
                                 bt_out=bt_out, len_out=len_out)
            return step
        warm = make_step(wl.kv_cache, wl.k_new, wl.v_new)
        cold = [warm] + [make_step(_device_copy(wl.kv_cache, gen), _device_copy(wl.k_new, gen),
                                   _device_copy(wl.v_new, gen)) for _ in range(COLD_COPIES - 1)]
        nbytes = host.algorithmic_bytes()
        metric = "beam KV fork+append us/step + HBM GB/s at 16 requests x 128 beams"
        workload = "fork+append: 16 requests x 128 beams, old suffix U[1,15], 8 kv heads x 128, block 16, bf16"
        dtype = "u16 (bf16 bit copies) + int32 tables"
    else:
        host = workloads.prune_beam128(seed=0)
        wl = host.to(dev)
        ws = torch.empty(ops.prune_workspace_bytes(64, 128, 8192, 128), dtype=torch.uint8, device=dev)
        outs = (torch.empty((64, 128), dtype=torch.int32, device=dev),
                torch.empty((64, 128), dtype=torch.int32, device=dev),
                torch.empty((64, 128), dtype=torch.float32, device=dev),
                torch.empty((64, 128), dtype=torch.float32, device=dev))

        def make_step(logits):
            def step():
                ops.beam_prune_topk(logits, wl.cum, 128, -1, workspace=ws, out=outs)
            return step
        warm = make_step(wl.logits)
        cold = [warm, make_step(_device_copy(wl.logits, gen))]  # 2 x 256 MiB of logits
        nbytes = host.algorithmic_bytes()
        metric = "fused beam pruning us/step + HBM GB/s at 64 requests x 128 beams x vocab 8192"
        workload = "prune: log_softmax + cum + top-128 over 128 beams x 8192 vocab, 64 requests, fp32"
        dtype = "f32 (f64 scores)"
    us = _time_launches(cold, args.steps, args.warmup, "cold")
    us_warm = None if args.no_warm else _time_launches(warm, args.steps, args.warmup, "warm")
    gbps = nbytes / (us * 1e-6) / 1e9
    _log(f"bench: {args.workload}: cold {us:.2f} us/step, {gbps:.1f} GB/s algorithmic ({nbytes} B/step); "
         f"warm {us_warm} us/step")
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import cpu_baseline as cb
        torch.set_num_threads(n_cpu)
        if args.workload == "fork":
            kc, vc = host.kv_cache[0].clone(), host.kv_cache[1].clone()
            run = lambda: cb.fork_append_torch(host.parent, host.suffix_bt, host.suffix_len, kc, vc,
                                               host.k_new, host.v_new, block_size=host.block_size)
            what = "torch index ops (owner / copy-on-write tables, slot gather-scatter, append)"
        else:
            run = lambda: cb.prune_topk_torch(host.logits, host.cum, 128)
            what = "torch float32 log_softmax + per-beam top-128, then per-request top-128 of cum + logprob"
        run()  # warm-up
        times = []
        t_end = time.perf_counter() + 10.0
        while len(times) < 3 or time.perf_counter() < t_end:
            t0 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t0)
        times.sort()
        us_cpu = times[len(times) // 2] * 1e6
        sample = f"the full step, median of {len(times)} runs after a warm-up; {what}"
        cores = n_cpu
        cpu = {"value": round(nbytes / (us_cpu * 1e-6) / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
               "us_per_step": round(us_cpu, 1), "sample": sample}
        _log(f"bench: cpu {cpu} (host has {n_cpu} cores)")
    line = {"metric": metric, "value": round(gbps, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(us / 1000.0, 5), "us_per_step": round(us, 3),
            "pct_hbm_peak": round(100.0 * gbps / HBM_PEAK_GBPS, 2), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": dtype, "data": "synthetic (seeded)",
            "config": {"workload": workload, "algorithmic_bytes_per_step": nbytes,
                       "inputs": f"{len(cold)} copies rotated per launch (cold: no reuse through the "
                                 f"256 MB Infinity Cache)"},
            "warm": None if us_warm is None else {
                "us_per_step": round(us_warm, 3), "gbps": round(nbytes / (us_warm * 1e-6) / 1e9, 2),
                "inputs": "one copy relaunched"},
            "host_us_per_enqueue": dict(HOST_US),
            "timing": TIMING_NOTE,
            "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": _traffic_from_profile(args.workload)},
            "cpu_baseline": cpu}
    print(json.dumps(line), flush=True)
    return 0


MFMA_BF16_PEAK_TFLOPS = 2500.0
PMC_SUMMARY["prefill"] = os.path.join(ROOT, "profiles", "prefill_sid_prompt_hbm_traffic.txt")


def bench_prefill(args) -> int:
    """One layer's prompt attention of the semantic-ID workload: 4 requests x
    2048-token prompts, 16 q / 8 kv heads, head_dim 128, bf16, causal over the
    paged cache (the standard path's flash_attn_varlen_func call,
    beam_attn.py:643-654).  The kernel is MFMA-bound: the line's roofline is
    TFLOP/s against the dense bf16 peak."""
    import torch
    from vllm_gr_amd import ops

    dev = torch.device("cuda:0")
    R, S, Hq, Hkv, D, bs = 4, 2048, 16, 8, 128, 16
    nb = R * S // bs
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    bt = torch.randperm(nb, generator=gen, device=dev).to(torch.int32).view(R, S // bs)
    qs = torch.arange(0, R * S + 1, S, device=dev, dtype=torch.int32)
    sl = torch.full((R,), S, device=dev, dtype=torch.int32)
    flops = R * Hq * 4 * D * (S * (S + 1) // 2)  # QK^T and PV over the causal triangle
    nbytes = 2 * R * S * Hq * D * 2 + 2 * R * S * Hkv * D * 2  # Q, O; K, V once

    def make_step():
        kv = torch.randn((2, nb, bs, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
        q = torch.randn((R * S, Hq, D), generator=gen, device=dev).to(torch.bfloat16)
        out = torch.empty_like(q)

        def step():
            ops.paged_attn_prefill(q, kv[0], kv[1], bt, qs, sl, max_query_len=S, scale=D ** -0.5, out=out)
        return step
    copies = -(-MALL_BYTES // nbytes) + 2
    cold = [make_step() for _ in range(copies)]
    us = _time_launches(cold, args.steps, args.warmup, "cold")
    us_warm = None if args.no_warm else _time_launches(cold[0], args.steps, args.warmup, "warm")
    tflops = flops / (us * 1e-6) / 1e12
    gbps = nbytes / (us * 1e-6) / 1e9
    _log(f"bench: prefill: cold {us:.2f} us/step, {tflops:.1f} TFLOP/s, {gbps:.1f} GB/s; warm {us_warm}")
    cpu = None
    if not args.no_cpu_baseline:
        n_cpu = len(os.sched_getaffinity(0))
        torch.set_num_threads(n_cpu)
        g = torch.Generator().manual_seed(0)
        qh = torch.randn((1, 2, S, D), generator=g)  # one request, one KV head's two query heads
        kh = torch.randn((1, 1, S, D), generator=g).expand(1, 2, S, D)
        vh = torch.randn((1, 1, S, D), generator=g).expand(1, 2, S, D)
        run = lambda: torch.nn.functional.scaled_dot_product_attention(qh, kh, vh, is_causal=True)
        run()
        times = []
        t_end = time.perf_counter() + 10.0
        while len(times) < 3 or time.perf_counter() < t_end:
            t0 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t0)
        times.sort()
        us_cpu = times[len(times) // 2] * 1e6 * R * Hkv
        cpu = {"value": round(flops / (us_cpu * 1e-6) / 1e12, 4), "unit": "TFLOP/s", "cores": n_cpu,
               "kind": "port", "us_per_step": round(us_cpu, 1),
               "sample": f"one request's one KV head (2 query heads, 2048 causal tokens) in torch float32 "
                         f"SDPA, median of {len(times)} runs, scaled x{R * Hkv} to the layer"}
    line = {"metric": "paged causal prefill us/layer + TFLOP/s (% bf16 MFMA peak) at 4 x 2048-token prompts",
            "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(us / 1000.0, 5), "us_per_step": round(us, 3),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded N(0,1) Q/K/V, random block table)",
            "config": {"workload": "prefill: 4 requests x 2048-token prompts, causal, 16 q / 8 kv heads, "
                                   "head_dim 128, block 16 (one layer)", "flops_per_step": flops,
                       "algorithmic_bytes_per_step": nbytes, "gbps": round(gbps, 2),
                       "inputs": f"{len(cold)} copies rotated per launch"},
            "warm": None if us_warm is None else {"us_per_step": round(us_warm, 3),
                                                  "tflops": round(flops / (us_warm * 1e-6) / 1e12, 2)},
            "host_us_per_enqueue": dict(HOST_US),
            "timing": TIMING_NOTE,
            "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                         "traffic": _traffic_from_profile("prefill")},
            "cpu_baseline": cpu}
    print(json.dumps(line), flush=True)
    return 0


def e2e_cpu_baseline(cfg, prompt, n_req: int, budget_s: float = 15.0):
    """The prefill phase of the batch on the host cores: one decoder layer
    over one 2048-token prompt in torch float32 (the oracle's full forward),
    timed and scaled by layers x requests."""
    import dataclasses
    import torch
    from oracle import sid_beam as so
    from vllm_gr_amd.v1.sid_decoder import init_weights

    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    one = dataclasses.replace(cfg, num_layers=1, dtype=torch.float32)
    w = init_weights(one, seed=0)
    times = []
    t0 = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t0 < budget_s and len(times) < 10):
        t1 = time.perf_counter()
        with torch.no_grad():
            so.decoder_logits(w, one, prompt)
        times.append(time.perf_counter() - t1)
    times.sort()
    per_layer = times[len(times) // 2]
    ms = per_layer * cfg.num_layers * n_req * 1e3
    return {"value": round(ms, 1), "unit": "ms (prefill phase)", "cores": n, "kind": "port",
            "sample": f"1 decoder layer (+ embedding/lm_head) over one {len(prompt)}-token prompt, torch "
                      f"float32, median of {len(times)}, scaled x{cfg.num_layers} layers x{n_req} requests"}


def bench_e2e(args) -> int:
    """Semantic-ID beam decode of 4 prompts x 2048 tokens, 128 beams, 3 SID
    tokens through the 28-layer decoder: prefill once, then per step decode
    -> prune -> fork.  One timed step = one whole batch (every request of it
    completes together), host wall clock from the call to the results on the
    host."""
    import torch
    from vllm_gr_amd.entrypoints.beam_search import BeamSearchParams
    from vllm_gr_amd.entrypoints.llm import LLM
    from vllm_gr_amd.v1.sid_decoder import SID_DECODER_1P7B as cfg
    from vllm_gr_amd.v1.sid_runner import blocks_needed

    R, P, W, T = 4, 2048, 128, 3
    _log("bench: e2e: initialising the 28-layer decoder (seed 0, N(0, 0.02) bf16)")
    llm = LLM(cfg, seed=0, num_blocks=blocks_needed(R, P, W, T, 16) + 64)
    g = torch.Generator().manual_seed(0)
    prompts = [torch.randint(0, cfg.vocab, (P,), generator=g).tolist() for _ in range(R)]
    params = BeamSearchParams(beam_width=W, max_tokens=T)
    for _ in range(args.warmup):
        llm.beam_search(prompts, params)
    torch.cuda.synchronize()
    # as a serving engine does once it is up (vLLM's engine core calls
    # gc.collect() + gc.freeze() after start-up): the long-lived objects of
    # initialisation leave the collector's generations, so a collection
    # during a batch scans only that batch's garbage
    gc.collect()
    gc.freeze()
    walls, pre, steps = [], [], []
    t0 = time.perf_counter()
    for i in range(args.steps):
        llm.beam_search(prompts, params)
        t = llm.last_times
        walls.append(t.wall_ms)
        pre.append(t.prefill_ms)
        steps.append(t.step_ms)
        if (i + 1) % 10 == 0:
            _log(f"bench: e2e batch {i + 1}/{args.steps}: wall {t.wall_ms:.2f} ms")
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    srt = sorted(walls)
    p99 = srt[min(len(srt) - 1, int(math.ceil(0.99 * len(srt))) - 1)]
    med = srt[len(srt) // 2]
    pre_med = sorted(pre)[len(pre) // 2]
    step_med = [sorted(s[j] for s in steps)[len(steps) // 2] for j in range(len(steps[0]))]
    tokens = R * P
    prefill_flops = 2 * cfg.num_params() * tokens + 4 * cfg.num_layers * cfg.num_heads * cfg.head_dim * R * P * (P + 1) // 2
    tflops = prefill_flops / (pre_med * 1e-3) / 1e12
    _log(f"bench: e2e p99 {p99:.2f} ms, median {med:.2f} ms, prefill {pre_med:.2f} ms ({tflops:.0f} TFLOP/s), "
         f"steps {[round(x, 3) for x in step_med]} ms")
    cpu = None
    if not args.no_cpu_baseline:
        cpu = e2e_cpu_baseline(cfg, prompts[0], R)
        _log(f"bench: cpu {cpu}")
    line = {"metric": "semantic-ID beam decode request latency (p99) at 4 prompts x 2048 tokens, "
                      "128 beams, 3 SID tokens, 28-layer decoder",
            "value": round(p99, 3), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(elapsed * 1e3 / args.steps, 3), "median_ms": round(med, 3),
            "prefill_ms": round(pre_med, 3), "decode_step_ms": [round(x, 3) for x in step_med],
            "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (random-init N(0,0.02) weights, seeded random prompt ids)",
            "config": {"workload": "e2e semantic-ID beam decode: 4 requests x 2048-token prompt, beam 128, "
                                   "3 tokens; 28 layers, hidden 2048, 16/8 heads x 128, FFN 6144, vocab 8192",
                       "requests": R, "prompt": P, "beams": W, "max_tokens": T},
            "roofline": {"bound": "mfma", "scope": "prefill phase (GEMM-dominated)",
                         "achieved": round(tflops, 1), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None},
            "cpu_baseline": cpu}
    print(json.dumps(line), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-warm", action="store_true",
                    help="skip the warm (one relaunched copy) timing; the cold rotation is the headline")
    ap.add_argument("--kernel", choices=["auto", "generic"], default="auto")
    ap.add_argument("--option", choices=["none", "window", "sinks", "alibi", "fp8", "softcap"], default="none",
                    help="decode with one optional attention feature of the reference's impl "
                         "(beam_attn.py:597-625): a 1024-token sliding window, per-head sinks, ALiBi "
                         "slopes, an fp8 e4m3 KV cache (scales 1), or a logit soft cap of 50")
    ap.add_argument("--shape", choices=["c2", "sid"], default="c2",
                    help="decode shape: c2 (8 requests x 128 beams, 32/8 heads; the headline) or sid (one "
                         "layer of the semantic-ID decode step: 4 x 128 beams, 16/8 heads, suffix 1-3, "
                         "the split prefix with the longest-prefix hint, as the backend runs it)")
    ap.add_argument("--workload", choices=["decode", "fork", "prune", "prefill", "e2e"], default="decode",
                    help="decode (the headline line), the fork+append / pruning kernels, prefill (one "
                         "layer's prompt attention of the semantic-ID workload), or e2e (whole semantic-ID "
                         "beam decode through a 28-layer decoder; a step is one batch)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a 256 MiB device-to-device copy (5 launches), the reference point "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (requests are "
              "independent, so N GPUs shard requests data-parallel with no exchange).", file=sys.stderr)
        return 2

    import torch

    if args.calibrate_copy:
        n = 256 << 20
        src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read_per_launch": n, "bytes_written_per_launch": n,
                          "launches": 5}), flush=True)
        return 0
    from vllm_gr_amd import ops, workloads

    if args.workload == "e2e":
        return bench_e2e(args)
    if args.workload == "prefill":
        return bench_prefill(args)
    if args.workload != "decode":
        return bench_other(args)

    dev = torch.device("cuda:0")
    sid = args.shape == "sid"
    _log(f"bench: building {'decode_sid_step' if sid else 'decode_beam128'} inputs (seed 0)")
    host_wl = workloads.decode_sid_step(seed=0) if sid else workloads.decode_beam128(seed=0)
    hint = int(host_wl.prefix_len.max()) if sid else None
    wl = host_wl.to(dev)
    ops.set_decode_kernel(args.kernel)

    Hq = wl.q.shape[1]
    opt_kw = {}
    if args.option == "window":
        opt_kw["window"] = (1023, -1)
    elif args.option == "sinks":
        opt_kw["sinks"] = torch.linspace(-1.0, 1.0, Hq, device=dev)
    elif args.option == "alibi":
        opt_kw["alibi_slopes"] = torch.tensor([2.0 ** (-8.0 * (h + 1) / Hq) for h in range(Hq)], device=dev)
    elif args.option == "softcap":
        opt_kw["softcap"] = 50.0
    elif args.option == "fp8":
        one = torch.ones(1, dtype=torch.float32, device=dev)
        opt_kw.update(k_scale=one, v_scale=one)
        wl.kv_cache = wl.kv_cache.to(torch.float8_e4m3fn)

    def make_step(kv, q):
        out = torch.empty_like(q)

        def step():
            ops.beam_attn_decode(q, kv[0], kv[1], wl.prefix_bt, wl.prefix_len, wl.beam_start,
                                 wl.suffix_bt, wl.suffix_len, scale=wl.scale, max_beams_per_req=wl.max_beams,
                                 out=out, max_prefix_len=hint, **opt_kw)
        return step

    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    warm = make_step(wl.kv_cache, wl.q)
    nbytes = host_wl.algorithmic_bytes()
    if args.option == "fp8":  # one byte per cached element
        nbytes -= (int(host_wl.prefix_len.sum()) + int(host_wl.suffix_len.sum())) * 2 * 8 * 128
    if args.option == "window":  # prefix keys no row of a request can see are not read
        hidden = sum(max(0, int(p) - 1 - opt_kw["window"][0]) for p in host_wl.prefix_len.tolist())
        nbytes -= hidden * 2 * 8 * 128 * 2
    copies = max(COLD_COPIES, -(-MALL_BYTES // nbytes) + 2)
    # each copy: its own cache pool and queries (the same tables: tiny), drawn on the device
    cold = [warm] + [make_step(_device_copy(wl.kv_cache, gen), _device_copy(wl.q, gen))
                     for _ in range(copies - 1)]
    assert (copies - 1) * nbytes > MALL_BYTES
    us_step = _time_launches(cold, args.steps, args.warmup, "cold")
    us_warm = None if args.no_warm else _time_launches(warm, args.steps, args.warmup, "warm")
    gbps = nbytes / (us_step * 1e-6) / 1e9
    _log(f"bench: cold {us_step:.2f} us/step, {gbps:.1f} GB/s algorithmic ({nbytes} B/step); "
         f"warm {us_warm} us/step")

    cpu = None
    if not args.no_cpu_baseline:
        _log("bench: timing the CPU baseline")
        cpu = cpu_baseline(host_wl)
        _log(f"bench: cpu {cpu}")

    R, W = host_wl.prefix_len.numel(), host_wl.max_beams
    Hq_, Hkv_ = host_wl.q.shape[1], host_wl.kv_cache.shape[3]
    lmin, lmax = int(host_wl.suffix_len.min()), int(host_wl.suffix_len.max())
    line = {
        "metric": METRIC_SID if sid else METRIC,
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_step / 1000.0, 5),
        "us_per_step": round(us_step, 3),
        "pct_hbm_peak": round(100.0 * gbps / HBM_PEAK_GBPS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)/sqrt(128) Q/K/V, random block tables)",
        "config": {"workload": f"beam decode: {R} requests x {W} beams, shared prefix 2048, suffix "
                               f"{'U[1,3]' if sid else 'U[1,8]'} (drawn {lmin}-{lmax}), {Hq_} q / {Hkv_} kv "
                               f"heads, head_dim 128, block 16" + (", split prefix" if sid else ""),
                   "requests": R, "beams": W, "prefix": 2048, "kernel": args.kernel, "option": args.option,
                   "algorithmic_bytes_per_step": nbytes, "flops_per_step": host_wl.flops(),
                   "inputs": f"{len(cold)} copies rotated per launch (cold: no reuse through the 256 MB "
                             f"Infinity Cache)"},
        "warm": None if us_warm is None else {
            "us_per_step": round(us_warm, 3), "gbps": round(nbytes / (us_warm * 1e-6) / 1e9, 2),
            "inputs": "one copy relaunched"},
        "host_us_per_enqueue": dict(HOST_US),
        "timing": TIMING_NOTE,
        "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4),
                     # the committed counter profiles cover the option-free decodes
                     "traffic": (_traffic_from_profile("decode_sid" if sid else "decode")
                                 if args.option == "none" else None)},
        # the kernel sits near the ridge: its matrix-core use beside the HBM roofline
        "mfma": {"achieved": round(host_wl.flops() / (us_step * 1e-6) / 1e12, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                 "unit": "TFLOP/s", "frac": round(host_wl.flops() / (us_step * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
