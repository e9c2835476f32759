"""Benchmark: paged decode-attention KV GB/s on one MI355X.

Workload (the headline metric's configuration): one layer of Qwen3-8B-shaped
decode attention — batch 1, 32 query / 8 KV heads, head_dim 128, bf16 KV,
32,768-token context in 2,048 pages of 16 tokens under a seeded random page
table, q/K/V ~ N(0,1), scale 1/sqrt(128), all pages resident.  A step is one
attention call over the whole context.  Eight independent 128 MiB pools are
rotated so the 256 MB Infinity Cache cannot serve the KV.  `value` is the
algorithmic bytes of one call over its time (decode kernel + split merge,
HIP events around the calls); `roofline` is the dominant kernel's: the same
bytes over the decode kernel's own duration, from HIP events attached to its
launch in a second pass of the same calls (helm_profile_split_kernels),
with the whole-call figures beside it under `roofline.per_call`.

Also measured (extra keys of the one JSON line):
* the same workload with the oldest 50% of pages in pinned host RAM (host
  link GB/s against the measured pinned H2D copy bandwidth);
* the CPU baseline: HELM's CPU streaming attention restated by the oracle
  (torch CPU, HELM's Path 2 and masked online-softmax loop) on the same
  shape, timed on this host's cores for a bounded sample;
* decode steps/s at 32k = 1 / (36 layers x per-layer call time), for the
  raw C-ABI call and for HELM's production call (``_decode_batched`` under
  its decode mask, wall time per layer call);
* the full 40-layer Qwen3-14B decode step (batch 4 x 65,536 tokens, per layer
  token append + residency policy + attention through the runtime API), with
  the 64 GB device KV budget (nothing evicted) and with a 32 GB budget that
  keeps about 25% of the pages in pinned host RAM;
* a prefill chunk: 512 query tokens over 32,768 cached tokens of one
  Qwen3-8B-shaped layer under the chunk-causal mask, through the runtime's
  prefill path (TFLOP/s against the matrix cores' dense bf16 peak);
* HELM's CPU-stage fp16 linear (helm/kernels): one Qwen3-8B layer's
  decode-step GEMVs on this host's cores, the native GEMV beside HELM's own
  AVX2 kernel built from its source and HELM's float32 fallback;
* the headline shape under HELM's decode mask (zeros [1,1,1,T]), the mask
  every production decode step passes;
* the other configurations at their stated shapes: Qwen3-0.6B 2k (fp16),
  Qwen3-14B B8 ragged 4k-32k, Llama-2-13B 128k with 75% of its pages in
  pinned host RAM — time, GB/s, roofline fraction, error against fp64;
* the production decode call (``_decode_batched``: append, residency,
  attention) on the Qwen3-8B 32k shape, masked and unmasked, and the
  40-layer step under the decode mask;
* Qwen3-0.6B 2k on the host CPU path, HELM's CPU-stage attention: the native
  host kernel beside the oracle's restatement of HELM's torch code.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "paged decode-attn KV GB/s (% HBM peak) + decode steps/s at 32k ctx"
HBM_PEAK_GBS = 8000.0
PCIE5_X16_GBS = 63.0
QWEN3_8B_LAYERS = 36


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--pools", type=int, default=8, help="rotated KV pools (MALL hygiene)")
    ap.add_argument("--offload-steps", type=int, default=20)
    ap.add_argument("--offload-idle", type=float, default=0.0, metavar="SECONDS",
                    help="idle this long before the offload leg (after the heavy legs, "
                         "copies that overlap kernels run at half rate for a while)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-offload", action="store_true")
    ap.add_argument("--pps", type=int, default=0, help="pages per split (0 = auto)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 1 GiB device copy (PMC byte-count calibration)")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill-chunk leg")
    ap.add_argument("--no-gemv", action="store_true",
                    help="skip the host-CPU fp16 GEMV leg (HELM's CPU-stage linears)")
    ap.add_argument("--no-full-step", action="store_true",
                    help="skip the 40-layer Qwen3-14B B4 x 64k decode step (64 GB device KV "
                         "budget, and a 32 GB budget that forces eviction)")
    ap.add_argument("--full-step-steps", type=int, default=64)
    ap.add_argument("--full-step-budgets", default="64,32",
                    help="device KV budgets (GB) of the full-step runs")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the qwen3-0.6b / qwen3-14b ragged / llama2-13b 128k legs")
    ap.add_argument("--no-runtime", action="store_true",
                    help="skip the _decode_batched production-call leg")
    ap.add_argument("--all", action="store_true",
                    help="also measure every benchmark configuration (one line each on stderr)")
    ap.add_argument("--stamps", action="store_true",
                    help="also record per-workgroup start / page-loop-end / end times of the "
                         "headline decode kernel (helm_profile_workgroup_stamps)")
    ap.add_argument("--read-probe", action="store_true",
                    help="also time a kernel that only reads the headline call's K/V bytes "
                         "(with and without a merge-sized second kernel): the call's floor")
    ap.add_argument("--all-json", default=None, metavar="PATH",
                    help="with --all, also write the configurations' rows to PATH as JSON")
    return ap.parse_args()


def split_kernel_us(torch, step, steps):
    """HIP-event durations (us) of the attention (split) kernel of `steps`
    calls of `step`, the split merge after it excluded: start / stop events
    attached to that launch (helm_profile_split_kernels).  Mean, median and
    the 90th percentile and maximum."""
    from helm_amd import _native
    lib = _native.load()
    _native.call("helm_profile_split_kernels", steps)
    try:
        for i in range(steps):
            step(i)
        torch.cuda.synchronize()
        buf = np.zeros(steps, dtype=np.float32)
        n = lib.helm_profile_split_read(_native.ptr(buf), steps)
        if n != steps:
            raise RuntimeError(f"split-kernel timing read {n} of {steps} calls: "
                               f"{_native.load().helm_last_error_string()}")
    finally:
        _native.call("helm_profile_split_kernels", 0)
    return (float(buf.mean()), float(np.median(buf)), float(np.percentile(buf, 90)),
            float(buf.max()))


def gpu_headline(args, torch, W, paged, name="qwen3-8b-32k", seed=1, n_pools=None, steps=None,
                 masked=False, kernel_timing=False):
    """Pool-layout decode attention of one workload, all pages resident.
    Pools are rotated so that at least 1 GiB of KV passes between two reads
    of the same pool (the 256 MB Infinity Cache cannot serve it).  masked:
    HELM's decode mask, zeros [B, 1, 1, T] (pipeline_runtime.py:79-92), the
    mask every production decode step passes."""
    w = W.WORKLOADS[name]
    dev = torch.device("cuda:0")
    case = W.make_pool_case(w, seed=seed, device=dev)
    if n_pools is None:
        pool_b = case["pool"].numel() * case["pool"].element_size()
        n_pools = max(args.pools, min(128, -(-(1 << 30) // pool_b)))
    pools = [case["pool"]] + [torch.empty_like(case["pool"]).copy_(case["pool"])
                              for _ in range(n_pools - 1)]
    lens = case["lens_list"]
    alg = W.algorithmic_bytes(w, lens)
    # argument list built once: a step is one C-ABI call (decode kernel +
    # split merge) on torch's current stream, over the next rotated pool
    mask = (torch.zeros(w.B, 1, 1, max(lens), device=dev) if masked else None)
    prep = paged.prepare_paged_decode(case["q"], case["k_pool"], case["v_pool"], case["table"],
                                      case["lens"], max_pages=case["max_pages"],
                                      total_pages=sum(case["n_pages"]), pages_per_split=args.pps,
                                      attention_mask=mask, host_lens=lens)
    views = [(p[:, 0], p[:, 1]) for p in pools]

    def step(i):
        prep.run(*views[i % len(views)])

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    steps = steps or args.steps
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        step(i)
    t_issued = time.perf_counter()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_events = e0.elapsed_time(e1)
    per_call_s = ms_events / 1e3 / steps
    # a second pass of the same calls, the attention kernel timed alone
    kern = split_kernel_us(torch, step, steps) if kernel_timing else (None,) * 4
    return {
        "split_kernel_us_mean": kern[0], "split_kernel_us_median": kern[1],
        "split_kernel_us_p90": kern[2], "split_kernel_us_max": kern[3],
        "w": w, "case": case, "alg_bytes": alg, "kv_bytes": W.kv_bytes(w, lens),
        "per_call_s": per_call_s, "wall_ms_per_step": wall * 1e3 / steps,
        "host_issue_us_per_call": (t_issued - t0) * 1e6 / steps,
        "ms_per_step": ms_events / steps, "pools": n_pools, "lens": lens, "prep": prep,
        "step": step, "pool_tensors": pools,
    }


def read_pass_floor(torch, h, iters=200):
    """The headline call's floor (helm_profile_read_pass): a kernel that only
    streams the call's K/V bytes out of the same rotated pools, at 256 to 2048
    workgroups, alone and followed by a 32-workgroup kernel reading the
    split merge's 0.53 MB of partials (the two launches of a call)."""
    from helm_amd import _native
    pools = h["pool_tensors"]
    kv = h["kv_bytes"]
    if any(p.numel() * p.element_size() < kv for p in pools):
        raise RuntimeError("read-pass probe: a pool holds fewer bytes than the call reads")
    ptrs = np.array([p.data_ptr() for p in pools], dtype=np.uint64)
    stream = torch.cuda.current_stream().cuda_stream
    tail = 32 * 4 * 8 * 130 * 4          # splits x rows x KV heads x (D + 2) x fp32
    out = {"kv_bytes": kv, "tail_bytes": tail, "iters": iters}
    us = np.zeros(1, dtype=np.float32)
    for wg in (256, 512, 1024, 2048):
        row = {}
        for label, tb, twg in (("read", 0, 0), ("read_then_tail", tail, 32)):
            _native.call("helm_profile_read_pass", _native.ptr(ptrs), len(pools), kv, wg, tb,
                         twg, iters, stream, _native.ptr(us))
            row[label + "_us"] = round(float(us[0]), 3)
        row["read_GBs"] = round(kv / (row["read_us"] * 1e-6) / 1e9, 1)
        out[f"workgroups_{wg}"] = row
    out["how"] = ("helm_profile_read_pass over the headline's rotated pools: each pass reads "
                  "the call's K/V bytes (each workgroup a contiguous run; 16-byte "
                  "non-temporal loads, 8 in flight per thread), "
                  "alone and followed by a 32-workgroup kernel reading the merge's partial "
                  "bytes; HIP events around the passes")
    return out


def workgroup_stamps(torch, h, captures=5, run=40):
    """Per-workgroup timing of the decode kernel (helm_profile_workgroup_stamps):
    in each of `captures` runs of `run` back-to-back calls, the middle call's
    workgroups record the s_memrealtime counter (100 MHz) at their start,
    after their page loop and at their end, with their XCD and CU.  Returns
    the spread of those times (us from the kernel's first workgroup start)
    and their means per XCD and per KV head."""
    from helm_amd import _native
    step = h["step"]
    nwg = 1 << 16
    buf = torch.zeros(nwg * 4, dtype=torch.int64, device="cuda")
    caps = []
    for c in range(captures):
        for i in range(run // 2):
            step(i)
        _native.call("helm_profile_workgroup_stamps", buf.data_ptr(), nwg)
        for i in range(run // 2, run):
            step(i)
        torch.cuda.synchronize()
        _native.call("helm_profile_workgroup_stamps", None, 0)
        a = buf.view(-1, 4).cpu().numpy().astype(np.uint64)
        used = a[:, 0] > 0
        a = a[used]
        buf.zero_()
        t0 = a[:, 0].min()
        rel = (a[:, :3] - t0).astype(np.float64) / 100.0           # 100 MHz -> us
        xcd = (a[:, 3] >> np.uint64(32)).astype(np.int64)
        hw = (a[:, 3] & np.uint64(0xffffffff)).astype(np.int64)
        caps.append((rel, xcd, hw))
    rel, xcd, hw = caps[-1]
    n = len(rel)
    splits = n // max(1, h["w"].Hkv)
    head = np.arange(n) // splits                               # grid (split, head)
    loop = np.stack([c[0][:, 1] for c in caps])                 # [captures, wg]
    end = np.stack([c[0][:, 2] for c in caps])
    start = np.stack([c[0][:, 0] for c in caps])

    def stats(x):
        return {"min": round(float(x.min()), 2), "mean": round(float(x.mean()), 2),
                "max": round(float(x.max()), 2), "std": round(float(x.std()), 2)}

    # does a workgroup's lateness repeat from call to call (a slow place) or not
    lo = loop - loop.mean(axis=1, keepdims=True)
    repeat = float(np.corrcoef(lo[:-1].ravel(), lo[1:].ravel())[0, 1]) if captures > 1 else None
    return {
        "workgroups": n, "captures": captures,
        "start_us": stats(start), "loop_end_us": stats(loop), "end_us": stats(end),
        "loop_end_spread_us_per_capture": [round(float(r.max() - r.min()), 2) for r in loop],
        "last_end_us_per_capture": [round(float(r.max()), 2) for r in end],
        "loop_end_mean_per_xcd_us": {int(x): round(float(loop[-1][xcd == x].mean()), 2)
                                     for x in sorted(set(xcd.tolist()))},
        "loop_end_mean_per_kv_head_us": {int(k): round(float(loop[-1][head == k].mean()), 2)
                                         for k in sorted(set(head.tolist()))},
        "lateness_correlation_between_calls": None if repeat is None else round(repeat, 3),
        "how": "helm_profile_workgroup_stamps: s_memrealtime (100 MHz) at each workgroup's "
               "start, after its page loop (all waves), and at its end, relative to the "
               f"first start; middle call of {run} back-to-back calls, {captures} captures",
    }


def h2d_peak(torch):
    """Pinned host -> device copy bandwidth (256 MiB, best of 5)."""
    n = 256 << 20
    src = torch.empty(n, dtype=torch.uint8).pin_memory()
    dst = torch.empty(n, dtype=torch.uint8, device="cuda")
    best = 0.0
    for _ in range(6):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        dst.copy_(src, non_blocking=True)
        e1.record()
        torch.cuda.synchronize()
        best = max(best, n / (e0.elapsed_time(e1) / 1e3) / 1e9)
    return best


def gpu_offload(args, torch, W, name="qwen3-8b-32k-offload50", seed=2, steps=None,
                check_heads=None):
    """The oldest offload_frac of the context in pinned host pages, streamed
    through the engine's staging ring while the resident pages are attended."""
    from helm_amd import _native
    from helm_amd.runtime import engine
    w = W.WORKLOADS[name]
    dev = torch.device("cuda:0")
    case = W.make_pool_case(w, seed=seed, device=dev)
    n = case["n_pages"][0]
    n_host = int(n * w.offload_frac)
    es = torch.tensor([], dtype=w.dtype).element_size()
    slot_b = 2 * w.Hkv * w.page_size * w.D * es
    kcode = _native.dtype_code(w.dtype)
    host = torch.empty((n_host, 2, w.Hkv, w.page_size, w.D), dtype=w.dtype).pin_memory()
    table = case["table_cpu"][0, :n].long()
    eng = engine.get_engine(dev)
    # the host pages are written as the runtime evicts them: one engine
    # eviction (device -> pinned host), which the side-stream staging copies
    # are ordered after by its event
    cold = case["pool"][table[:n_host].to(dev)].contiguous()
    reg = [np.array([x], dtype=np.uint64)
           for x in (cold.data_ptr(), host.data_ptr(), cold.numel() * cold.element_size())]
    _native.call("helm_evict_pages", eng, 1, _native.ptr(reg[0]), _native.ptr(reg[1]),
                 _native.ptr(reg[2]), 1, torch.cuda.current_stream(dev).cuda_stream)
    del cold
    pages = np.zeros(n, dtype=_native.PAGE_DTYPE)
    for j in range(n):
        if j < n_host:
            base = host.data_ptr() + j * slot_b
            flags = _native.HELM_PAGE_HOST
        else:
            base = case["pool"].data_ptr() + int(table[j]) * slot_b
            flags = 0
        pages[j] = (base, base + slot_b // 2, w.page_size, j * w.page_size,
                    w.page_size * w.D, flags)
    seq_off = np.array([0, n], dtype=np.int32)
    out = torch.empty_like(case["q"])
    stream = torch.cuda.current_stream(dev)

    def call():
        _native.call("helm_stream_attn", eng, case["q"].data_ptr(), out.data_ptr(), 1, w.Hq,
                     w.Hkv, 1, w.D, _native.ptr(pages), _native.ptr(seq_off), case["scale"], 0.0,
                     None, 0, 0, 0, _native.HELM_F32, 0, kcode, kcode, stream.cuda_stream)

    steps = steps or args.offload_steps

    host_calls = {}

    def timed(label, **env):
        """Seconds per call under `env` (engine switches, read per call): the
        best of three timed runs, so that a rare host stall of a few
        milliseconds in one run does not stand for the steady state.  The
        host time of each call of every run (issue, including any wait
        inside it) is kept under `label`."""
        saved = {k: os.environ.pop(k, None)
                 for k in ("HELM_AMD_HOST_READ", "HELM_AMD_STAGE_STREAM", "HELM_AMD_SIDE_AHEAD")}
        os.environ.update(env)
        try:
            for _ in range(3):
                call()
            torch.cuda.synchronize()
            best = None
            host = []
            for _ in range(3):
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(steps):
                    h0 = time.perf_counter()
                    call()
                    host.append((time.perf_counter() - h0) * 1e6)
                e1.record(stream)
                torch.cuda.synchronize()
                t = e0.elapsed_time(e1) / 1e3 / steps
                best = t if best is None else min(best, t)
            host.sort()
            host_calls[label] = {"median": round(host[len(host) // 2], 1),
                                 "p90": round(host[(9 * len(host)) // 10], 1),
                                 "max": round(host[-1], 1),
                                 "over_5ms": sum(h > 5000 for h in host), "calls": len(host)}
            return best
        finally:
            for k in env:
                os.environ.pop(k, None)
            os.environ.update({k: v for k, v in saved.items() if v is not None})

    # host pages staged through the device ring by hipMemcpyAsync (copies on
    # the engine's side stream, which wait only for the eviction and for the
    # earlier readers of their ring slots, overlapped with the device pages'
    # launch and the earlier calls' kernels, the host at most two calls ahead,
    # or with no bound on that; or on the caller's stream after
    # the device pages' launch), read in place by the kernel over the
    # host link, and the engine's default (per call: pages in long address
    # runs are staged, copies on the caller's stream)
    per_staged = timed("staged", HELM_AMD_HOST_READ="copy")
    per_side = timed("staged_side_stream", HELM_AMD_HOST_READ="copy", HELM_AMD_STAGE_STREAM="side")
    # the same without the engine's bound on how far the host queues ahead
    per_side_unb = timed("staged_side_stream_unbounded", HELM_AMD_HOST_READ="copy",
                         HELM_AMD_STAGE_STREAM="side", HELM_AMD_SIDE_AHEAD="0")
    per_one = timed("staged_one_stream", HELM_AMD_HOST_READ="copy", HELM_AMD_STAGE_STREAM="one")
    per_direct = timed("in_place", HELM_AMD_HOST_READ="direct")
    per = timed("default")
    host_bytes = n_host * slot_b
    peak = h2d_peak(torch)
    # parity spot check of this exact configuration against the oracle
    from oracle.attention import attention_fp64_batched
    err = 0.0
    for kvh in (check_heads if check_heads is not None else range(w.Hkv)):
        K = case["pool"][table.to(dev), 0, kvh].reshape(-1, w.D)[None].cpu()
        V = case["pool"][table.to(dev), 1, kvh].reshape(-1, w.D)[None].cpu()
        hs = slice(kvh * w.G, (kvh + 1) * w.G)
        ref = attention_fp64_batched(case["q"][0, hs].cpu(), K, V)
        err = max(err, (out[0, hs].double().cpu() - ref).abs().max().item())
    return {
        "host_pages": n_host, "host_bytes": host_bytes, "ms_per_call": per * 1e3,
        "host_link_GBs": host_bytes / per / 1e9, "measured_h2d_GBs": peak,
        "frac_of_measured_h2d": host_bytes / per / 1e9 / peak,
        "pcie5_x16_theoretical_GBs": PCIE5_X16_GBS, "max_abs_err_vs_fp64": err,
        "resident_bytes": (n - n_host) * slot_b,
        "host_read": "engine default (staged when the host pages form long address runs, "
                     "else read in place; staging copies on the caller's stream)",
        "staged_ms_per_call": per_staged * 1e3,
        "staged_host_link_GBs": host_bytes / per_staged / 1e9,
        "staged_side_stream_ms_per_call": per_side * 1e3,
        "staged_side_stream_frac_of_measured_h2d": host_bytes / per_side / 1e9 / peak,
        "staged_side_stream_unbounded_ms_per_call": per_side_unb * 1e3,
        "staged_one_stream_ms_per_call": per_one * 1e3,
        "timing": f"best of 3 runs of {steps} calls after 3 warm-up calls",
        "in_place_ms_per_call": per_direct * 1e3,
        "in_place_host_link_GBs": host_bytes / per_direct / 1e9,
        "host_us_per_call": host_calls,
        "host_us_per_call_how": "host time of each helm_stream_attn call (issue and any wait "
                                "inside the HIP runtime), over the 3 timed runs of each mode",
    }


def gpu_full_step(args, torch, W, budget_gb, steps, name="qwen3-14b-40l-b4-64k", seed=5,
                  masked_steps=0):
    """The 40-layer Qwen3-14B decode step through HELM's runtime API.

    Four sequences of 65,536 tokens per layer in 16-token pages taken from a
    seeded shuffle of the free list, one KVCacheManager per sequence sharing
    one KVAllocator, the device KV budget split evenly over the sequences (as
    KVOffloadManager does, kv_offload.py:683-688).  A step runs, for each of
    the 40 layers, ``_decode_batched``: append each sequence's new token (a
    fresh page every 16 tokens), enforce the residency watermark (evicting the
    oldest full pages to pinned host RAM when over budget), and attend over
    every page (host pages streamed back through the staging ring).  Then
    `masked_steps` more steps under the pipeline's decode mask, zeros
    [B, 1, 1, T] (pipeline_runtime.py:79-92, :217): HELM's production path.
    """
    import random
    from helm_amd.runtime import kv_cache as KC
    from helm_amd.runtime.kv_allocator import KVAllocator
    from helm_amd.runtime.kv_cache import KVCacheManager
    from helm_amd.runtime.kv_offload import _decode_batched
    w = W.WORKLOADS[name]
    dev = torch.device("cuda:0")
    P, L, B = w.page_size, w.layers, w.B
    per_item = int(budget_gb * 1e9) // B
    alloc = KVAllocator(L, w.Hkv, w.D, page_size=P, dtype=w.dtype)
    n_pages = L * B * (w.T // P + steps // P + 2)
    t_setup = time.perf_counter()
    alloc.reserve_batch(n_pages, dev)
    random.Random(seed).shuffle(alloc.gpu_free_pool)
    kvcms = [KVCacheManager(alloc, gpu_high_watermark_bytes=per_item) for _ in range(B)]
    for m in kvcms:
        m.initialize_layer_caches(L)
    KC.reset_paging_stats()
    g = torch.Generator(device=dev).manual_seed(seed)
    for layer in range(L):
        for m in kvcms:
            k = torch.randn((1, w.Hkv, w.T, w.D), generator=g, device=dev, dtype=w.dtype)
            v = torch.randn((1, w.Hkv, w.T, w.D), generator=g, device=dev, dtype=w.dtype)
            m.append_prefill(layer, k, v)
            del k, v
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup
    prefill_stats = KC.get_paging_stats()
    q = torch.randn((L, B, w.Hq, 1, w.D), generator=g, device=dev, dtype=w.dtype)
    kn = torch.randn((L, B, w.Hkv, 1, w.D), generator=g, device=dev, dtype=w.dtype)
    vn = torch.randn((L, B, w.Hkv, 1, w.D), generator=g, device=dev, dtype=w.dtype)
    scale = 1.0 / math.sqrt(w.D)
    warmup = 2
    for s in range(warmup):
        for layer in range(L):
            _decode_batched(kvcms, q[layer], kn[layer], vn[layer], layer, scale)
    KC.reset_paging_stats()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    out = None
    for s in range(steps):
        for layer in range(L):
            out = _decode_batched(kvcms, q[layer], kn[layer], vn[layer], layer, scale)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_s = e0.elapsed_time(e1) / 1e3
    stats = KC.get_paging_stats()
    masked = None
    if masked_steps:
        torch.cuda.synchronize()
        tm = time.perf_counter()
        for s in range(masked_steps):
            # HELM's decode mask: built once per step in the model's dtype and
            # handed to every layer (pipeline_runtime.py:79-92, :217)
            mask = torch.zeros((B, 1, 1, kvcms[0].layers[0].total_tokens + 1), device=dev,
                               dtype=w.dtype)
            for layer in range(L):
                out = _decode_batched(kvcms, q[layer], kn[layer], vn[layer], layer, scale, mask)
        torch.cuda.synchronize()
        wm = time.perf_counter() - tm
        ctx_m = w.T + warmup + steps + masked_steps
        kv_m = L * B * (ctx_m - (masked_steps - 1) / 2) * w.token_bytes()
        masked = {"steps": masked_steps, "steps_per_s": masked_steps / wm,
                  "ms_per_step": wm * 1e3 / masked_steps, "kv_GBs": kv_m * masked_steps / wm / 1e9,
                  "mask": "zeros [B, 1, 1, T] in bf16, built once per step and passed to "
                          "every layer (HELM's decode mask)"}
    # spot check: the last layer's output of the last step against the oracle
    from oracle.attention import attention_fp64_batched
    pages = kvcms[0].layers[L - 1].pages
    K = torch.cat([p.k_tensor[0, :, :p.used_tokens].cpu() for p in pages], 1)
    V = torch.cat([p.v_tensor[0, :, :p.used_tokens].cpu() for p in pages], 1)
    ref = attention_fp64_batched(q[L - 1, 0].cpu(), K, V)
    err = (out[0].double().cpu() - ref).abs().max().item()
    ctx = w.T + warmup + steps + masked_steps
    # KV read per step: the mean context over the timed steps
    kv_step = L * B * (w.T + warmup + steps - (steps - 1) / 2) * w.token_bytes()
    host_pages = sum(layer._n_host for m in kvcms for layer in m.layers.values())
    res = {
        "workload": f"{name}: 40 layers x (append + decode attention), B={B}, Hq={w.Hq}, "
                    f"Hkv={w.Hkv}, D={w.D}, bf16, {w.T} tokens per sequence in pages of {P}",
        "device_kv_budget_GB": budget_gb, "steps": steps, "warmup_steps": warmup,
        "context_at_end": ctx,
        "steps_per_s": steps / wall, "ms_per_step": wall * 1e3 / steps,
        "gpu_ms_per_step": gpu_s * 1e3 / steps,
        "kv_GBs": kv_step * steps / wall / 1e9,
        "host_pages_at_end": host_pages,
        "host_frac_at_end": host_pages / (L * B * -(-ctx // P)),
        "evicted_in_setup": prefill_stats["pages_evicted"],
        "paging_stats_timed": stats,
        "setup_s": setup_s, "max_abs_err_vs_fp64": err,
        "masked_production_decode": masked,
    }
    del kvcms, alloc, q, kn, vn, out
    torch.cuda.empty_cache()
    return res


def gpu_prefill(args, torch, T=32768, S=512, reps=20, seed=6):
    """A prefill chunk through the runtime: Qwen3-8B attention shape (32 query /
    8 KV heads, head_dim 128, bf16, pages of 16), an S-token chunk attending
    over the T tokens of its layer's pages (the chunk's own K/V appended last)
    under the additive chunk-causal mask HELM's pipeline passes
    (pipeline_runtime.py:94-113), via ``_stream_prefill_batched``
    (kv_offload.py:207-227).  Roofline: the matrix cores (4 Hq S T D flops)."""
    from helm_amd.runtime.kv_allocator import KVAllocator
    from helm_amd.runtime.kv_cache import KVCacheManager
    from helm_amd.runtime.kv_offload import _stream_prefill_batched
    from oracle.attention import attention_fp64_batched
    Hq, Hkv, D, P = 32, 8, 128, 16
    dev = torch.device("cuda:0")
    a = KVAllocator(1, Hkv, D, page_size=P, dtype=torch.bfloat16)
    m = KVCacheManager(a, gpu_high_watermark_bytes=10 ** 13)
    g = torch.Generator(device=dev).manual_seed(seed)
    k = torch.randn(1, Hkv, T, D, generator=g, device=dev).bfloat16()
    v = torch.randn(1, Hkv, T, D, generator=g, device=dev).bfloat16()
    m.append_prefill(0, k, v)
    q = torch.randn(1, Hq, S, D, generator=g, device=dev).bfloat16()
    mask = torch.zeros(1, 1, S, T, device=dev)
    lim = T - S + torch.arange(S, device=dev)
    mask[0, 0][torch.arange(T, device=dev)[None, :] > lim[:, None]] = torch.finfo(torch.float32).min
    scale = 1.0 / math.sqrt(D)
    run = lambda: _stream_prefill_batched([m], q, 0, scale, attention_mask=mask)
    out = run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        out = run()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / reps
    flops = 4.0 * Hq * S * T * D
    # spot check: KV head 0's four query heads at 64 chunk positions
    rows = torch.arange(0, S, S // 64)
    ref = attention_fp64_batched(q[0, :4, rows].cpu(), k[0, :1].cpu(), v[0, :1].cpu(),
                                 mask=mask[0, :, rows].double().cpu())
    err = (out[0, :4, rows].double().cpu() - ref).abs().max().item()
    res = {"workload": f"qwen3-8b attention shape, 1 layer: {S}-token chunk over {T} cached "
                       f"tokens (pages of {P}), bf16, additive chunk-causal mask [1,1,{S},{T}] "
                       f"(recognised as causal masking at offset {T - S}: no mask reads)",
           "ms_per_call": dt * 1e3, "TFLOPs": flops / dt / 1e12,
           "mfma_peak_TFLOPs": 2500.0, "frac_of_peak": flops / dt / 1e12 / 2500.0,
           "calls": reps, "max_abs_err_vs_fp64": err}
    del m, a, k, v, q, mask, out
    torch.cuda.empty_cache()
    return res


def all_configs(args, torch, W, paged):
    """Every decode-attention configuration of the benchmark set, one line
    each on stderr and, with --all-json PATH, all of them in PATH."""
    rows = []
    for name, seed in (("qwen3-0.6b-2k", 0), ("qwen3-8b-32k", 1), ("qwen3-14b-ragged-b8", 3)):
        h = gpu_headline(args, torch, W, paged, name=name, seed=seed, steps=100)
        gbs = h["alg_bytes"] / h["per_call_s"] / 1e9
        r = {"workload": name, "us_per_call": h["per_call_s"] * 1e6, "GBs": gbs,
             "hbm_frac": gbs / HBM_PEAK_GBS, "alg_bytes": h["alg_bytes"], "pools": h["pools"],
             "total_tokens": sum(h["lens"])}
        rows.append(r)
        log(json.dumps(r))
        del h
        torch.cuda.empty_cache()
    for name, seed in (("qwen3-8b-32k-offload50", 2), ("llama2-13b-128k-offload75", 4)):
        o = gpu_offload(args, torch, W, name=name, seed=seed, steps=10)
        o["workload"] = name
        rows.append(o)
        log(json.dumps(o))
        torch.cuda.empty_cache()
    if args.all_json:
        os.makedirs(os.path.dirname(os.path.abspath(args.all_json)), exist_ok=True)
        with open(args.all_json, "w") as f:
            json.dump(rows, f, indent=1)
    return rows


def pool_error(torch, h, heads):
    """max |out - fp64| of a pool-layout leg's last call (all pools hold the
    same data), over the query heads of the given KV heads of every sequence."""
    from oracle.attention import attention_fp64_batched
    w, case, out = h["w"], h["case"], h["prep"].out
    G = w.Hq // w.Hkv
    worst = 0.0
    for b, t in enumerate(case["lens_list"]):
        n = case["n_pages"][b]
        slots = case["table_cpu"][b, :n].long().to(case["pool"].device)
        for kvh in heads:
            K = case["pool"][slots, 0, kvh].reshape(-1, w.D)[:t][None].cpu()
            V = case["pool"][slots, 1, kvh].reshape(-1, w.D)[:t][None].cpu()
            hs = slice(kvh * G, (kvh + 1) * G)
            ref = attention_fp64_batched(case["q"][b, hs].cpu(), K, V)
            worst = max(worst, (out[b, hs].double().cpu() - ref).abs().max().item())
    return worst


def gpu_records_decode(torch, W, h, steps=100):
    """The pool leg's batch (`h`, same data) through helm_paged_attn_seqs, the
    entry point _decode_batched takes for a batch whose pages are all on the
    device (kv_offload.py:152-174): one device-resident helm_page record
    array per sequence, the grid numbering exactly the sequences' splits (the
    pool entry point's grid also holds workgroups that find no split of a
    short sequence).  The same number of pool copies rotated, HIP events
    around `steps` calls; max |error| against fp64 on the first and last KV
    heads of every sequence."""
    from helm_amd import _native
    from helm_amd.runtime import engine
    from oracle.attention import attention_fp64_batched
    w, case = h["w"], h["case"]
    dev = case["q"].device
    pool0 = case["pool"]
    pools = [pool0] + [torch.empty_like(pool0).copy_(pool0) for _ in range(h["pools"] - 1)]
    P, es = w.page_size, pool0.element_size()
    lens = case["lens_list"]
    keep, sets = [], []
    for pool in pools:
        ptrs = []
        for b, n in enumerate(case["n_pages"]):
            slots = case["table_cpu"][b, :n].numpy().astype(np.uint64)
            rec = np.zeros(n, dtype=_native.PAGE_DTYPE)
            rec["k"] = pool.data_ptr() + slots * np.uint64(pool.stride(0) * es)
            rec["v"] = rec["k"] + np.uint64(pool.stride(1) * es)
            rec["used"] = P                      # the kernel caps by seq_tokens
            rec["tok_off"] = np.arange(n, dtype=np.int32) * P
            rec["head_stride"] = pool.stride(2)
            t = torch.from_numpy(rec.view(np.uint8).copy()).to(dev)
            keep.append(t)
            ptrs.append(t.data_ptr())
        sets.append(np.array(ptrs, dtype=np.uint64))
    npages = np.array(case["n_pages"], dtype=np.int32)
    tokens = np.array(lens, dtype=np.int32)
    eng = engine.get_engine(dev)
    stream = torch.cuda.current_stream(dev)
    out = torch.empty_like(case["q"])
    kcode = _native.dtype_code(w.dtype)
    fn = _native.load().helm_paged_attn_seqs
    args_of = [(eng, case["q"].data_ptr(), out.data_ptr(), w.B, w.Hq, w.Hkv, 1, w.D,
                _native.ptr(st), _native.ptr(npages), _native.ptr(tokens), P, 1,
                case["scale"], 0.0, None, 0, 0, 0, _native.HELM_F32, 0, kcode, kcode,
                stream.cuda_stream)
               for st in sets]

    def call(i):
        rc = fn(*args_of[i % len(args_of)])
        if rc:
            _native.check("helm_paged_attn_seqs", rc)

    for i in range(10):
        call(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(steps):
        call(i)
    e1.record(stream)
    torch.cuda.synchronize()
    per = e0.elapsed_time(e1) / 1e3 / steps
    G = w.Hq // w.Hkv
    worst = 0.0
    for b, t in enumerate(lens):
        slots = case["table_cpu"][b, :case["n_pages"][b]].long().to(dev)
        for kvh in (0, w.Hkv - 1):
            K = pool0[slots, 0, kvh].reshape(-1, w.D)[:t][None].cpu()
            V = pool0[slots, 1, kvh].reshape(-1, w.D)[:t][None].cpu()
            hs = slice(kvh * G, (kvh + 1) * G)
            ref = attention_fp64_batched(case["q"][b, hs].cpu(), K, V)
            worst = max(worst, (out[b, hs].double().cpu() - ref).abs().max().item())
    gbs = h["alg_bytes"] / per / 1e9
    del pools, keep
    return {"entry": "helm_paged_attn_seqs (device-resident page records per sequence, the "
                     "batched decode of _decode_batched)",
            "us_per_call": round(per * 1e6, 3), "GBs": round(gbs, 1),
            "roofline_frac": round(gbs / HBM_PEAK_GBS, 4), "max_abs_err_vs_fp64": worst}


def gpu_configs(args, torch, W, paged):
    """The other configurations of the benchmark set, each at its stated
    shape: Qwen3-0.6B 2k (fp16) and Qwen3-14B B8 ragged 4k-32k (bf16) through
    the pool-layout decode call (rotated pools), Llama-2-13B 128k (fp16, MHA)
    with its oldest 75% of pages in pinned host memory through
    helm_stream_attn; per-call time, GB/s, roofline fraction, max |error|
    against the fp64 oracle."""
    res = {}
    for name, seed, tol in (("qwen3-0.6b-2k", 0, 2e-3), ("qwen3-14b-ragged-b8", 3, 1e-2)):
        h = gpu_headline(args, torch, W, paged, name=name, seed=seed, steps=100)
        gbs = h["alg_bytes"] / h["per_call_s"] / 1e9
        w = h["w"]
        res[name] = {
            "workload": f"{name}: B={w.B}, Hq={w.Hq}, Hkv={w.Hkv}, D={w.D}, "
                        f"{str(w.dtype).split('.')[-1]}, contexts {h['lens']}, pages of 16, "
                        f"all resident, {h['pools']} rotated pools",
            "us_per_call": round(h["per_call_s"] * 1e6, 3), "GBs": round(gbs, 1),
            "roofline_frac": round(gbs / HBM_PEAK_GBS, 4), "alg_bytes": h["alg_bytes"],
            "max_abs_err_vs_fp64": pool_error(torch, h, [0, w.Hkv - 1]), "tolerance": tol}
        if w.B > 1:
            res[name]["records_entry"] = gpu_records_decode(torch, W, h)
        log(json.dumps(res[name]))
        del h
        torch.cuda.empty_cache()
    o = gpu_offload(args, torch, W, name="llama2-13b-128k-offload75", seed=4, steps=5,
                    check_heads=[0, 13, 27, 39])
    o["workload"] = ("llama2-13b-128k-offload75: B=1, Hq=Hkv=40, D=128, fp16, 131072 tokens "
                     "in 8192 pages, oldest 75% in pinned host")
    o["tolerance"] = 2e-3
    res["llama2-13b-128k-offload75"] = o
    log(json.dumps(o))
    torch.cuda.empty_cache()
    return res


def gpu_runtime_decode(args, torch, W, layers=8, steps=25, seed=11):
    """HELM's production decode call on the Qwen3-8B 32k shape: the per-layer
    ``_decode_batched`` of the patched forwards (append the token, residency,
    attention over the layer's records) under the pipeline's decode mask,
    zeros [1, 1, 1, T] in bf16 built once per step and handed to every layer
    (pipeline_runtime.py:79-92, :217; its allocation is in the timed steps, as
    in HELM's decode loop), and without a mask for comparison.  Eight layers
    of 32k tokens are rotated (1 GiB of KV, so
    the Infinity Cache cannot serve a layer twice).  Wall time per layer call
    (host issue included) and the GPU time between events around the loop."""
    import random
    from helm_amd.runtime.kv_allocator import KVAllocator
    from helm_amd.runtime.kv_cache import KVCacheManager
    from helm_amd.runtime.kv_offload import _decode_batched
    from oracle.attention import attention_fp64_batched
    w = W.WORKLOADS["qwen3-8b-32k"]
    dev = torch.device("cuda:0")
    P = w.page_size
    a = KVAllocator(layers, w.Hkv, w.D, page_size=P, dtype=w.dtype)
    a.reserve_batch(layers * (w.T // P + (8 * steps + 8) // P + 4), dev)
    random.Random(seed).shuffle(a.gpu_free_pool)
    m = KVCacheManager(a, gpu_high_watermark_bytes=10 ** 13)
    m.initialize_layer_caches(layers)
    g = torch.Generator(device=dev).manual_seed(seed)
    for lid in range(layers):
        m.append_prefill(lid, torch.randn((1, w.Hkv, w.T, w.D), generator=g, device=dev,
                                          dtype=w.dtype),
                         torch.randn((1, w.Hkv, w.T, w.D), generator=g, device=dev,
                                     dtype=w.dtype))
    q = torch.randn((layers, 1, w.Hq, 1, w.D), generator=g, device=dev, dtype=w.dtype)
    kn = torch.randn((layers, 1, w.Hkv, 1, w.D), generator=g, device=dev, dtype=w.dtype)
    vn = torch.randn((layers, 1, w.Hkv, 1, w.D), generator=g, device=dev, dtype=w.dtype)
    scale = 1.0 / math.sqrt(w.D)
    stream = torch.cuda.current_stream(dev)
    out = None

    def run(n, masked):
        nonlocal out
        for _ in range(n):
            # HELM's decode mask: one per step in the model's dtype, handed to
            # every layer (pipeline_runtime.py:79-92, :217)
            mask = (torch.zeros((1, 1, 1, m.layers[0].total_tokens + 1), device=dev,
                                dtype=w.dtype) if masked else None)
            for lid in range(layers):
                out = _decode_batched([m], q[lid], kn[lid], vn[lid], lid, scale, mask)

    res = {"workload": f"qwen3-8b-32k through _decode_batched: {layers} layers of {w.T} "
                       "tokens rotated, B=1, bf16, one call per layer per step",
           "timing": f"median of 3 runs of {steps} steps per label, masked and unmasked runs "
                     "interleaved, after 3 warm-up steps of each"}
    runs = {"masked": [], "unmasked": []}
    for label, masked in (("masked", True), ("unmasked", False)):
        run(3, masked)
    for _ in range(3):
        for label, masked in (("masked", True), ("unmasked", False)):
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            e0.record(stream)
            run(steps, masked)
            e1.record(stream)
            t_issue = time.perf_counter() - t0
            torch.cuda.synchronize()
            wall = time.perf_counter() - t0
            runs[label].append((wall, e0.elapsed_time(e1) / 1e3, t_issue))
    n = steps * layers
    alg = W.algorithmic_bytes(w, [m.layers[0].total_tokens])
    for label, rr in runs.items():
        wall, gpu, issue = (sorted(x[i] for x in rr)[1] / n for i in range(3))
        res[label] = {"us_per_call_wall": round(wall * 1e6, 2),
                      "us_per_call_gpu_events": round(gpu * 1e6, 2),
                      "us_per_call_host_issue": round(issue * 1e6, 2),
                      "us_per_call_wall_runs": [round(x[0] / n * 1e6, 2) for x in rr],
                      "GBs_wall": round(alg / wall / 1e9, 1),
                      "roofline_frac_wall": round(alg / wall / 1e9 / HBM_PEAK_GBS, 4)}
    # the last call (layer layers-1, unmasked) against the oracle on two KV heads
    lid = layers - 1
    pages = m.layers[lid].pages
    err = 0.0
    for kvh in (0, w.Hkv - 1):
        K = torch.cat([p.k_tensor[0, kvh, :p.used_tokens] for p in pages], 0)[None].cpu()
        V = torch.cat([p.v_tensor[0, kvh, :p.used_tokens] for p in pages], 0)[None].cpu()
        hs = slice(kvh * w.G, (kvh + 1) * w.G)
        ref = attention_fp64_batched(q[lid, 0, hs].cpu(), K, V)
        err = max(err, (out[0, hs].double().cpu() - ref).abs().max().item())
    res["max_abs_err_vs_fp64"] = err
    m.clear()
    del m, a, q, kn, vn
    torch.cuda.empty_cache()
    return res


def cpu_info():
    """The host CPU: model name, logical CPUs this process may use, and the
    physical cores behind them (distinct (package, core) pairs)."""
    model, cores, cur = None, set(), {}
    allowed = os.sched_getaffinity(0)
    try:
        with open("/proc/cpuinfo") as f:
            for line in f.read().splitlines() + [""]:
                if not line.strip():
                    if cur.get("processor") is not None and cur["processor"] in allowed:
                        cores.add((cur.get("physical id"), cur.get("core id", cur["processor"])))
                    cur = {}
                    continue
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model is None:
                    model = v
                if k == "processor":
                    cur["processor"] = int(v)
                elif k in ("physical id", "core id"):
                    cur[k] = v
    except OSError:
        pass
    return {"model": model, "logical_cpus_allowed": len(allowed),
            "physical_cores_allowed": len(cores) or len(allowed)}


def cpu_threads():
    """Threads for the host-CPU legs: one per physical core this process may
    use, at most the OpenMP thread count the machine sets (its CPU share)."""
    info = cpu_info()
    cap = int(os.environ.get("OMP_NUM_THREADS", "16") or 16)
    return max(1, min(info["physical_cores_allowed"], cap)), info


def cpu_c1(args, torch, W, seconds=4.0):
    """Qwen3-0.6B 2k (fp16) on the host CPU path, the path HELM runs a CPU
    stage's attention on: the native host kernel here (libhelm_cpu.so,
    helm_cpu_stream_attn, production decode mask) beside the oracle's
    restatement of HELM's torch code (Path 2, cat + fp32 SDPA; and the masked
    per-page loop), same inputs; bounded samples."""
    from helm_amd.runtime.kv_cache import _attend_records_cpu
    from oracle import attention as A
    threads, info = cpu_threads()
    torch.set_num_threads(threads)
    w = W.WORKLOADS["qwen3-0.6b-2k"]
    case = W.make_pool_case(w, seed=0, device="cpu")
    arr, seq_off = W.pool_records(case, w)
    T = w.T
    mask = torch.zeros(1, 1, 1, T)
    slots = case["table_cpu"][0].long()
    K = case["pool"][slots, 0].permute(1, 0, 2, 3).reshape(w.Hkv, -1, w.D)
    V = case["pool"][slots, 1].permute(1, 0, 2, 3).reshape(w.Hkv, -1, w.D)
    pages = A.split_pages(K[None], V[None], [w.page_size] * (T // w.page_size))
    alg = W.algorithmic_bytes(w, [T])
    legs = {
        "native_host_kernel": lambda: _attend_records_cpu(case["q"], arr, seq_off, T, w.Hkv,
                                                          w.dtype, case["scale"], mask, None, 0),
        "oracle_path2_concat_sdpa": lambda: A.concat_sdpa(case["q"], pages),
        "oracle_masked_online_softmax": lambda: A.online_softmax_pages(case["q"], pages,
                                                                       attention_mask=mask),
    }
    res = {"workload": "qwen3-0.6b-2k: B=1, Hq=16, Hkv=8, D=128, fp16, 2048 tokens in 128 "
                       "pages of 16 (random page table), on the host CPU",
           "threads": threads, "cpu": info}
    outs = {}
    for name, fn in legs.items():
        outs[name] = fn()
        t0, calls = time.perf_counter(), 0
        while True:
            fn()
            calls += 1
            if time.perf_counter() - t0 > seconds / 3:
                break
        per = (time.perf_counter() - t0) / calls
        res[name] = {"us_per_call": round(per * 1e6, 2), "GBs": round(alg / per / 1e9, 3),
                     "calls": calls}
    ref = A.attention_fp64_batched(case["q"][0].float(), K.float(), V.float())
    res["native_max_abs_err_vs_fp64"] = (outs["native_host_kernel"][0].double() - ref).abs().max().item()
    res["native_speedup_vs_path2"] = round(res["oracle_path2_concat_sdpa"]["us_per_call"]
                                           / res["native_host_kernel"]["us_per_call"], 1)
    return res


# Qwen3-8B decode-step linears of one layer (out x in): q, k, v, o, gate, up, down
GEMV_SHAPES = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (12288, 4096),
               (12288, 4096), (4096, 12288)]


def cpu_gemv(args, torch, reps=10, layers=2, seed=7):
    """HELM's CPU-stage linear (helm/kernels): the decode step's fp16 GEMVs of
    one Qwen3-8B layer (q/k/v/o/gate/up/down, 386 MB of fp16 weights), two
    layers' weights rotated so the host caches cannot hold them, on this
    host's cores.  Timed: the native GEMV here (libhelm_cpu.so); HELM's own
    AVX2 kernel built from its source (oracle/_ref, when present: the CPU
    baseline); HELM's fallback when its kernel is unavailable (F.linear in
    float32, the weight widened every call).  Bound: host DRAM bandwidth
    (bytes = the weights; x and y are cache resident)."""
    from helm_amd import kernels
    threads, _ = cpu_threads()
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(seed)
    Ws = [[(0.02 * torch.randn(n, k, generator=g)).half() for n, k in GEMV_SHAPES]
          for _ in range(layers)]
    xs = {k: torch.randn(1, 1, k, generator=g).half() for _, k in GEMV_SHAPES}
    wbytes = sum(2 * n * k for n, k in GEMV_SHAPES)
    res = {"workload": "qwen3-8b decode-step linears of one layer: q/k/v/o/gate/up/down, "
                       f"fp16 weights {wbytes / 1e6:.0f} MB, batch 1, {layers} layers rotated",
           "threads": threads, "cpu_isa": kernels.isa(), "weight_bytes_per_layer": wbytes}

    def timed(fn, reps):
        for li in range(layers):
            fn(Ws[li])
        t0 = time.perf_counter()
        for r in range(reps):
            fn(Ws[r % layers])
        return (time.perf_counter() - t0) / reps

    try:
        from oracle import build_ref
        ref = build_ref.load()
    except Exception as e:          # a module built for another torch: say so
        ref, res["reference_error"] = None, str(e)
    if ref is not None:
        os.environ.setdefault("OMP_NUM_THREADS", str(threads))
    # the native GEMV and HELM's kernel timed in turn, three rounds, best of
    # each (the host is shared: one back-to-back pair can differ by 1.5x)
    legs = {}
    if kernels.is_available():
        x8 = {k: torch.randn(8, k, generator=g).half() for _, k in GEMV_SHAPES}
        # the product call (HELM's fp16_linear surface), as HELM's leg calls
        # its extension's helm_fp16_linear
        legs["native"] = lambda ws: [kernels.fp16_linear(xs[w.shape[1]], w) for w in ws]
        legs["native_8_tokens"] = lambda ws: [kernels.fp16_linear(x8[w.shape[1]], w)
                                              for w in ws]
    else:
        res["native"] = {"unavailable": kernels.load_error()}
    if ref is not None:
        legs["reference_kernel"] = lambda ws: [ref.helm_fp16_linear(xs[w.shape[1]], w)
                                               for w in ws]
    best = {}
    for _ in range(3):
        for name, fn in legs.items():
            best[name] = min(best.get(name, float("inf")), timed(fn, reps))
    for name, dt in best.items():
        res[name] = {"ms_per_layer": dt * 1e3, "GBs": wbytes / dt / 1e9, "rounds": 3}
    if kernels.is_available():
        # parity spot check on the down projection
        from oracle import gemv as O
        w = Ws[0][-1]
        x = xs[w.shape[1]]
        y = kernels.gemv_fp16(x, w, threads=threads).double().numpy()
        ex = O.gemv_fp64(x.reshape(-1).numpy(), w.numpy())
        res["native"]["within_oracle_bound"] = bool(
            (np.abs(y - ex) <= O.error_bound(x.reshape(-1).numpy(), w.numpy())).all())
    dt = timed(lambda ws: [torch.nn.functional.linear(xs[w.shape[1]].float(), w.float()).half()
                           for w in ws], 2)
    res["torch_fp32_fallback"] = {"ms_per_layer": dt * 1e3, "GBs": wbytes / dt / 1e9}
    del Ws
    return res


def cpu_baseline(args, torch, W):
    """The oracle's restatement of HELM's CPU streaming attention (torch CPU)
    on the headline shape; bounded to about args.cpu_seconds."""
    from oracle import attention as A
    w = W.WORKLOADS["qwen3-8b-32k"]
    threads, info = cpu_threads()
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(1)
    P, n = w.page_size, w.T // w.page_size
    k = torch.randn(n, 1, w.Hkv, P, w.D, generator=g).to(w.dtype)
    v = torch.randn(n, 1, w.Hkv, P, w.D, generator=g).to(w.dtype)
    q = torch.randn(1, w.Hq, 1, w.D, generator=g).to(w.dtype)
    pages = [(k[i], v[i]) for i in range(n)]
    mask = torch.zeros(1, 1, 1, w.T)
    alg = W.algorithmic_bytes(w, [w.T])
    res = {}
    budget = args.cpu_seconds / 2
    for name, fn in (("path2_concat_sdpa", lambda: A.concat_sdpa(q, pages)),
                     ("masked_online_softmax", lambda: A.online_softmax_pages(
                         q, pages, attention_mask=mask))):
        fn()
        t0, calls = time.perf_counter(), 0
        while True:
            fn()
            calls += 1
            if time.perf_counter() - t0 > budget:
                break
        per = (time.perf_counter() - t0) / calls
        res[name] = {"s_per_call": per, "GBs": alg / per / 1e9, "calls": calls}
    res["cpu"] = info
    return res, threads


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the paged decode "
              "attention shards by sequence / KV head with no exchange between GPUs",
              file=sys.stderr)
        sys.exit(2)
    import torch
    from helm_amd import workloads as W
    from helm_amd import paged
    if not torch.cuda.is_available():
        print("bench.py needs a HIP GPU", file=sys.stderr)
        sys.exit(1)
    # the device profile first: its copies also bring the GPU to its working
    # clocks before any timed leg
    log("device profile: HBM copy and pinned host-link bandwidth (native probe)")
    from helm_amd import device_profiler as DP
    dprof = DP.measure_links(0)
    dprof = {"hbm_copy_GBs": round(dprof["device_copy_bytes_per_s"] / 1e9, 1),
             "pinned_h2d_GBs": round(dprof["h2d_bytes_per_s"] / 1e9, 2),
             "pinned_d2h_GBs": round(dprof["d2h_bytes_per_s"] / 1e9, 2),
             "probe": "helm_measure_bandwidth: 256 MB streaming copy (read + write), "
                      "64 MB pinned copies each way, 8 timed repetitions after >= 20 ms of "
                      "untimed ones"}
    log(json.dumps(dprof))

    log("headline: qwen3-8b-32k all resident")
    h = gpu_headline(args, torch, W, paged, kernel_timing=True)
    value = h["alg_bytes"] / h["per_call_s"] / 1e9
    kern_us = h["split_kernel_us_mean"]
    kern_gbs = h["alg_bytes"] / (kern_us * 1e-6) / 1e9
    log(f"per call {h['per_call_s'] * 1e6:.2f} us, {value:.1f} GB/s; decode kernel "
        f"{kern_us:.2f} us, {kern_gbs:.1f} GB/s")

    stamps = None
    if args.stamps:
        stamps = workgroup_stamps(torch, h)
        log("workgroup stamps: " + json.dumps(stamps))

    read_floor = None
    if args.read_probe:
        read_floor = read_pass_floor(torch, h)
        log("read-pass floor: " + json.dumps(read_floor))

    if args.copy_calibration:
        n = 1 << 30
        a = torch.empty(n, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        log("copy calibration: 3 x 1 GiB device copies done")

    if args.all:
        all_configs(args, torch, W, paged)

    log("headline shape under HELM's decode mask (zeros [1,1,1,T])")
    hm = gpu_headline(args, torch, W, paged, masked=True)
    hm_gbs = hm["alg_bytes"] / hm["per_call_s"] / 1e9
    masked_c2 = {"us_per_call": round(hm["per_call_s"] * 1e6, 3), "GBs": round(hm_gbs, 1),
                 "roofline_frac": round(hm_gbs / HBM_PEAK_GBS, 4),
                 "max_abs_err_vs_fp64": pool_error(torch, hm, [0, 7]),
                 "mask": "zeros [1, 1, 1, 32768] (HELM's decode mask), read by the kernel"}
    del hm
    log(json.dumps(masked_c2))

    configs = None
    if not args.no_configs:
        log("configs: qwen3-0.6b-2k, qwen3-14b-ragged-b8, llama2-13b-128k-offload75")
        configs = gpu_configs(args, torch, W, paged)

    runtime = None
    if not args.no_runtime:
        log("production decode call: _decode_batched over 8 rotated 32k layers")
        runtime = gpu_runtime_decode(args, torch, W)
        log(json.dumps(runtime))

    full = None
    if not args.no_full_step:
        full = {}
        budgets = [float(x) for x in args.full_step_budgets.split(",") if x]
        for budget in budgets:
            label = f"budget_{budget:g}GB" + ("" if budget >= 64 else "_eviction")
            log(f"full step: qwen3-14b 40 layers, B4 x 64k, device KV budget {budget:.0f} GB")
            r = gpu_full_step(args, torch, W, budget, args.full_step_steps,
                              masked_steps=args.full_step_steps if budget >= 64 else 16)
            log(json.dumps(r))
            full[label] = r

    pre = None
    if not args.no_prefill:
        log("prefill chunk: qwen3-8b shape, 512 tokens over 32k cached, chunk mask")
        pre = gpu_prefill(args, torch)
        log(f"prefill {pre['ms_per_call']:.3f} ms/call, {pre['TFLOPs']:.1f} TFLOP/s")

    off = None
    if not args.no_offload:
        if args.offload_idle > 0:
            log(f"idle {args.offload_idle:g} s before the offload leg")
            time.sleep(args.offload_idle)
        log("offload: qwen3-8b-32k, oldest 50% in pinned host")
        off = gpu_offload(args, torch, W)
        log(f"offload {off['ms_per_call']:.3f} ms/call, host link {off['host_link_GBs']:.1f} GB/s "
            f"({off['frac_of_measured_h2d'] * 100:.1f}% of measured {off['measured_h2d_GBs']:.1f}); "
            f"side stream {off['staged_side_stream_ms_per_call']:.3f} ms/call "
            f"({off['staged_side_stream_frac_of_measured_h2d'] * 100:.1f}%), unbounded "
            f"{off['staged_side_stream_unbounded_ms_per_call']:.3f}")

    gemv = None
    if not args.no_gemv:
        log("cpu gemv: qwen3-8b decode-step linears on host cores (HELM's CPU stages)")
        gemv = cpu_gemv(args, torch)
        log(json.dumps(gemv))


    c1_cpu = None
    if not args.no_cpu:
        log("cpu path: qwen3-0.6b-2k on the host (native kernel beside the oracle's torch code)")
        c1_cpu = cpu_c1(args, torch, W)
        log(json.dumps(c1_cpu))

    cpu = None
    threads = 0
    if not args.no_cpu:
        log("cpu baseline (oracle restatement of HELM's CPU path)")
        cpu, threads = cpu_baseline(args, torch, W)
        log(json.dumps(cpu))

    # HBM bytes per launch from the committed FETCH_SIZE / WRITE_SIZE counters:
    # the decode kernel's own (the roofline's kernel), and the whole call's
    traffic = call_traffic = None
    tpath = os.path.join(ROOT, "profiles", "paged_decode_qwen3-8b-32k_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tj = json.load(f)
        traffic = tj.get("decode_hbm_bytes_per_launch")
        call_traffic = tj.get("hbm_bytes_per_launch")
    # the rocprofv3 kernel durations of the same call (decode + merge kernels),
    # from the committed profile: the live call time above should agree
    prof = None
    ppath = os.path.join(ROOT, "profiles", "paged_decode_qwen3-8b-32k_kernel_times.json")
    if os.path.exists(ppath):
        with open(ppath) as f:
            prof = json.load(f)

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(h["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) q/K/V, seeded random page table, 8 rotated pools",
        "config": {"workload": "qwen3-8b-32k: 1 layer decode attention, B=1, Hq=32, Hkv=8, "
                               "D=128, bf16, 32768 tokens in 2048 pages of 16, all resident",
                   "global_batch": 1, "seq_len": 32768, "page_size": 16},
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "decode_steps_per_s_32k": round(1.0 / (QWEN3_8B_LAYERS * h["per_call_s"]), 2),
        # the same through HELM's production decode call (_decode_batched per
        # layer under HELM's decode mask, wall time per layer call)
        "decode_steps_per_s_32k_production": (
            None if runtime is None else
            round(1e6 / (QWEN3_8B_LAYERS * runtime["masked"]["us_per_call_wall"]), 2)),
        "roofline": {"bound": "hbm", "achieved": round(kern_gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(kern_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "alg_bytes_per_launch": h["alg_bytes"],
                     "avg_launch_us": round(kern_us, 3),
                     "median_launch_us": round(h["split_kernel_us_median"], 3),
                     "p90_launch_us": round(h["split_kernel_us_p90"], 3),
                     "max_launch_us": round(h["split_kernel_us_max"], 3),
                     "launch": "decode_mfma_kernel<bf16, PoolSrc, 0, 4>, the dominant kernel "
                               "of one helm_paged_decode_attn call (256 workgroups: 32 splits "
                               "of 64 pages x 8 KV heads; it reads all K/V, q and the page "
                               "table), timed with HIP start / stop events attached to its "
                               "launch (helm_profile_split_kernels), mean of "
                               f"{args.steps} calls; the split merge after it is outside",
                     "per_call": {"us": round(h["per_call_s"] * 1e6, 3),
                                  "GBs": round(value, 2),
                                  "frac": round(value / HBM_PEAK_GBS, 4),
                                  "traffic": call_traffic,
                                  "launch": "one whole helm_paged_decode_attn call: the "
                                            "decode kernel + the split merge kernel, HIP "
                                            "events around the calls"},
                     "rocprof_kernel_us": prof,
                     "host_issue_us_per_call": round(h["host_issue_us_per_call"], 2)},
        "decode_masked_32k": masked_c2,
        "workgroup_stamps": stamps,
        "read_pass_floor": read_floor,
        "configs": configs,
        "runtime_decode_32k": runtime,
        "c1_cpu_path": c1_cpu,
        "device_profile": dprof,
        "offload50": off,
        "full_step_40l": full,
        "prefill_chunk": pre,
        "cpu_gemv": gemv,
        "cpu_baseline": None if cpu is None else {
            "value": round(cpu["path2_concat_sdpa"]["GBs"], 3), "unit": "GB/s",
            "cores": threads, "kind": "port",
            "cpu_model": cpu["cpu"]["model"],
            "physical_cores_allowed": cpu["cpu"]["physical_cores_allowed"],
            "logical_cpus_allowed": cpu["cpu"]["logical_cpus_allowed"],
            "sample": (f"qwen3-8b-32k shape on {threads} host threads (one per physical core "
                       f"of this process's CPU share), HELM Path 2 (cat + fp32 SDPA) "
                       f"{cpu['path2_concat_sdpa']['calls']} calls; masked online-softmax loop "
                       f"{cpu['masked_online_softmax']['calls']} calls at "
                       f"{cpu['masked_online_softmax']['GBs']:.3f} GB/s")},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
