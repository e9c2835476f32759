"""rocprofv3 summaries of the decode-attention path: the measurement harness
behind ``profiles/``.

The runs are rocprofv3 invocations of ``bench.py`` (``RUNS``: kernel traces of
the headline call, the other configurations and the 40-layer step; one counter
per pass for the HBM byte counters; two SQ counter passes for each matrix-core
kernel).  ``commands`` prints them as a shell script that writes every run
under one directory; ``all`` then writes the summaries (markdown tables and
the JSON files ``bench.py`` reads) from that directory:

    python -m helm_amd.rocprof_report commands --out rocprof_runs > run_prof.sh
    bash run_prof.sh                      # on the GPU machine
    python -m helm_amd.rocprof_report all --in rocprof_runs --out profiles

Single summaries: ``kernels`` (per kernel and grid: dispatches and durations
from ``*_kernel_trace.csv``), ``traffic`` (HBM bytes per dispatch from the
FETCH_SIZE / WRITE_SIZE passes, scaled by what the counters read for a plain
1 GiB device copy of known size), ``counters`` (per-kernel means of SQ
counters and the ratios the design notes quote).

HBM bytes: FETCH_SIZE and WRITE_SIZE count KiB per dispatch; on MI355X a copy
of N bytes reads N / 2 KiB of FETCH_SIZE and N KiB of WRITE_SIZE, so the
scale of each counter is measured from the copies that ``bench.py
--copy-calibration`` makes (three 1 GiB device-to-device copies), not assumed.
"""
from __future__ import annotations

import argparse
import collections
import csv
import glob
import json
import os
import re
import statistics
import sys
from typing import Dict, Iterable, List, Optional

# ── the runs ──────────────────────────────────────────────────────────────────
_BENCH_QUIET = ["--no-full-step", "--no-offload", "--no-gemv", "--no-cpu", "--no-configs",
                "--no-runtime", "--no-prefill"]
# the headline's decode call and the prefill chunk, with the calibration copies
_PMC_DECODE = ["--steps", "20", "--warmup", "4", "--no-cpu", "--no-offload", "--no-full-step",
               "--no-configs", "--no-runtime", "--no-gemv", "--copy-calibration"]
# algorithmic bytes of the prefill leg's chunk call (Qwen3-8B shape, 512 query
# tokens over 32,768 cached, bf16): K and V once, the queries read, the output
# written
PREFILL_READ_BYTES = 32768 * 8 * 128 * 2 * 2 + 512 * 32 * 128 * 2
PREFILL_ALG_BYTES = PREFILL_READ_BYTES + 512 * 32 * 128 * 2
_PMC_A = ["SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_INSTS_VMEM_RD",
          "SQ_WAVES", "SQ_BUSY_CYCLES", "SQ_VALU_MFMA_BUSY_CYCLES"]
_PMC_B = ["SQ_WAVE_CYCLES", "SQ_WAIT_INST_ANY", "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_ANY",
          "SQ_WAIT_INST_LDS", "SQ_LDS_BANK_CONFLICT", "SQ_VALU_MFMA_COEXEC_CYCLES",
          "GRBM_GUI_ACTIVE"]
_PREFILL_ONLY = ["--steps", "20", "--warmup", "5", "--no-full-step", "--no-offload", "--no-gemv",
                 "--no-cpu", "--no-configs", "--no-runtime"]

# name -> (rocprofv3 options, bench.py options, seconds allowed)
RUNS = collections.OrderedDict([
    ("headline", (["--kernel-trace", "--stats"],
                  ["--steps", "200", "--warmup", "20"] + _BENCH_QUIET, 300)),
    ("configs", (["--kernel-trace", "--stats"],
                 ["--steps", "20", "--warmup", "5", "--no-full-step", "--no-offload", "--no-gemv",
                  "--no-cpu", "--no-runtime", "--no-prefill"], 300)),
    ("fullstep", (["--kernel-trace", "--stats"],
                  ["--steps", "20", "--warmup", "5", "--no-offload", "--no-gemv", "--no-cpu",
                   "--no-configs", "--no-runtime", "--no-prefill", "--full-step-budgets", "64"],
                  400)),
    ("fetch", (["--pmc", "FETCH_SIZE"], _PMC_DECODE, 150)),
    ("write", (["--pmc", "WRITE_SIZE"], _PMC_DECODE, 150)),
    ("copies", (["--kernel-trace", "--memory-copy-trace"],
                ["--no-configs", "--no-runtime", "--no-full-step", "--no-prefill", "--no-gemv",
                 "--no-cpu"], 300)),
    ("pmc_a", (["--pmc"] + _PMC_A, _PREFILL_ONLY, 150)),
    ("pmc_b", (["--pmc"] + _PMC_B, _PREFILL_ONLY, 150)),
])


def run_commands(out_dir: str, repo: str = "$R") -> List[str]:
    """The shell lines of every run: rocprofv3 from /tmp (TMPDIR=/tmp), the
    program itself after ``--``, each run under its own time limit; the
    counter passes under SIGKILL limits (a pass that asks for more counters
    than a block holds hangs)."""
    lines = ["#!/bin/bash", "# rocprofv3 runs behind profiles/ (helm_amd/rocprof_report.py)",
             'R="$(pwd)"   # run from the repository root', "cd /tmp && export TMPDIR=/tmp",
             f"mkdir -p {repo}/{out_dir}"]
    for name, (prof, bench, secs) in RUNS.items():
        kill = "-s KILL" if "--pmc" in prof else "-k 10"
        cmd = (f"timeout {kill} {secs} rocprofv3 {' '.join(prof)} --output-format csv "
               f"-d {repo}/{out_dir}/{name} -o run -- python3 -u {repo}/bench.py "
               f"{' '.join(bench)} > {repo}/{out_dir}/{name}.log 2>&1 || exit $?")
        lines += [f'echo "step: {name}"', cmd]
    lines.append('echo "runs done"')
    return lines


def command_of(name: str, out_dir: str = "rocprof_runs") -> str:
    prof, bench, _ = RUNS[name]
    return (f"rocprofv3 {' '.join(prof)} --output-format csv -d $R/{out_dir}/{name} -o run -- "
            f"python3 -u $R/bench.py {' '.join(bench)}")


# ── parsing ───────────────────────────────────────────────────────────────────
def short_name(n: str) -> str:
    """``helm::decode_mfma_kernel<helm::bf16_t, helm::PoolSrc, 0, 4>(...)`` ->
    ``decode_mfma_kernel<bf16, PoolSrc, 0, 4>``."""
    n = n.replace("(anonymous namespace)::", "").replace("helm::", "")
    depth, cut = 0, len(n)
    for i, ch in enumerate(n):          # drop the argument list (not template args)
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            cut = i
            break
    n = n[:cut].replace("bf16_t", "bf16").replace("f16_t", "f16").replace("void ", "")
    n = re.sub(r"\s+", " ", n).strip()
    if len(n) > 90 and "<" in n:       # torch's long functor templates
        n = n[:n.index("<")] + "<...>"
    return n


def _csvs(paths: Iterable[str], suffix: str) -> List[str]:
    out = []
    for p in paths:
        if os.path.isdir(p):
            out += sorted(glob.glob(os.path.join(p, "**", f"*{suffix}"), recursive=True))
        else:
            out.append(p)
    return out


def kernel_trace(paths: Iterable[str]) -> List[dict]:
    """Dispatches of every ``*_kernel_trace.csv`` under `paths`."""
    rows = []
    for path in _csvs(paths, "_kernel_trace.csv"):
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                rows.append({
                    "name": short_name(r["Kernel_Name"]),
                    "grid": f'{r["Grid_Size_X"]} x {r["Grid_Size_Y"]} x {r["Grid_Size_Z"]}',
                    "us": (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3,
                    "vgpr": int(r["VGPR_Count"]), "agpr": int(r["Accum_VGPR_Count"]),
                    "scratch": int(r["Scratch_Size"]), "lds": int(r["LDS_Block_Size"]),
                })
    return rows


def kernel_stats(rows: List[dict]) -> "collections.OrderedDict":
    """(kernel, grid) -> dispatches, mean / median / min / max microseconds,
    registers and LDS."""
    g = collections.OrderedDict()
    for r in rows:
        g.setdefault((r["name"], r["grid"]), []).append(r)
    out = collections.OrderedDict()
    for key, rs in g.items():
        d = [r["us"] for r in rs]
        out[key] = {"dispatches": len(d), "mean_us": statistics.mean(d),
                    "median_us": statistics.median(d), "min_us": min(d), "max_us": max(d),
                    "vgpr": rs[0]["vgpr"], "agpr": rs[0]["agpr"], "scratch": rs[0]["scratch"],
                    "lds": rs[0]["lds"]}
    return out


def counter_rows(paths: Iterable[str]) -> List[dict]:
    """One row per (dispatch, counter) of every ``*_counter_collection.csv``."""
    rows = []
    for path in _csvs(paths, "_counter_collection.csv"):
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                rows.append({"dispatch": int(r["Dispatch_Id"]), "name": short_name(r["Kernel_Name"]),
                             "grid": int(r["Grid_Size"]), "counter": r["Counter_Name"],
                             "value": float(r["Counter_Value"])})
    return rows


def counter_means(rows: List[dict]) -> Dict[str, Dict[str, float]]:
    """kernel -> counter -> mean per dispatch (a counter's instances summed
    per dispatch first), with the dispatch count under ``dispatches``."""
    per = collections.defaultdict(lambda: collections.defaultdict(float))
    names = {}
    for r in rows:
        per[(r["dispatch"], r["counter"])]["v"] += r["value"]
        names[r["dispatch"]] = r["name"]
    by_kernel = collections.defaultdict(lambda: collections.defaultdict(list))
    for (disp, ctr), v in per.items():
        by_kernel[names[disp]][ctr].append(v["v"])
    out = {}
    for k, ctrs in by_kernel.items():
        out[k] = {c: statistics.mean(v) for c, v in ctrs.items()}
        out[k]["dispatches"] = max(len(v) for v in ctrs.values())
    return out


# ── summaries ─────────────────────────────────────────────────────────────────
def kernels_md(stats, title: str, commands: List[str]) -> str:
    lines = [f"# {title}", "", "Commands (repo root `R`, from `/tmp` with `TMPDIR=/tmp`):", "",
             "```", *commands, "```", "",
             "Per dispatch duration = end - start of the kernel trace "
             "(`python -m helm_amd.rocprof_report kernels <run dir>`).", "",
             "| Kernel | Grid (threads) | Dispatches | Mean (us) | Median (us) | Min (us) | "
             "Max (us) | VGPR | LDS (B) | Scratch |",
             "|---|---|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for (name, grid), s in stats.items():
        lines.append(f"| `{name}` | {grid} | {s['dispatches']} | {s['mean_us']:.2f} | "
                     f"{s['median_us']:.2f} | {s['min_us']:.2f} | {s['max_us']:.2f} | "
                     f"{s['vgpr']} | {s['lds']} | {s['scratch']} |")
    return "\n".join(lines) + "\n"


def _pick(stats: dict, pattern: str):
    """The (kernel, grid) entry matching `pattern` with the most dispatches."""
    hits = [(k, s) for k, s in stats.items() if re.search(pattern, k[0])]
    if not hits:
        return None
    return max(hits, key=lambda ks: ks[1]["dispatches"])


def headline_times(stats: dict) -> dict:
    """The decode and merge kernels of the headline call (bench.py reads this
    file as the rocprof side of its roofline)."""
    dec = _pick(stats, r"^decode_mfma_kernel<bf16, PoolSrc, 0, 4>")
    mer = _pick(stats, r"^merge_splits_d128_kernel")
    if dec is None or mer is None:
        raise ValueError("no headline decode / merge dispatches in the trace")
    return {"source": "profiles/paged_decode_qwen3-8b-32k_kernel_stats.md",
            "decode_kernel_avg_us": round(dec[1]["mean_us"], 2),
            "decode_kernel_median_us": round(dec[1]["median_us"], 2),
            "merge_kernel_avg_us": round(mer[1]["mean_us"], 2),
            "call_kernels_us": round(dec[1]["mean_us"] + mer[1]["mean_us"], 2),
            "dispatches": dec[1]["dispatches"]}


COPY_KERNEL = r"copyBuffer"
SIMDS, XCDS = 1024, 8          # MI355X: 256 CUs x 4 SIMDs in 8 XCDs


def traffic(fetch_paths, write_paths, alg_bytes: int, decode: str, merge: str,
            calib_bytes: int = 1 << 30) -> dict:
    """HBM bytes per dispatch of the decode and merge kernels from the two
    counter passes, each counter scaled by what it reads for the calibration
    copies (a copy of calib_bytes reads and writes calib_bytes)."""
    fm = counter_means(counter_rows(fetch_paths))
    wm = counter_means(counter_rows(write_paths))

    def calib(paths, ctr):
        # the copy dispatches of the largest size (the calibration copies; the
        # run's other copies are small)
        vals = collections.defaultdict(float)
        for r in counter_rows(paths):
            if r["counter"] == ctr and re.search(COPY_KERNEL, r["name"]):
                vals[r["dispatch"]] += r["value"]
        if not vals:
            raise ValueError(f"no calibration copy in the {ctr} pass (run with --copy-calibration)")
        top = max(vals.values())
        big = [v for v in vals.values() if v >= 0.9 * top]
        return calib_bytes / (statistics.median(big) * 1024)

    fs, ws = calib(fetch_paths, "FETCH_SIZE"), calib(write_paths, "WRITE_SIZE")

    def kernel_bytes(means, ctr, pat, scale):
        hits = [m[ctr] for k, m in means.items() if re.search(pat, k) and ctr in m]
        if not hits:
            raise ValueError(f"no {pat} dispatches in the {ctr} pass")
        return hits[0] * 1024 * scale

    dfb = kernel_bytes(fm, "FETCH_SIZE", decode, fs)
    dwb = kernel_bytes(wm, "WRITE_SIZE", decode, ws)
    mfb = kernel_bytes(fm, "FETCH_SIZE", merge, fs)
    mwb = kernel_bytes(wm, "WRITE_SIZE", merge, ws)
    return {"fetch_scale": fs, "write_scale": ws,
            "decode_fetch_bytes": dfb, "decode_write_bytes": dwb,
            "merge_fetch_bytes": mfb, "merge_write_bytes": mwb,
            "hbm_bytes_per_launch": dfb + dwb + mfb + mwb,
            "algorithmic_bytes": alg_bytes,
            "traffic_over_algorithmic": (dfb + dwb + mfb + mwb) / alg_bytes,
            "decode_hbm_bytes_per_launch": dfb + dwb,
            "decode_traffic_over_algorithmic": (dfb + dwb) / alg_bytes}


def copy_runs(paths: Iterable[str], min_us: float = 500.0) -> List[dict]:
    """Runs of large host-to-device copies (at least `min_us` each) from
    ``*_memory_copy_trace.csv``: consecutive copies on one stream form a run;
    per run its stream, start (ms after the first large copy), copy count,
    median copy duration and median start-to-start interval (the call's
    cycle when each call makes one such copy)."""
    big = []
    for path in _csvs(paths, "_memory_copy_trace.csv"):
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                a, b = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
                if "HOST_TO_DEVICE" in r["Direction"] and (b - a) / 1e3 >= min_us:
                    big.append((r["Stream_Id"], a, b))
    big.sort(key=lambda x: x[1])
    runs: List[dict] = []
    for stream, a, b in big:
        if runs and runs[-1]["stream"] == stream and a - runs[-1]["_last"] < 5e6:
            runs[-1]["_copies"].append((a, b))
            runs[-1]["_last"] = a
        else:
            runs.append({"stream": stream, "_first": a, "_last": a, "_copies": [(a, b)]})
    t0 = big[0][1] if big else 0
    out = []
    for r in runs:
        cs = r["_copies"]
        dur = [(y - x) / 1e3 for x, y in cs]
        cyc = [(y[0] - x[0]) / 1e3 for x, y in zip(cs, cs[1:])]
        out.append({"stream": r["stream"], "start_ms": round((r["_first"] - t0) / 1e6, 1),
                    "copies": len(cs), "copy_us_median": round(statistics.median(dur), 1),
                    "cycle_us_median": round(statistics.median(cyc), 1) if cyc else None})
    return out


def counters_md(means: dict, kernels: str, title: str, commands: List[str]) -> str:
    lines = [f"# {title}", "", "Commands (repo root `R`, from `/tmp` with `TMPDIR=/tmp`):", "",
             "```", *commands, "```", "",
             "Per dispatch means (`python -m helm_amd.rocprof_report counters <run dirs>`).", ""]
    keys = sorted(k for k in means if re.search(kernels, k))
    ctrs = sorted({c for k in keys for c in means[k] if c != "dispatches"})
    lines += ["| Kernel | Dispatches | " + " | ".join(ctrs) + " |",
              "|---|---:|" + "---:|" * len(ctrs)]
    for k in keys:
        m = means[k]
        lines.append(f"| `{k}` | {m['dispatches']} | " +
                     " | ".join(f"{m[c]:,.0f}" if c in m else "" for c in ctrs) + " |")
    derived = []
    for k in keys:
        m = means[k]
        row = []
        if m.get("SQ_INSTS_MFMA"):
            for c in ("SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_LDS"):
                if c in m:
                    row.append(f"{c[9:]} per MFMA {m[c] / m['SQ_INSTS_MFMA']:.2f}")
        if m.get("GRBM_GUI_ACTIVE") and "SQ_VALU_MFMA_BUSY_CYCLES" in m:
            # GRBM_GUI_ACTIVE sums the 8 XCDs' busy cycles; 1,024 SIMDs
            busy = m["SQ_VALU_MFMA_BUSY_CYCLES"] / (SIMDS * m["GRBM_GUI_ACTIVE"] / XCDS)
            row.append(f"matrix pipe busy {busy:.3f} of the kernel")
        if m.get("SQ_WAVE_CYCLES") and "SQ_ACTIVE_INST_ANY" in m:
            row.append(f"issuing {m['SQ_ACTIVE_INST_ANY'] / m['SQ_WAVE_CYCLES']:.3f} of wave "
                       "cycles")
        if row:
            derived.append(f"* `{k}`: " + "; ".join(row))
    if derived:
        lines += ["", "Ratios:", "", *derived]
    return "\n".join(lines) + "\n"


def write_all(in_dir: str, out_dir: str, alg_bytes: int = 134242304) -> List[str]:
    """Every summary whose runs are present under `in_dir` (the layout of
    ``commands``), written to `out_dir`; returns the files written."""
    written = []
    os.makedirs(out_dir, exist_ok=True)

    def cmd_of(run):   # the run's command as it wrote under in_dir
        return command_of(run, os.path.normpath(in_dir))

    def put(name, text):
        path = os.path.join(out_dir, name)
        with open(path, "w") as f:
            f.write(text)
        written.append(path)

    def have(run):
        return os.path.isdir(os.path.join(in_dir, run))

    if have("headline"):
        st = kernel_stats(kernel_trace([os.path.join(in_dir, "headline")]))
        put("paged_decode_qwen3-8b-32k_kernel_stats.md",
            kernels_md(st, "Kernel time: Qwen3-8B 32k decode attention (the bench headline)",
                       [cmd_of("headline")]))
        put("paged_decode_qwen3-8b-32k_kernel_times.json",
            json.dumps(headline_times(st), indent=1) + "\n")
    if have("configs"):
        st = kernel_stats(kernel_trace([os.path.join(in_dir, "configs")]))
        put("configs_c1_c3_c4_kernel_stats.md",
            kernels_md(st, "Kernel time: the other configurations (C1, C3, C4 and the masked "
                           "headline)", [cmd_of("configs")]))
    if have("fullstep"):
        st = kernel_stats(kernel_trace([os.path.join(in_dir, "fullstep")]))
        put("full_step_qwen3-14b-40l-b4-64k_kernel_stats.md",
            kernels_md(st, "Kernel time: the 40-layer Qwen3-14B decode step (B4 x 64k, 64 GB "
                           "budget)", [cmd_of("fullstep")]))
    if have("fetch") and have("write"):
        t = traffic([os.path.join(in_dir, "fetch")], [os.path.join(in_dir, "write")], alg_bytes,
                    r"^decode_mfma_kernel<bf16, PoolSrc, 0, 4>", r"^merge_splits_d128_kernel")
        t = {"kernel": "decode_mfma_kernel<bf16, PoolSrc, 0, 4> + merge_splits_d128_kernel<bf16>",
             "workload": "qwen3-8b-32k", **t}
        put("paged_decode_qwen3-8b-32k_traffic.json", json.dumps(t, indent=1) + "\n")
        md = ["# HBM traffic per call: Qwen3-8B 32k decode attention", "",
              "Commands (repo root `R`, from `/tmp` with `TMPDIR=/tmp`), one counter per pass:",
              "", "```", cmd_of("fetch"), cmd_of("write"), "```", "",
              "`--copy-calibration` adds three plain 1 GiB device copies; each counter's scale "
              "to bytes is what it reads for them (`python -m helm_amd.rocprof_report traffic`).",
              "", f"* FETCH_SIZE: x{t['fetch_scale']:.5f} KiB; WRITE_SIZE: "
              f"x{t['write_scale']:.5f} KiB",
              f"* decode kernel: {t['decode_fetch_bytes']:,.0f} B read, "
              f"{t['decode_write_bytes']:,.0f} B written per dispatch: "
              f"x{t['decode_traffic_over_algorithmic']:.4f} of the {alg_bytes:,} algorithmic "
              "bytes",
              f"* merge kernel: {t['merge_fetch_bytes']:,.0f} B read, "
              f"{t['merge_write_bytes']:,.0f} B written",
              f"* whole call: {t['hbm_bytes_per_launch']:,.0f} B, "
              f"x{t['traffic_over_algorithmic']:.4f}"]
        put("paged_decode_qwen3-8b-32k_traffic.md", "\n".join(md) + "\n")
        try:
            c = traffic([os.path.join(in_dir, "fetch")], [os.path.join(in_dir, "write")],
                        PREFILL_ALG_BYTES, r"^chunk32_mfma_kernel<bf16, DescSrc, 4, 8>",
                        r"^merge_rows_d128_kernel")
        except ValueError:
            c = None          # runs made without the prefill leg
        if c is not None:
            md = ["# HBM traffic per call: the prefill chunk (512 tokens over 32k, Qwen3-8B "
                  "shape)", "",
                  "The same two counter passes as the decode call's traffic:", "", "```",
                  cmd_of("fetch"), cmd_of("write"), "```", "",
                  f"* chunk kernel `chunk32_mfma_kernel<bf16, DescSrc, 4, 8>`: "
                  f"{c['decode_fetch_bytes']:,.0f} B read, {c['decode_write_bytes']:,.0f} B "
                  f"written per dispatch (the written bytes are the splits' partials)",
                  f"* merge `merge_rows_d128_kernel`: {c['merge_fetch_bytes']:,.0f} B read, "
                  f"{c['merge_write_bytes']:,.0f} B written",
                  f"* algorithmic bytes (K and V once, queries, output): {PREFILL_ALG_BYTES:,}, "
                  f"of which {PREFILL_READ_BYTES:,} read; the chunk kernel reads "
                  f"x{c['decode_fetch_bytes'] / PREFILL_READ_BYTES:.4f} of those: the eight "
                  "workgroups that share a KV head's split run on one XCD and share its L2, so "
                  "each K/V byte crosses from HBM about once",
                  f"* whole call: {c['hbm_bytes_per_launch']:,.0f} B"]
            put("prefill_chunk32_qwen3-8b-512x32k_traffic.md", "\n".join(md) + "\n")
    if have("copies"):
        runs = copy_runs([os.path.join(in_dir, "copies")])
        md = ["# Host-to-device copies of the Qwen3-8B 32k call with 50% of its pages in "
              "pinned host memory", "",
              "Command (repo root `R`, from `/tmp` with `TMPDIR=/tmp`):", "", "```",
              cmd_of("copies"), "```", "",
              "Runs of consecutive large (>= 0.5 ms) host-to-device copies on one stream, in "
              "the order the bench makes them: the device profile's 64 MiB link probe (its "
              "own stream), then the offload leg's modes, each call copying its 64 MiB of "
              "host pages in one copy (3 warm-up calls and 3 timed runs per mode): forced "
              "staging (HELM_AMD_HOST_READ=copy, copies on the caller's stream), the side "
              "stream (HELM_AMD_STAGE_STREAM=side: the engine's copy stream, the host at "
              "most two calls ahead), the same with no such bound (HELM_AMD_SIDE_AHEAD=0), "
              "one stream (=one, the same as forced staging), the engine default (which stages this "
              "one-run layout; the in-place mode before it copies nothing), and the bench's "
              "256 MiB pinned-copy peak.  A call's cycle is its copy plus whatever its "
              "copy waits for; on one stream that includes the previous call's kernels.  "
              "`python -m helm_amd.rocprof_report all` on the run directory.", "",
              "| Stream | Starts (ms) | Copies | Copy (us, median) | Start to start (us, "
              "median) |", "|---|---:|---:|---:|---:|"]
        for r in runs:
            md.append(f"| {r['stream']} | {r['start_ms']} | {r['copies']} | "
                      f"{r['copy_us_median']} | {r['cycle_us_median']} |")
        put("offload_qwen3-8b-32k-offload50_copies.md", "\n".join(md) + "\n")
    if have("pmc_a") or have("pmc_b"):
        dirs = [os.path.join(in_dir, d) for d in ("pmc_a", "pmc_b") if have(d)]
        means = counter_means(counter_rows(dirs))
        put("paged_decode_and_prefill_chunk_counters.md",
            counters_md(means, r"^(decode_mfma_kernel|chunk32_mfma_kernel|merge_)",
                        "SQ counters: decode kernel (Qwen3-8B 32k) and prefill chunk kernel "
                        "(512 tokens over 32k)", [cmd_of("pmc_a"), cmd_of("pmc_b")]))
    return written


def bench_summaries(line_path: str, out_dir: str, command: str) -> List[str]:
    """The workgroup stamps and the read-pass floor of a ``bench.py --stamps
    --read-probe`` JSON line (the last line of `line_path` that parses),
    written as markdown to `out_dir`."""
    line = None
    with open(line_path) as f:
        for raw in f:
            raw = raw.strip()
            if raw.startswith("{"):
                try:
                    line = json.loads(raw)
                except json.JSONDecodeError:
                    pass
    if line is None:
        raise ValueError(f"{line_path}: no JSON line")
    written = []
    head = ["Command (repo root `R`):", "", "```", command, "```", ""]
    per_call = line.get("roofline", {}).get("per_call", {}).get("us")
    st = line.get("workgroup_stamps")
    if st:
        md = ["# Workgroup stamps: Qwen3-8B 32k decode kernel (the bench headline)", "", *head,
              st["how"] + ".", "",
              f"* per call (bench line): {per_call} us; decode kernel (HIP events of its "
              f"launch): {line['roofline']['avg_launch_us']} us",
              f"* workgroups: {st['workgroups']}; captures: {st['captures']}", "",
              "| us after the first start | min | mean | max | std |", "|---|---:|---:|---:|---:|"]
        for k in ("start_us", "loop_end_us", "end_us"):
            v = st[k]
            md.append(f"| {k[:-3].replace('_', ' ')} | {v['min']} | {v['mean']} | {v['max']} | "
                      f"{v['std']} |")
        md += ["", f"* page-loop end spread per capture (us): "
                   f"{st['loop_end_spread_us_per_capture']}",
               f"* last workgroup end per capture (us): {st['last_end_us_per_capture']}",
               f"* mean page-loop end per XCD (us): {st['loop_end_mean_per_xcd_us']}",
               f"* mean page-loop end per KV head (us): {st['loop_end_mean_per_kv_head_us']}",
               f"* correlation of a workgroup's lateness between consecutive captures: "
               f"{st['lateness_correlation_between_calls']}"]
        path = os.path.join(out_dir, "paged_decode_qwen3-8b-32k_workgroup_stamps.md")
        with open(path, "w") as f:
            f.write("\n".join(md) + "\n")
        written.append(path)
    rf = line.get("read_pass_floor")
    if rf:
        md = ["# Read-pass floor of the Qwen3-8B 32k decode call", "", *head, rf["how"] + ".", "",
              f"K/V bytes per pass: {rf['kv_bytes']:,}; tail kernel: {rf['tail_bytes']:,} bytes "
              f"at 32 workgroups; {rf['iters']} passes.", "",
              "| Workgroups | read pass (us) | GB/s | read pass + tail kernel (us) |",
              "|---:|---:|---:|---:|"]
        for k, v in rf.items():
            if k.startswith("workgroups_"):
                md.append(f"| {k.split('_')[1]} | {v['read_us']} | {v['read_GBs']} | "
                          f"{v['read_then_tail_us']} |")
        md += ["", f"Decode call of the same run: {per_call} us per call; its decode kernel "
                   f"{line['roofline']['avg_launch_us']} us (HIP events of its launch)."]
        path = os.path.join(out_dir, "paged_decode_qwen3-8b-32k_read_floor.md")
        with open(path, "w") as f:
            f.write("\n".join(md) + "\n")
        written.append(path)
    return written


def main(argv: Optional[List[str]] = None) -> int:
    ap = argparse.ArgumentParser(prog="python -m helm_amd.rocprof_report")
    sub = ap.add_subparsers(dest="cmd", required=True)
    c = sub.add_parser("commands", help="the rocprofv3 runs as a shell script")
    c.add_argument("--out", default="rocprof_runs")
    a = sub.add_parser("all", help="every summary from a directory of runs")
    a.add_argument("--in", dest="in_dir", required=True)
    a.add_argument("--out", default="profiles")
    k = sub.add_parser("kernels", help="kernel-trace table of run directories or CSVs")
    k.add_argument("paths", nargs="+")
    t = sub.add_parser("traffic", help="HBM bytes per dispatch from FETCH_SIZE / WRITE_SIZE")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--alg-bytes", type=int, default=134242304)
    t.add_argument("--decode", default=r"^decode_mfma_kernel<bf16, PoolSrc, 0, 4>")
    t.add_argument("--merge", default=r"^merge_splits_d128_kernel")
    b = sub.add_parser("bench", help="workgroup stamps and read-pass floor of a bench line")
    b.add_argument("line")
    b.add_argument("--out", default="profiles")
    b.add_argument("--command", default="python3 -u $R/bench.py --stamps --read-probe "
                   "--no-configs --no-runtime --no-full-step --no-prefill --no-offload "
                   "--no-gemv --no-cpu")
    n = sub.add_parser("counters", help="per-kernel counter means")
    n.add_argument("paths", nargs="+")
    n.add_argument("--kernels", default=".")
    args = ap.parse_args(argv)
    if args.cmd == "commands":
        print("\n".join(run_commands(args.out)))
    elif args.cmd == "all":
        for p in write_all(args.in_dir, args.out):
            print("wrote", p)
    elif args.cmd == "kernels":
        print(kernels_md(kernel_stats(kernel_trace(args.paths)), "Kernel time", []))
    elif args.cmd == "traffic":
        print(json.dumps(traffic([args.fetch], [args.write], args.alg_bytes, args.decode,
                                 args.merge), indent=1))
    elif args.cmd == "bench":
        for p in bench_summaries(args.line, args.out, args.command):
            print("wrote", p)
    elif args.cmd == "counters":
        print(counters_md(counter_means(counter_rows(args.paths)), args.kernels, "Counters", []))
    return 0


if __name__ == "__main__":
    sys.exit(main())
