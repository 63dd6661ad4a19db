#!/usr/bin/env python3
"""Benchmark of the K2 decode layer on one MI355X (the chained layer at M=8 rows).

A step is one launch of the chained layer (indexer scores -> exact top-2048 ->
sparse MLA -> W_UV -> W_o + residual -> RMSNorm -> router top-8 -> MXFP4 routed +
FP8 shared experts -> residual) over 8 decode rows.  Weights and caches of
several distinct layers are resident in HBM and the steps cycle through them, so
no step finds its weights in the 256 MB last-level cache a previous step left.
Steps are replayed from one HIP graph and timed with events on the launch stream.

Prints ONE JSON line (see the driver contract): value = us per layer.
"""

from __future__ import annotations

import argparse
import json
import os
import shlex
import statistics
import sys
import time
from dataclasses import replace

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "sgl-amd-mono_amd"), os.path.join(ROOT, "tests")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_HBM_GBS = 8000.0
METRIC = "us per fused decoder layer @8 decode rows, 1 GPU; % of peak HBM GB/s"
CSRC = os.path.join(ROOT, "sgl-amd-mono_amd", "csrc")
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "k2_layer_m8_traffic.json")
LAYER_KERNEL = "k_k2_layer"  # the persistent layer kernel's name (rocprof)


# the sources the layer launch is built from (its kernels and the headers they include)
LAYER_SOURCES = ("common.hip", "front_stages.h", "indexer_stages.h", "k2_persistent.hip", "layer.hip",
                 "mk2_device.h", "mk2_host.h", "mla_stages.h", "moe_stages.h")


def sources_digest():
    """sha256 over the layer launch's HIP sources: a recorded traffic figure applies to
    these only."""
    import hashlib

    h = hashlib.sha256()
    for name in sorted(os.listdir(CSRC)):
        if name in LAYER_SOURCES:
            h.update(name.encode())
            with open(os.path.join(CSRC, name), "rb") as f:
                h.update(f.read())
    return h.hexdigest()


def recorded_traffic():
    """HBM bytes per layer launch from the committed PMC summary, if it was taken on
    the current sources (else None)."""
    try:
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    if rec.get("sources_sha256") != sources_digest():
        return None
    return rec.get("traffic_bytes_per_launch")


def _pmc_dispatches(dirs):
    """Per-dispatch counters from rocprofv3 --pmc databases, one list per database:
    (dispatch_id, kernel name, {counter: value}).  GRBM counters repeat over instances
    and take the max (as rocprof's MFMA_UTIL does); the others add up over instances."""
    import glob
    import sqlite3

    out = []
    for d in dirs:
        for f in sorted(glob.glob(os.path.join(d, "**", "*.db"), recursive=True)):
            db = sqlite3.connect(f)
            tables = {r[0] for r in db.execute("select name from sqlite_master where type in ('table','view')")}
            if "pmc_events" not in tables:
                continue
            disp = {}
            q = ("select name, dispatch_id, counter_name, sum(counter_value), max(counter_value) "
                 "from pmc_events group by dispatch_id, counter_name")
            for name, did, counter, total, top in db.execute(q):
                disp.setdefault(did, (name, {}))[1][counter] = top if counter.startswith("GRBM_") else total
            out.append([(did, n, c) for did, (n, c) in sorted(disp.items())])
    return out


def _copy_scale(per_db, calib_bytes):
    """Factor turning FETCH_SIZE / WRITE_SIZE (KiB) into bytes, from the calibration copy:
    the last three copyBuffer dispatches of each database (bench.py --copy-calib-mib runs
    them after everything else), each reading and writing calib_bytes / 2."""
    vals = {}
    for rows in per_db:
        copies = [c for _, n, c in rows if "copyBuffer" in n][-3:]
        for c in ("FETCH_SIZE", "WRITE_SIZE"):
            if len(copies) == 3 and all(c in x for x in copies):
                v = [x[c] for x in copies]
                if max(v) > 1.02 * min(v):
                    raise SystemExit(f"calibration copies disagree on {c}: {v}")
                vals[c] = statistics.mean(v)
    return {c: (calib_bytes / 2) / (v * 1024) for c, v in vals.items() if v > 0}


def pmc_summary(dirs, calib_bytes):
    """Mean FETCH_SIZE / WRITE_SIZE (KiB a dispatch) of the layer kernel and of the
    calibration copy, from rocprofv3 --pmc databases; each scaled by the factor that
    turns the copy's counter into its known byte count."""
    per_db = _pmc_dispatches(dirs)
    layer = {}
    for rows in per_db:
        for _, n, c in rows:
            if LAYER_KERNEL in n:
                for k, v in c.items():
                    layer.setdefault(k, []).append(v)
    mean = {k: statistics.mean(v) for k, v in layer.items()}
    scale = _copy_scale(per_db, calib_bytes)
    out = {"sources_sha256": sources_digest(), "layer_kib_per_dispatch": mean,
           "calibration_copy_bytes": calib_bytes, "scale": scale}
    try:
        out["traffic_bytes_per_launch"] = int(mean["FETCH_SIZE"] * 1024 * scale["FETCH_SIZE"] +
                                              mean["WRITE_SIZE"] * 1024 * scale["WRITE_SIZE"])
    except KeyError:
        out["traffic_bytes_per_launch"] = None
    return out


def algorithmic_bytes(cfg, rows, distinct_experts, key_positions=None, kv_rows=None):
    """HBM bytes a layer must move at least once: index keys
    of every request, the gathered latent-KV rows with their scales, W_UV and W_o,
    the router, the shared expert and each distinct routed expert's weights+scales,
    plus queries and the top-k list.  key_positions: the keys the requests hold (rows
    of one request share them; default one full context a row); kv_rows: the distinct
    (request, position) rows the top-k lists select (default rows x topk)."""
    ic, mc, ec = cfg.indexer, cfg.mla, cfg.moe
    if key_positions is None:
        key_positions = rows * ic.context
    if kv_rows is None:
        kv_rows = rows * mc.topk
    keys = key_positions * (ic.dim // 2 + ic.dim // 32)
    idx_io = rows * ic.heads * ic.dim * 2 + rows * ic.heads * 2 + rows * ic.topk * 4
    kv = kv_rows * (mc.qk_dim + 4)
    attn_w = mc.heads * mc.v_dim * mc.kv_lora * 2 + mc.hidden * mc.heads * mc.v_dim * 2
    q = rows * mc.heads * mc.qk_dim * 2
    router = ec.n_experts * ec.hidden * 2
    shared = 3 * ec.hidden * ec.shared_inter * (1 + 4 / (128 * 128)) if ec.n_shared else 0
    per_expert = 3 * ec.hidden * ec.inter * (0.5 + 1 / 32)
    total = keys + idx_io + kv + attn_w + q + router + shared + distinct_experts * per_expert
    return int(total)


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or the platform's processor string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def cpu_baseline(layer, reps):
    import torch

    from refs import CpuLayer

    # the host cores this process may use: the OMP_NUM_THREADS share when it is set (a
    # GPU box gives each GPU a share of its cores), else every core
    cores = os.cpu_count() or 1
    share = os.environ.get("OMP_NUM_THREADS", "")
    if share.isdigit() and int(share) > 0:
        cores = min(cores, int(share))
    torch.set_num_threads(cores)
    t0 = time.perf_counter()
    cl = CpuLayer(layer)
    prep = time.perf_counter() - t0
    cl.forward()  # warm-up
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        cl.forward()
        times.append(time.perf_counter() - t)
    med = statistics.median(times)
    return {
        "value": round(med * 1e6, 1),
        "unit": "us/layer",
        "cores": torch.get_num_threads(),
        "cpu_model": cpu_model(),
        "kind": "port",
        "trials_us": [round(t * 1e6, 1) for t in times],
        "sample": f"1 warm-up + median of {reps} oracle forwards of one configs[4] layer at M={layer.rows} "
                  f"(f64 index scores over {layer.rows} x 65536 keys); expert dequant {prep:.1f}s outside timing",
    }


def pmc_kernels(dirs, calib_bytes):
    """Per-kernel counter table of this library's kernels (names with mk2::), from
    rocprofv3 databases: a --kernel-trace run (durations) and --pmc runs.  HBM bytes are
    FETCH_SIZE and WRITE_SIZE scaled by the calibration copy's factors (as in the
    traffic record), and, where collected, TCC_EA0_RDREQ_DRAM_32B and
    TCC_EA0_WRREQ_WRITE_DRAM_32B x 32 B; MFMA busy is SQ_VALU_MFMA_BUSY_CYCLES over
    GRBM_GUI_ACTIVE x SIMDs; MFMA FLOP from the MOPS counters (512 FLOP a count)."""
    import glob
    import sqlite3
    from collections import defaultdict

    dur = defaultdict(list)
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*.db"), recursive=True):
            db = sqlite3.connect(f)
            tables = {r[0] for r in db.execute("select name from sqlite_master where type in ('table','view')")}
            has_pmc = "pmc_events" in tables and db.execute("select count(*) from pmc_events").fetchone()[0]
            if "kernels" in tables and not has_pmc:  # durations from the trace run only
                for name, ns in db.execute("select name, duration from kernels"):
                    if "mk2::" in name:
                        dur[name].append(ns)
    per_db = _pmc_dispatches(dirs)
    pmc = defaultdict(lambda: defaultdict(list))
    for rows in per_db:
        for _, name, c in rows:
            if "mk2::" in name:
                for k, v in c.items():
                    pmc[name][k].append(v)
    scale = _copy_scale(per_db, calib_bytes)
    simds = 4 * 256
    out = []
    for name in sorted(set(dur) | set(pmc), key=lambda n: -sum(dur.get(n, [0]))):
        m = {c: statistics.mean(v) for c, v in pmc.get(name, {}).items()}
        us = statistics.mean(dur[name]) / 1000 if dur.get(name) else None
        row = {"kernel": name.split("(")[0].replace("void ", ""), "calls": len(dur.get(name, [])),
               "avg_us": round(us, 2) if us else None}
        if "FETCH_SIZE" in m and "WRITE_SIZE" in m and len(scale) == 2:
            rd = m["FETCH_SIZE"] * 1024 * scale["FETCH_SIZE"]
            wr = m["WRITE_SIZE"] * 1024 * scale["WRITE_SIZE"]
            row["read_mb"], row["write_mb"] = round(rd / 1e6, 2), round(wr / 1e6, 2)
            if us:
                row["hbm_gbs"] = round((rd + wr) / (us * 1e-6) / 1e9, 1)
        if "TCC_EA0_RDREQ_DRAM_32B" in m:
            row["dram32_read_mb"] = round(m["TCC_EA0_RDREQ_DRAM_32B"] * 32 / 1e6, 2)
        if "TCC_EA0_WRREQ_WRITE_DRAM_32B" in m:
            row["dram32_write_mb"] = round(m["TCC_EA0_WRREQ_WRITE_DRAM_32B"] * 32 / 1e6, 2)
        if m.get("GRBM_GUI_ACTIVE") and "SQ_VALU_MFMA_BUSY_CYCLES" in m:
            row["mfma_busy_pct"] = round(100.0 * m["SQ_VALU_MFMA_BUSY_CYCLES"] / (m["GRBM_GUI_ACTIVE"] * simds), 2)
        mops = {c[len("SQ_INSTS_VALU_MFMA_MOPS_"):]: v * 512 for c, v in m.items()
                if c.startswith("SQ_INSTS_VALU_MFMA_MOPS_") and v}
        if mops and us:
            row["mfma_tflops"] = {k: round(v / (us * 1e-6) / 1e12, 2) for k, v in mops.items()}
        if "SQ_LDS_BANK_CONFLICT" in m:
            row["lds_bank_conflict_cycles"] = round(m["SQ_LDS_BANK_CONFLICT"])
        out.append(row)
    return {"sources_sha256": sources_digest(), "scale": scale, "kernels": out}


TIMELINE_STAGES = ("score", "slice", "select", "split", "merge + W_UV", "W_o", "router", "route",
                   "up/gate", "down")
ROUTE_MARKS = ("route: logits polled", "route: top-k done", "route: list out")


def timeline_stats(t):
    """Per-stage figures of one persistent launch from its stamps t [grid][33] (100 MHz
    s_memrealtime; per stage s: 3s enter, 3s+1 the first task's input ready, 3s+2
    leave; 0 = not stamped), in us after the earliest enter of the launch: the first
    workgroup in, the median and the last first-input-ready, the last workgroup out."""
    import torch

    t = t.to(torch.int64)
    t0 = int(t[:, 0][t[:, 0] > 0].min())
    rows = {}
    for s, name in enumerate(TIMELINE_STAGES):
        col = lambda i: t[:, i][t[:, i] > 0].double().sub(t0).div(100.0)  # noqa: E731
        enter, ready, leave = col(3 * s), col(3 * s + 1), col(3 * s + 2)
        rows[name] = {
            "first_in": float(enter.min()) if enter.numel() else None,
            "ready_median": float(ready.median()) if ready.numel() else None,
            "ready_last": float(ready.max()) if ready.numel() else None,
            "last_out": float(leave.max()) if leave.numel() else None,
        }
    for i, name in enumerate(ROUTE_MARKS):
        extra = t[:, 3 * len(TIMELINE_STAGES) + i]
        extra = extra[extra > 0].double().sub(t0).div(100.0)
        rows[name] = {"first_in": None, "ready_median": None, "ready_last": None,
                      "last_out": float(extra.max()) if extra.numel() else None}
    return rows


def timeline(ops, outs, launches, dev):
    """Median over `launches` eager persistent launches (cycling the resident layers)
    of each stage's timeline_stats."""
    import statistics as st

    import torch

    G = torch.cuda.get_device_properties(dev).multi_processor_count
    tl = torch.zeros(G, 3 * len(TIMELINE_STAGES) + len(ROUTE_MARKS), dtype=torch.int64, device=dev)
    runs = []
    for i in range(launches):
        tl.zero_()
        ops[i % len(ops)](outs[i % len(ops)], timeline=tl)
        torch.cuda.synchronize()
        runs.append(timeline_stats(tl.cpu()))
    out = {}
    for name in TIMELINE_STAGES + ROUTE_MARKS:
        out[name] = {}
        for k in ("first_in", "ready_median", "ready_last", "last_out"):
            v = [r[name][k] for r in runs if r[name][k] is not None]
            out[name][k] = round(st.median(v), 2) if v else None
    return out


def timeline_markdown(tl, argv, rows, launches):
    lines = [f"# Persistent K2 layer, per-stage timeline at M={rows}", "",
             "Command, run from the repository root on the MI355X box:", "",
             "    python3 " + shlex.join(argv), "",
             f"HIP sources sha256 {sources_digest()}.  Median over {launches} eager launches",
             "(4 resident layers cycled) of the stamps each workgroup takes with s_memrealtime",
             "(100 MHz) as it enters a stage, when its first task's input is ready (its",
             "dependency wait returned) and as it leaves; in us after the launch's first",
             "stamp.  select and route run on one workgroup each (a row's select on its",
             "last slice to count out; the route on a workgroup without a router task).", "",
             "| stage | first in | first input ready: median | first input ready: last | last out |",
             "|---|---|---|---|---|"]
    f = lambda v: "-" if v is None else f"{v:.2f}"  # noqa: E731
    for name in TIMELINE_STAGES + ROUTE_MARKS:
        r = tl[name]
        lines.append(f"| {name} | {f(r['first_in'])} | {f(r['ready_median'])} | {f(r['ready_last'])} | "
                     f"{f(r['last_out'])} |")
    return "\n".join(lines) + "\n"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--rows", type=int, default=8)
    ap.add_argument("--layers", type=int, default=4, help="distinct resident layers cycled")
    ap.add_argument("--cpu-reps", type=int, default=5)
    ap.add_argument("--extra-rows", default="1,4,32",
                    help="more widths measured after the headline one (reported under 'widths')")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--staged", action="store_true", help="one kernel a stage instead of one launch")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="after timing, copy this many MiB (x3) for a PMC calibration")
    ap.add_argument("--pmc-summary", nargs="+", metavar="DIR",
                    help="no GPU: summarize rocprofv3 --pmc databases into the traffic record")
    ap.add_argument("--calib-bytes", type=int, default=512 << 20,
                    help="bytes the calibration copy moves (read + write)")
    ap.add_argument("--pmc-kernels", nargs="+", metavar="DIR",
                    help="no GPU: per-kernel table (durations, HBM bytes, MFMA busy) from rocprofv3 databases")
    ap.add_argument("--timeline", metavar="MD",
                    help="write the persistent launch's per-stage timeline (markdown) to this file and exit")
    ap.add_argument("--timeline-launches", type=int, default=24)
    ap.add_argument("--probes", metavar="MD",
                    help="run the HBM streaming-read and XCD hand-off probes, write a markdown summary and exit")
    ap.add_argument("--standalone", metavar="MD",
                    help="time configs[0..3], the tail and the front as their own launches; write a table")
    args = ap.parse_args()
    if args.pmc_kernels:
        print(json.dumps(pmc_kernels(args.pmc_kernels, args.calib_bytes), indent=1))
        return
    if args.pmc_summary:
        rec = pmc_summary(args.pmc_summary, args.calib_bytes)
        print(json.dumps(rec, indent=1))
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU's share of the layer; --gpus {args.gpus} "
              "is not supported (TP all-reduce omitted by design)", file=sys.stderr)
        sys.exit(2)

    import torch

    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth

    dev = torch.device("cuda:0")
    if args.standalone:
        standalone(args, dev)
        return
    if args.probes:
        run_probes(args.probes, dev)
        return
    cfg, rows = C.C5_LAYER, args.rows
    extra = [int(r) for r in args.extra_rows.split(",") if r] if args.extra_rows else []
    extra = [r for r in extra if r != rows]
    # widths above 8 rows are verify steps of 8 requests (8 x 4 draft tokens at 32
    # rows, as configs[4] names it), built at their width; the decode widths are views
    # of one set of layers built at the widest of them
    def is_verify(r):
        return r > 8 and r % 8 == 0

    decode = [r for r in [rows] + extra if not is_verify(r)]
    layers = ([synth.make_layer(cfg, max(decode), seed=1000 + 17 * i, device=dev) for i in range(args.layers)]
              if decode else [])

    def views(r):
        if is_verify(r):
            return [synth.make_layer(cfg, r, seed=1000 + 17 * i, device=dev, draft=r // 8) for i in range(args.layers)]
        return [synth.view_rows(L, r) for L in layers]

    def layout(r):
        return f"verify: 8 requests x {r // 8} draft tokens" if is_verify(r) else f"decode: {r} requests x 1 token"

    torch.cuda.synchronize()
    if args.timeline:
        if args.staged:
            raise SystemExit("--timeline needs the persistent launch")
        ops, outs = _ops(cfg, views(rows), rows, dev, args.staged)
        for op, o in zip(ops, outs):  # warm-up
            op(o)
        tl = timeline(ops, outs, args.timeline_launches, dev)
        md = timeline_markdown(tl, sys.argv, rows, args.timeline_launches)
        with open(args.timeline, "w") as f:
            f.write(md)
        print(md)
        for op in ops:
            op.check()
        return

    head_views = views(rows)
    head = measure(cfg, head_views, rows, dev, args)
    us, ms = head["us"], head["us"] / 1000.0
    gbs = head["algorithmic_bytes"] / (us * 1e-6) / 1e9
    widths = {}

    def width_entry(m, r, lay):
        g = m["algorithmic_bytes"] / (m["us"] * 1e-6) / 1e9
        return {"layout": lay, "us_per_layer": round(m["us"], 2),
                "tokens_per_s_per_layer": round(r / (m["us"] * 1e-6), 1),
                "algorithmic_bytes_per_layer": int(m["algorithmic_bytes"]), "hbm_gbps": round(g, 1),
                "roofline_frac": round(g / PEAK_HBM_GBS, 4), "distinct_experts": m["distinct"],
                "trials_us": m["trials_us"]}

    for r in extra:
        vl = views(r)
        widths[str(r)] = width_entry(measure(cfg, vl, r, dev, args), r, layout(r))
        if is_verify(r):
            # the same step with the FP4 x FP4 index scorer (queries quantized to MXFP4
            # in the kernel: a contract of its own, not the bf16-query config)
            q4 = replace(cfg, indexer=replace(cfg.indexer, keys=C.KEYS_FP4_Q4))
            widths[f"{r}_fp4_queries"] = width_entry(measure(q4, vl, r, dev, args), r,
                                                     layout(r) + ", FP4 x FP4 index scores")
        del vl

    result = {
        "metric": METRIC,
        "value": round(us, 2),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": head["steps"],
        "warmup": head["warmup"],
        "ms_per_step": round(ms, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp4+fp8 weights, bf16/fp8 MFMA, f32 accumulate",
        "data": "synthetic (seeded random-init weights ~N(0,0.02), rows ~N(0,1), shuffled pages)",
        "config": {
            "workload": "configs[4] chained K2 layer: indexer 64x128 FP4 keys ctx 65536 top-2048 -> "
                        "sparse MLA 16 heads 512+64 FP8 KV -> W_UV/W_o -> RMSNorm 1e-6 -> "
                        "MXFP4 MoE 256 experts top-8 inter 256 + FP8 shared",
            "rows": rows,
            "layout": layout(rows),
            "distinct_layers_cycled": len(layers),
            "parallelism": "1 GPU (TP reduce omitted)",
        },
        "tokens_per_s_per_layer": round(rows / (us * 1e-6), 1),
        "trials_us": head["trials_us"],
        "distinct_experts": head["distinct"],
        "algorithmic_bytes_per_layer": int(head["algorithmic_bytes"]),
        "hbm_gbps": round(gbs, 1),
        "pct_peak_hbm": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "replays_checked": "status words 0 and the last replay's outputs bit-equal to the eager launch's",
        "roofline": {
            "bound": "hbm",
            "kernel": "k2 layer: " + ("12 stage kernels a layer" if args.staged else
                                      "one persistent launch a layer (k_k2_layer)"),
            "achieved": round(gbs, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4),
            "traffic": None if args.staged else recorded_traffic(),
        },
        "widths": widths,
        "cpu_baseline": None,
    }
    if args.copy_calib_mib:
        n = args.copy_calib_mib << 20
        src = torch.ones(n // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(head_views[0], args.cpu_reps)
    print(json.dumps(result))


def run_probes(path, dev):
    """The streaming-read ceiling and the hand-off litmus (sgl_amd_mono.k2.probes)."""
    from sgl_amd_mono.k2 import probes
    lines = ["# HBM streaming-read ceiling and XCD hand-off litmus", "",
             "Command, run from the repository root on the MI355X box:", "",
             "    python3 " + shlex.join(sys.argv), "",
             f"HIP sources sha256 {sources_digest()}.", "",
             "Streaming read in the layer's launch shape (one 512-thread workgroup a CU, 16-B",
             "loads, 8 in flight a lane, `mk2_probe_stream_read`), event-timed. Back to back:",
             "20 launches in a row over distinct buffers cycled through more than 1 GiB (as",
             "bench.py cycles its resident layers), median of 5 reps. Cold: one launch after a",
             "1 GiB write that flushes the L2s and the 256 MB MALL, median of 5:", "",
             "| bytes a launch | back to back GB/s | fraction of 8 TB/s | µs a launch | cold GB/s | cold µs |",
             "|---|---|---|---|---|---|"]
    for mib in (48, 147, 209, 512, 2048):
        print(f"== stream {mib} MiB", flush=True)
        nbytes, b2b, cold = probes.stream_read(mib, reps=5, dev=dev)
        g, c = sorted(b2b)[2], sorted(cold)[2]
        lines.append(f"| {nbytes / 2**20:.0f} MiB | {g:.0f} | {g / 8000:.3f} | {nbytes / g / 1e3:.1f} | "
                     f"{c:.0f} | {nbytes / c / 1e3:.1f} |")
    lines += ["", "Hand-off litmus (`mk2_probe_handoff`): one workgroup a CU, 100 rounds, 4 KiB or",
              "8 KiB a consumer a round, producers and consumers on different XCDs; three",
              "launches a mode:", "", "| mode | protocol | stale words | waits given up | us a round |",
              "|---|---|---|---|---|"]
    for mode, name in probes.HANDOFF_MODES.items():
        print(f"== handoff mode {mode}", flush=True)
        runs = [probes.handoff(mode, rounds=100, dev=dev) for _ in range(3)]
        lines.append(f"| {mode} | {name} | {' / '.join(str(r[0]) for r in runs)} | "
                     f"{' / '.join(str(r[1]) for r in runs)} | {' / '.join(f'{r[2]:.2f}' for r in runs)} |")
    md = "\n".join(lines) + "\n"
    with open(path, "w") as f:
        f.write(md)
    print(md)


def time_graph(calls, steps=200, warmup=20):
    """us per call of `calls` (a list of no-argument launches, cycled) replayed from one
    HIP graph on a side stream, timed with events on that stream: median of 5 trials."""
    import torch

    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        for c in calls:
            c()
        stream.synchronize()
        with torch.cuda.graph(g, stream=stream):
            for c in calls:
                c()
    torch.cuda.synchronize()
    replays = max(1, -(-steps // len(calls)))
    with torch.cuda.stream(stream):
        for _ in range(max(1, -(-warmup // len(calls)))):
            g.replay()
    torch.cuda.synchronize()
    trials = []
    for _ in range(5):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            a.record(stream)
            for _ in range(replays):
                g.replay()
            b.record(stream)
        torch.cuda.synchronize()
        trials.append(a.elapsed_time(b) * 1000.0 / (replays * len(calls)))
    return statistics.median(trials), [round(t, 2) for t in trials]


def _cpu_time(fn, reps):
    """Median us of `reps` calls of fn after one warm-up call (the oracle on the host);
    None with reps = 0 (not timed)."""
    if reps <= 0:
        return None
    fn()
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return statistics.median(times) * 1e6


def standalone(args, dev):
    """configs[0..3] as their own launches (the MoE block at C1 and C2, sparse MLA at C3,
    the indexer at C4), the tail (C6) and the front (C7), each on one resident copy:
    GPU us (graph replay), algorithmic bytes and the share of 8 TB/s, the oracle's CPU
    us on the same inputs, and the parity of the launch's outputs with the oracle's."""
    import torch

    from oracle import codecs as oc
    from oracle import reference as R
    from refs import MoEOracle, cpu, index_keys_f32, mla_oracle
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import FrontOp, IndexerOp, MoEOp, SparseMlaOp, TailOp

    cores = os.cpu_count() or 1
    share = os.environ.get("OMP_NUM_THREADS", "")
    if share.isdigit() and int(share) > 0:
        cores = min(cores, int(share))
    torch.set_num_threads(cores)
    reps = args.cpu_reps
    out = []

    def row(name, rows, us, trials, nbytes, cpu_us, parity):
        gbs = nbytes / (us * 1e-6) / 1e9
        out.append({"config": name, "rows": rows, "us": round(us, 2), "trials_us": trials, "bytes": int(nbytes),
                    "gbps": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4),
                    "cpu_us": None if cpu_us is None else round(cpu_us, 1), "parity": parity})
        print(json.dumps(out[-1]), flush=True)

    # C1 / C2: the MoE block
    for name, cfg, rows in (("C1 FP8 MoE", C.C1_MOE, 4), ("C2 MXFP4 MoE", C.C2_MOE, 8)):
        w = synth.make_moe(cfg, rows, 100 + rows, dev)
        op = MoEOp(cfg, w, rows)
        ids = torch.empty(rows, cfg.top_k, dtype=torch.int32, device=dev)
        y = op(w.x, topk_ids=ids)
        torch.cuda.synchronize()
        d = int(torch.unique(ids).numel())
        fp4 = cfg.expert_fmt in C.FP4_WEIGHT_FMTS
        per = 3 * cfg.hidden * cfg.inter * ((0.5 + 1 / 32) if fp4 else (1 + 4 / (128 * 128)))
        nbytes = d * per + cfg.n_experts * cfg.hidden * 2 + 3 * cfg.hidden * cfg.shared_inter * (1 + 4 / 16384)
        us, tr = time_graph([lambda: op(w.x, out=y)])
        orc = MoEOracle(w)
        ref = orc(w.x)[0]
        cpu_us = _cpu_time(lambda: orc(w.x), reps)
        row(name, rows, us, tr, nbytes, cpu_us, f"rel-L2 {R.rel_l2(cpu(y).float(), ref):.1e}, {d} experts")
    # C3: sparse MLA over given selections + W_UV + W_o
    cfg = C.C3_MLA
    ns = synth.make_mla(cfg, 8, 300, dev)
    op = SparseMlaOp(cfg, ns, 8, ns.page_table.shape[1])
    y = op(ns.q, ns.kv, ns.kv_scale, ns.page_table, ns.req_ids, ns.sel, h=ns.h)
    torch.cuda.synchronize()
    nbytes = 8 * cfg.topk * (cfg.qk_dim + 4) + cfg.heads * cfg.v_dim * cfg.kv_lora * 2 \
        + cfg.hidden * cfg.heads * cfg.v_dim * 2 + 8 * cfg.heads * cfg.qk_dim * 2
    us, tr = time_graph([lambda: op(ns.q, ns.kv, ns.kv_scale, ns.page_table, ns.req_ids, ns.sel, h=ns.h, out=y)])
    ref = mla_oracle(ns)[1]
    cpu_us = _cpu_time(lambda: mla_oracle(ns), reps)
    row("C3 sparse MLA", 8, us, tr, nbytes, cpu_us, f"rel-L2 {R.rel_l2(cpu(y).float(), ref):.1e}")
    # C4: the indexer and the exact top-2048
    cfg = C.C4_INDEXER
    ns = synth.make_indexer(cfg, 8, 400, dev)
    op = IndexerOp(cfg, 8, ns.page_table.shape[1])
    sc, tk = op(ns.q, ns.w, ns.cache, ns.cache_scale, ns.page_table, ns.req_ids, ns.ctx_len)
    torch.cuda.synchronize()
    nbytes = 8 * cfg.context * (cfg.dim // 2 + cfg.dim // 32) + 8 * cfg.heads * (cfg.dim + 1) * 2 + 8 * cfg.topk * 4
    # timed as configs[3] delivers it: the lists, the scores kept inside the launch (the
    # eager call above wrote them for the parity check; the lists are the same bits)
    tk2 = torch.empty_like(tk)
    us, tr = time_graph([lambda: op(ns.q, ns.w, ns.cache, ns.cache_scale, ns.page_table, ns.req_ids, ns.ctx_len,
                                    topk=tk2, with_scores=False)])
    if not torch.equal(tk2, tk):
        raise SystemExit("bench.py: the indexer's lists without the score output differ")
    keys = [index_keys_f32(ns.cache, ns.cache_scale, ns.page_table, r, cfg.context) for r in range(8)]
    qs, ws = cpu(ns.q).float(), cpu(ns.w).float()

    def idx_oracle():
        return [R.radix_lists(R.index_scores(qs[r], ws[r], keys[r]).float(), cfg.topk) for r in range(8)]

    exact = all(torch.equal(cpu(tk)[r].long(), R.radix_lists(cpu(sc)[r], cfg.topk)) for r in range(8))
    cpu_us = _cpu_time(idx_oracle, max(1, reps // 2))
    row("C4 indexer + top-2048", 8, us, tr, nbytes, cpu_us, f"lists exact: {exact}")
    # C6: the tail
    cfg = C.C6_TAIL
    ns = synth.make_tail(cfg, 8, 600, dev)
    op = TailOp(cfg, ns.g_norm, ns.w_head, 8)
    lg, nm = op(ns.x)
    torch.cuda.synchronize()
    nbytes = cfg.vocab_rows * cfg.hidden * 2 + 8 * (2 * cfg.hidden * 2 + cfg.vocab_rows * 4)
    us, tr = time_graph([lambda: op(ns.x, lg, nm)])
    x, gn, wh = cpu(ns.x), cpu(ns.g_norm), cpu(ns.w_head)
    ref = R.tail(x, gn, wh, cfg.eps)[0]
    cpu_us = _cpu_time(lambda: R.tail(x, gn, wh, cfg.eps), reps)
    row("C6 tail (norm + LM head)", 8, us, tr, nbytes, cpu_us, f"rel-L2 {R.rel_l2(cpu(lg), ref):.1e}")
    # C7: the front
    cfg = C.C7_FRONT
    ns = synth.make_front(cfg, 8, 700, dev)
    op = FrontOp(cfg, ns, 8)
    args7 = (ns.x, ns.positions, ns.slots, ns.rope_cos_sin, ns.kv_cache, ns.kv_scale, ns.index_cache, ns.index_scale)
    outs = op(*args7)
    torch.cuda.synchronize()
    wb = sum(t.numel() * t.element_size() for t in (ns.w_qkv_a, ns.s_qkv_a, ns.w_q_b, ns.s_q_b, ns.w_uk, ns.w_iq,
                                                    ns.s_iq, ns.w_ik, ns.s_ik, ns.w_iw))
    us, tr = time_graph([lambda: op(*args7, *outs)])
    from types import SimpleNamespace as NS

    deq = lambda q, s_: oc.fp8_block_dequant(cpu(q), cpu(s_))  # noqa: E731
    wref = NS(g_in=cpu(ns.g_in), g_q_a=cpu(ns.g_q_a), g_kv_a=cpu(ns.g_kv_a), w_qkv_a=deq(ns.w_qkv_a, ns.s_qkv_a),
              w_q_b=deq(ns.w_q_b, ns.s_q_b), w_uk=cpu(ns.w_uk).float(), w_iq=deq(ns.w_iq, ns.s_iq),
              w_ik=deq(ns.w_ik, ns.s_ik), g_ik=cpu(ns.g_ik), b_ik=cpu(ns.b_ik), w_iw=cpu(ns.w_iw).float())
    fr = lambda: R.front(cpu(ns.x).float(), wref, cpu(ns.positions), cpu(ns.rope_cos_sin), eps=cfg.eps,  # noqa: E731
                         index_eps=cfg.index_eps, nope=cfg.nope, heads=cfg.heads, index_heads=cfg.index_heads)
    ref = fr()
    cpu_us = _cpu_time(fr, reps)
    row("C7 front (K1)", 8, us, tr, wb, cpu_us, f"mla_q rel-L2 {R.rel_l2(cpu(outs[0]).float(), ref['mla_q']):.1e}")
    lines = [f"# Standalone launches on MI355X: configs[0..3], the tail and the front", "",
             f"Command: `python {shlex.join(sys.argv)}` (sources {sources_digest()[:12]}).", "",
             f"GPU: HIP-graph replay, median of 5 trials. CPU: the oracle on the same inputs, {cores} threads, "
             f"{cpu_model()}, median of {reps} after a warm-up (C4: {max(1, reps // 2)}).", "",
             "| config | rows | GPU us | GB/s | % of 8 TB/s | CPU us | parity |", "| --- | --- | --- | --- | --- | --- | --- |"]
    for r in out:
        lines.append(f"| {r['config']} | {r['rows']} | {r['us']} | {r['gbps']} | {100 * r['frac']:.1f} | "
                     f"{r['cpu_us']} | {r['parity']} |")
    md = "\n".join(lines) + "\n"
    with open(args.standalone, "w") as f:
        f.write(md)
    print(md)


def _ops(cfg, views, rows, dev, staged):
    import torch

    from sgl_amd_mono.k2.ops import LayerOp

    ops = [LayerOp(cfg, L, rows, device=dev, staged=staged) for L in views]
    outs = [torch.empty(rows, cfg.mla.hidden, dtype=torch.bfloat16, device=dev) for _ in views]
    return ops, outs


def _shared_rows(view, lists):
    """(key positions, distinct latent-KV rows) a layer view's requests hold and select:
    rows of one request share its keys (the longest row's context) and its selected
    rows (the union of their lists)."""
    req, ctx = view.idx.req_ids.cpu().tolist(), view.idx.ctx_len.cpu().tolist()
    keys, kv = {}, {}
    for r, (q, n) in enumerate(zip(req, ctx)):
        keys[q] = max(keys.get(q, 0), n)
        sel = lists[r][lists[r] >= 0].tolist()
        kv.setdefault(q, set()).update(sel)
    return sum(keys.values()), sum(len(s) for s in kv.values())


def measure(cfg, views, rows, dev, args):
    """us per layer at `rows` rows: the layers' launches replayed from one HIP graph and
    timed with events on the launch stream (median of 5 trials).  The replays carry
    each op's sticky status word; after the trials every word must read 0 and the last
    replay's outputs must equal, bit for bit, an eager launch's from before capture."""
    import torch

    ops, outs = _ops(cfg, views, rows, dev, args.staged)
    ids = [torch.empty(rows, cfg.moe.top_k, dtype=torch.int32, device=dev) for _ in ops]
    lists = [torch.empty(rows, cfg.indexer.topk, dtype=torch.int32, device=dev) for _ in ops]
    for op, o, t, tk in zip(ops, outs, ids, lists):  # realized routing and selections
        op(o, topk_ids=t, topk=tk)
    torch.cuda.synchronize()
    distinct = [int(torch.unique(t).numel()) for t in ids]
    eager = [o.clone() for o in outs]
    nbytes = statistics.mean(
        algorithmic_bytes(cfg, rows, d, *_shared_rows(v, tk.cpu())) for d, v, tk in zip(distinct, views, lists))
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        for op, o in zip(ops, outs):  # one eager pass on the capture stream first
            op(o)
        stream.synchronize()
        with torch.cuda.graph(g, stream=stream):
            for op, o in zip(ops, outs):
                op(o)
    torch.cuda.synchronize()
    per_replay = len(ops)
    warm_replays = max(1, -(-args.warmup // per_replay))
    replays = max(1, -(-args.steps // per_replay))
    steps = replays * per_replay
    with torch.cuda.stream(stream):
        for _ in range(warm_replays):
            g.replay()
    torch.cuda.synchronize()
    trials = []
    for _ in range(5):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            start.record(stream)
            for _ in range(replays):
                g.replay()
            end.record(stream)
        torch.cuda.synchronize()
        trials.append(start.elapsed_time(end) / steps)
    for op in ops:
        op.check()
    for o, e in zip(outs, eager):
        if not torch.equal(o, e):
            raise SystemExit(f"bench.py: a graph replay's output differs from the eager launch's at {rows} rows")
    return {"us": statistics.median(trials) * 1000.0, "trials_us": [round(t * 1000, 2) for t in trials],
            "distinct": distinct, "algorithmic_bytes": nbytes, "steps": steps,
            "warmup": warm_replays * per_replay}


if __name__ == "__main__":
    main()
