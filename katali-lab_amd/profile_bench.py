"""Profile one bench.py workload with rocprofv3 and write its summary.

    python katali-lab_amd/profile_bench.py --workload moe48 --out DIR [--steps 8]
    python katali-lab_amd/profile_bench.py --workload moe48 --out DIR --summarize-only
    python katali-lab_amd/profile_bench.py --workload moe48 --out DIR --phases [--stacked]

--phases: no profiler; bench.py runs on the measurement build
(libkatali_hip_stamps.so, `python katali-lab_amd/build.py --stamps`), whose
one-launch layers record s_memrealtime phase stamps, and the stamps of the
timed replays' last 64 layers become profiles/phases_<workload>[_stacked].md
(per phase, over the layers, the median of the workgroups' median and of
their latest time after the layer's first workgroup started).

Three runs of bench.py under rocprofv3 (each a child process; rocprofv3
runs from /tmp with TMPDIR=/tmp):
  1. --kernel-trace --stats: per-kernel call counts and average durations;
  2. --pmc FETCH_SIZE and 3. --pmc WRITE_SIZE: HBM KiB per dispatch.
Every run starts with bench.py --calibrate-copy 256, one plain copy kernel of
256 MiB read + 256 MiB written; the counter value that copy reports fixes the
scale factor between counter KiB and bytes. Writes profiles/<name>.md (the
commands, the kernel table and the traffic per workload unit) and
profiles/traffic_<workload>.txt (read by bench.py for roofline.traffic).
"""
from __future__ import annotations

import argparse
import csv
import glob
import os
import sqlite3
import subprocess
import sys
from collections import defaultdict

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
COPY_MIB = 256
# kernels summed per workload unit; the first is launched once per unit
KERNELS = {
    "floor48": ("k_floor_read",),
    "moe48": ("k_moe_xcd",),
    "moe40cold": ("k_moe_xcd",),
    "gemv6144": ("k_gemv",),
    "qwen8b": ("k_moe_down", "k_moe_gu", "k_gemv_multi", "k_gemv"),
    "moe48tok": ("k_argmax", "k_norm_router", "k_moe_xcd", "k_rmsnorm", "k_gemv"),
    "moebatch": ("k_mb_group", "k_quantize_q8_1", "k_moe_gu_grp", "k_mb_gu_mfma", "k_moe_down_grp", "k_mb_down_mfma",
                 "k_mb_combine"),
}
UNIT_NAME = {"floor48": "one read of a moe48 layer's weight bytes", "moe48": "MoE layer", "moe40cold": "MoE layer", "gemv6144": "GEMV", "qwen8b": "dense layer",
             "moebatch": "batched MoE layer (n_sel 8, 64 tokens)", "moe48tok": "decode token"}
EXTRA_ARGS = {"moebatch": ["--batch-points", "8x64"], "floor48": ["--floor-kind", "0"]}
PROFILE_NAME = {"moebatch": "batched_moe_moebatch_8x64", "moe48tok": "decode_token_moe48tok", "qwen8b": "k_gemv_k_moe_gu_k_moe_down_qwen8b"}
# eight-slot layers (and eight routed experts plus the shared expert at ffn
# 256 or 512) run as k_moe_xcd unless KATALI_HIP_XCD=0 (--two-launch)


def run(cmd, log, extra_env=None):
    print("[profile] " + " ".join(cmd), flush=True)
    env = dict(os.environ, TMPDIR="/tmp", **(extra_env or {}))
    with open(log, "w") as f:
        p = subprocess.run(cmd, cwd="/tmp", env=env, stdout=f, stderr=subprocess.STDOUT, timeout=600)
    print(f"[profile] exit {p.returncode}", flush=True)
    return p.returncode


def rows_from(outdir, stem):
    """Rows of a rocprofv3 CSV (any *<stem>.csv under outdir), else None."""
    files = glob.glob(os.path.join(outdir, "**", f"*{stem}.csv"), recursive=True)
    if not files:
        return None
    with open(files[0]) as f:
        return list(csv.DictReader(f))


def db_rows(outdir, query):
    files = glob.glob(os.path.join(outdir, "**", "*.db"), recursive=True)
    if not files:
        return []
    return sqlite3.connect(files[0]).execute(query).fetchall()


def kernel_stats(outdir):
    rows = rows_from(outdir, "kernel_stats")
    out = {}
    if rows:
        for r in rows:
            out[r["Name"]] = (int(r["Calls"]), float(r["AverageNs"]))
        return out
    acc = defaultdict(list)
    for name, dur in db_rows(outdir, "select kernel_name, duration from kernels"):
        acc[name].append(dur)
    return {k: (len(v), sum(v) / len(v)) for k, v in acc.items()}


def counter_means(outdir, counter):
    rows = rows_from(outdir, "counter_collection")
    acc = defaultdict(list)
    if rows:
        for r in rows:
            if r.get("Counter_Name") == counter:
                acc[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    else:
        for name, cname, v in db_rows(outdir, "select kernel_name, counter_name, value from counters_collection"):
            if cname == counter:
                acc[name].append(v)
    return {k: (len(v), sum(v) / len(v)) for k, v in acc.items()}


def kernel_of(name):
    """The kernel's base name (`void kq::k_moe_gu<8, 2>(...)` -> `k_moe_gu`)."""
    base = name.split("(")[0].split("<")[0].strip()
    return base.split("::")[-1].split(" ")[-1]


def pick(d, sub):
    return [(k, v) for k, v in d.items() if kernel_of(k) == sub]


PHASES = ["layer start (first workgroup = 0)", "routing and x in", "gate/up loads issued", "x staged (q8_1 in LDS)",
          "wave 0's gate/up dots done", "down loads issued", "h published", "first h poll issued (polling wave)",
          "slot's h seen (polling wave)", "h staged as q8_1", "down partials published", "eight partials seen",
          "y written", "stack: previous y poll started; normed: sum of squares done",
          "stack: previous y seen; normed: xn staged", "router logits seen (normed)"]


def phases(args, out):
    """Run bench.py on the measurement build, write the phase table."""
    import numpy as np
    lib = os.path.join(REPO, "katali-lab_amd", "libkatali_hip_stamps.so")
    if not os.path.exists(lib):
        sys.exit(f"{lib} missing: python katali-lab_amd/build.py --stamps")
    npy = os.path.join(out, "stamps.npy")
    extra = ["--stacked"] if args.stacked else []
    extra += ["--normed-layer"] if args.normed_layer else []
    extra += ["--given-routing"] if args.given_routing else []
    cmd = [sys.executable, os.path.join(REPO, "bench.py"), "--workload", args.workload, "--steps", str(args.steps),
           "--warmup", str(args.warmup), "--no-cpu-baseline", "--dump-stamps", npy] + extra
    if not args.summarize_only and run(cmd, os.path.join(out, "phases.log"), {"KATALI_HIP_DLL": lib}) != 0:
        sys.exit(f"bench run failed (see {out}/phases.log)")
    st = np.load(npy).astype(np.int64)          # [64 layer slots][256 workgroups][16 phases], 10 ns ticks
    slots = [l for l in range(st.shape[0]) if (st[l, :, 0] > 0).all() and (st[l, :, 12] > 0).any()]
    t0 = {l: int(st[l, :, 0].min()) for l in slots}
    order = sorted(slots, key=lambda l: t0[l])
    med, mx = [[] for _ in PHASES], [[] for _ in PHASES]
    for l in slots:
        for p in range(len(PHASES)):
            v = st[l, :, p]
            v = v[v > 0]
            if v.size:
                rel = (v - t0[l]) / 100.0
                med[p].append(float(np.median(rel)))
                mx[p].append(float(rel.max()))
    period = [(t0[b] - t0[a]) / 100.0 for a, b in zip(order, order[1:]) if 0 < t0[b] - t0[a] < 10000]
    gap = [(t0[b] - int(st[a, :, 12].max())) / 100.0 for a, b in zip(order, order[1:])
           if 0 < t0[b] - t0[a] < 10000]
    name = f"phases_{args.workload}" + ("_stacked" if args.stacked else "") + ("_normed" if args.normed_layer else "") \
        + ("_given" if args.given_routing else "")
    md = os.path.join(REPO, "profiles", f"{name}.md")
    flags = (" --stacked" if args.stacked else "") + (" --normed-layer" if args.normed_layer else "") \
        + (" --given-routing" if args.given_routing else "")
    with open(md, "w") as f:
        f.write(f"# Phase stamps: {args.workload}{flags}\n\n")
        f.write(f"Made by `python katali-lab_amd/build.py --stamps && python katali-lab_amd/profile_bench.py "
                f"--workload {args.workload} --steps {args.steps} --warmup {args.warmup} --out <out> --phases{flags}`, "
                f"which runs `KATALI_HIP_DLL=katali-lab_amd/libkatali_hip_stamps.so python3 bench.py --workload "
                f"{args.workload} --steps {args.steps} --warmup {args.warmup} --no-cpu-baseline --dump-stamps "
                f"<out>/stamps.npy{flags}` (the measurement build: the one-launch layers record s_memrealtime, "
                f"100 MHz, at each phase; wave 0 of every workgroup, the first polling wave for the h polls).\n\n")
        f.write(f"{len(slots)} layers of the timed replays. Times in us after the layer's first workgroup "
                f"started; per layer the median and the latest over its 256 workgroups, then the median over "
                f"the layers.\n\n")
        f.write("| phase | median workgroup | latest workgroup |\n|---|---|---|\n")
        for p, label in enumerate(PHASES):
            if med[p]:
                f.write(f"| {p}: {label} | {np.median(med[p]):.2f} | {np.median(mx[p]):.2f} |\n")
        if period:
            f.write(f"\nLayer period (first workgroup to the next layer's first workgroup): median "
                    f"{np.median(period):.2f} us over {len(period)} layer pairs; from the last y written to the next "
                    f"layer's first workgroup: median {np.median(gap):.2f} us.\n")
    print(open(md).read())


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="moe48", choices=sorted(KERNELS))
    ap.add_argument("--steps", type=int, default=8)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--out", required=True, help="directory for the raw rocprofv3 output")
    ap.add_argument("--summarize-only", action="store_true", help="parse an existing --out tree, run nothing")
    ap.add_argument("--fused", action="store_true",
                    help="the all-slots one-launch MoE layer (KATALI_HIP_FUSED=1, KATALI_HIP_XCD=0; moe48 and "
                         "moe40cold)")
    ap.add_argument("--two-launch", action="store_true",
                    help="moe48, moe40cold: kernels A and B instead of the XCD-sliced layer (KATALI_HIP_XCD=0)")
    ap.add_argument("--phases", action="store_true",
                    help="moe48, moe40cold, moe48tok: the measurement build's phase stamps (no profiler)")
    ap.add_argument("--stacked", action="store_true", help="with --phases: bench.py --stacked")
    ap.add_argument("--normed-layer", action="store_true", help="with --phases: bench.py --normed-layer")
    ap.add_argument("--given-routing", action="store_true",
                    help="with --phases: bench.py --given-routing (the selection passed with each call)")
    ap.add_argument("--one-stream", action="store_true",
                    help="moebatch: the grouped GEMM on the library stream (KATALI_HIP_ONE_STREAM=1), so "
                         "per-kernel times add up to the layer")
    args = ap.parse_args()
    wl = args.workload
    extra_env = {}
    kernels, profile_name, traffic_name = KERNELS[wl], PROFILE_NAME.get(wl, "_".join(KERNELS[wl]) + "_" + wl), wl
    if args.fused:
        if wl not in ("moe48", "moe40cold"):
            sys.exit("--fused applies to moe48 and moe40cold")
        extra_env = {"KATALI_HIP_FUSED": "1", "KATALI_HIP_XCD": "0"}
        kernels, profile_name, traffic_name = ("k_moe_fused",), "k_moe_fused_" + wl, "fused_" + wl
    if args.two_launch:
        if wl not in ("moe48", "moe40cold"):
            sys.exit("--two-launch applies to moe48 and moe40cold")
        extra_env = {"KATALI_HIP_XCD": "0"}
        kernels, profile_name, traffic_name = ("k_moe_gu", "k_moe_down"), "k_moe_gu_k_moe_down_" + wl, "two_launch_" + wl
    if args.one_stream:
        if wl != "moebatch":
            sys.exit("--one-stream applies to moebatch")
        extra_env = {"KATALI_HIP_ONE_STREAM": "1"}
        profile_name, traffic_name = profile_name + "_one_stream", wl + "_one_stream"
    out = os.path.join(os.path.abspath(args.out), traffic_name)   # rocprofv3 runs from /tmp
    os.makedirs(out, exist_ok=True)
    if args.phases:
        phases(args, out)
        return
    bench = [sys.executable, os.path.join(REPO, "bench.py"), "--workload", wl, "--steps", str(args.steps),
             "--warmup", str(args.warmup), "--no-cpu-baseline", "--calibrate-copy", str(COPY_MIB)] + \
        EXTRA_ARGS.get(wl, [])
    cmds = {
        "trace": ["rocprofv3", "--kernel-trace", "--stats", "--output-format", "csv", "-d", os.path.join(out, "trace"),
                  "-o", "run", "--"] + bench,
        "fetch": ["rocprofv3", "--pmc", "FETCH_SIZE", "--output-format", "csv", "-d", os.path.join(out, "fetch"),
                  "-o", "run", "--"] + bench,
        "write": ["rocprofv3", "--pmc", "WRITE_SIZE", "--output-format", "csv", "-d", os.path.join(out, "write"),
                  "-o", "run", "--"] + bench,
    }
    if wl == "moebatch":   # the int8 MFMA kernels: MFMA busy share and int8 MFMA ops, from counters
        cmds["mfma"] = ["rocprofv3", "--pmc", "MfmaUtil", "SQ_INSTS_VALU_MFMA_MOPS_I8", "--output-format", "csv",
                        "-d", os.path.join(out, "mfma"), "-o", "run", "--"] + bench
    for k, c in cmds.items():
        if args.summarize_only:
            break
        if run(c, os.path.join(out, f"{k}.log"), extra_env) not in (0, 139):   # 139: profiler's own exit after results
            sys.exit(f"rocprofv3 {k} run failed (see {out}/{k}.log)")
    stats = kernel_stats(os.path.join(out, "trace"))
    fetch = counter_means(os.path.join(out, "fetch"), "FETCH_SIZE")
    write = counter_means(os.path.join(out, "write"), "WRITE_SIZE")
    mfma = counter_means(os.path.join(out, "mfma"), "MfmaUtil") if "mfma" in cmds else {}
    mops = counter_means(os.path.join(out, "mfma"), "SQ_INSTS_VALU_MFMA_MOPS_I8") if "mfma" in cmds else {}
    copy_bytes = COPY_MIB << 20
    cf = pick(fetch, "k_copy")
    cw = pick(write, "k_copy")
    if not cf or not cw:
        sys.exit("calibration copy kernel missing from the counter runs")
    f_scale = copy_bytes / cf[0][1][1]     # bytes per counter unit
    w_scale = copy_bytes / cw[0][1][1]
    # per workload unit: every kernel's calls relative to the first kernel's
    # (one launch per unit), times its mean duration and traffic per dispatch
    ref = pick(stats, kernels[0])
    if not ref:
        sys.exit(f"{kernels[0]} missing from the trace")
    units = sum(c for _, (c, _) in ref)
    unit_fetch = unit_write = unit_time = 0.0
    table = []
    for sub in kernels:
        for name, (calls, avg) in pick(stats, sub):
            fb = fetch[name][1] * f_scale if name in fetch else float("nan")
            wb = write[name][1] * w_scale if name in write else float("nan")
            per = calls / units
            table.append((name, calls, avg / 1e3, fb, wb))
            unit_fetch += fb * per
            unit_write += wb * per
            unit_time += avg / 1e3 * per
    traffic = unit_fetch + unit_write
    md = os.path.join(REPO, "profiles", f"{profile_name}.md")
    os.makedirs(os.path.dirname(md), exist_ok=True)
    with open(md, "w") as f:
        f.write(f"# rocprofv3 summary: {wl}\n\n")
        flags = (" --fused" if args.fused else "") + (" --one-stream" if args.one_stream else "")
        env = "".join(f", {k}={v}" for k, v in extra_env.items())
        f.write(f"Made by `python katali-lab_amd/profile_bench.py --workload {wl} --steps {args.steps} "
                f"--warmup {args.warmup} --out <out>{flags}`, which runs (from /tmp, "
                f"TMPDIR=/tmp{env}; paths relative to the repository root):\n\n")
        for k, c in cmds.items():
            txt = " ".join(c).replace(out, "<out>").replace(REPO + "/", "").replace(sys.executable, "python3")
            f.write(f"- {k}: `{txt}`\n")
        f.write(f"\nCalibration: one k_copy of {copy_bytes} B read + {copy_bytes} B written reads "
                f"FETCH_SIZE {cf[0][1][1]:.1f} and WRITE_SIZE {cw[0][1][1]:.1f} (KiB units): "
                f"{f_scale:.2f} and {w_scale:.2f} bytes per counter unit.\n\n")
        if mfma:
            f.write("MFMA counters (mfma run): MfmaUtil = SQ_VALU_MFMA_BUSY_CYCLES summed over SIMDs / "
                    "(GRBM_GUI_ACTIVE x SIMDs) in percent, over each dispatch; SQ_INSTS_VALU_MFMA_MOPS_I8 "
                    "per dispatch (units of 512 int8 ops).\n\n")
            f.write("| kernel | MfmaUtil % | MOPS_I8 per dispatch |\n|---|---|---|\n")
            for sub in kernels:
                for name, _ in pick(stats, sub):
                    if name in mfma:
                        f.write(f"| {name} | {mfma[name][1]:.2f} | {mops.get(name, (0, float('nan')))[1]:,.0f} |\n")
            f.write("\n")
        f.write("| kernel | calls | avg us | HBM fetch B/dispatch | HBM write B/dispatch |\n|---|---|---|---|---|\n")
        for name, calls, us, fb, wb in table:
            f.write(f"| {name} | {calls} | {us:.2f} | {fb:,.0f} | {wb:,.0f} |\n")
        f.write(f"\nPer workload unit ({UNIT_NAME[wl]}; {units} units in the trace run, each kernel weighted by "
                f"its calls per unit): kernel time {unit_time:.2f} us, HBM traffic {traffic:,.0f} B "
                f"(fetch {unit_fetch:,.0f} + write {unit_write:,.0f}).\n\n")
        f.write("All kernels in the trace run (calls, avg us):\n\n")
        for name, (calls, avg) in sorted(stats.items(), key=lambda kv: -kv[1][0] * kv[1][1]):
            f.write(f"- {name[:110]}: {calls}, {avg / 1e3:.2f}\n")
    with open(os.path.join(REPO, "profiles", f"traffic_{traffic_name}.txt"), "w") as f:
        f.write(f"# HBM bytes per {UNIT_NAME[wl]} from {os.path.basename(md)}\n")
        f.write(f"traffic_bytes_per_unit: {traffic:.0f}\n")
    print(open(md).read())


if __name__ == "__main__":
    main()
