#!/usr/bin/env python3
"""Per-call busy / gap, per-stage shares, roofline and HBM traffic from rocprofv3 output.

The MI355X counterpart of the reference's scripts/analysis/nsys_report.py (per-call launch / busy /
gap breakdown), ncu_report.py (per-kernel hardware counters) and roofline.py (achieved vs peak).
It reads rocprofv3 CSV output only; nothing here runs on the GPU.

Inputs
  trace        <prefix>_kernel_trace.csv of `rocprofv3 --kernel-trace --output-format csv`
  --fetch / --write        counter_collection.csv of a `--pmc FETCH_SIZE` / `--pmc WRITE_SIZE` run
  --copy-fetch / --copy-write   the same counters over a plain device copy of --copy-bytes read and
                           written per dispatch (`bench.py --probe-copy`): the counters' scale
  --workload G,m,n,k,N[,beta]   a uniform group, for the algorithmic bytes / operations per launch

Calls.  The library's kernels are classified by name into stages (prep, i8_gemm, reconstruct,
native, memops).  A call starts at every prep kernel, and at a native FP64 kernel that follows
another native kernel; any other kernel between library kernels ends the current call.  Per call:
  span   first kernel start -> last kernel end
  busy   union of the call's kernel intervals
  gap    span - busy (device idle between the call's kernels)
  <stage> busy time of the stage's kernels
Per kernel: launches, average / min / max duration, and with --workload the roofline figure
(achieved = algorithmic bytes or operations per launch / average duration; peaks: HBM 8 TB/s,
dense INT8 5.0 POP/s).  With counter files: HBM bytes per launch = FETCH_SIZE / f + WRITE_SIZE / w
(KiB), f and w the counters' readings for the calibration copy divided by its true KiB.

Usage
  python3 rocprof_report.py out/run_kernel_trace.csv --workload 64,1024,1024,1024,15,0.5 \\
      [--fetch f/run_counter_collection.csv --write w/... --copy-fetch cf/... --copy-write cw/...] \\
      [-o report.md] [--csv report.csv]
"""
import argparse
import csv
import json
import os
import re
import statistics
import sys

HBM_PEAK = 8.0e12      # MI355X HBM3E, bytes / s
INT8_PEAK = 5.0e15     # MI355X dense INT8 MFMA, operations / s
FP64_PEAK = 78.6e12    # MI355X dense FP64 MFMA, flop / s

STAGES = ("prep", "i8_gemm", "reconstruct", "native", "memops")
_STAGE_RE = [
    (re.compile(r"\bprep_kernel\b"), "prep"),
    (re.compile(r"\bi8_(grouped|large)(_persistent)?_kernel\b"), "i8_gemm"),
    (re.compile(r"\b(recon|dots|gather|cross)_kernel\b"), "reconstruct"),
    (re.compile(r"\bf64_\w*kernel\b"), "native"),
    (re.compile(r"copyBuffer|fillBuffer|__amd_rocclr"), "memops"),
]


# The kernel of each stage that the stage's algorithmic amount is credited to.  The reconstruct
# stage's other kernels (dots_kernel, gather_kernel and cross_kernel: the FP64 dot products of flagged entries) do
# work that depends on the data (how many entries the certificate rejects), so they get no roofline
# column.
ALG_KERNEL = {"prep": r"\bprep_kernel\b", "i8_gemm": r"\bi8_", "reconstruct": r"\brecon_kernel\b"}


def stage_of(name):
    """Stage of a kernel by name, or None for kernels that are not the library's."""
    for rx, st in _STAGE_RE:
        if rx.search(name):
            return st
    return None


def short_name(name):
    """Kernel name without the return type, namespaces and parameter list (template arguments kept)."""
    base = name.replace("(anonymous namespace)::", "").split("(")[0].strip()
    base = re.sub(r"^void\s+", "", base)
    head, sep, tmpl = base.partition("<")
    return head.split("::")[-1] + sep + tmpl


def read_trace(path):
    """Kernel dispatches [(name, start_ns, end_ns)] sorted by start."""
    out = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r.get("Kind", "KERNEL_DISPATCH") != "KERNEL_DISPATCH":
                continue
            out.append((r["Kernel_Name"], int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    out.sort(key=lambda x: x[1])
    return out


def union_length(intervals):
    """Total length covered by a set of [start, end) intervals."""
    tot, cur_s, cur_e = 0, None, None
    for s, e in sorted(intervals):
        if cur_e is None or s > cur_e:
            if cur_e is not None:
                tot += cur_e - cur_s
            cur_s, cur_e = s, e
        else:
            cur_e = max(cur_e, e)
    if cur_e is not None:
        tot += cur_e - cur_s
    return tot


def split_calls(kernels):
    """Group the library's dispatches into calls (see the module docstring)."""
    calls, cur, prev_stage = [], None, None
    for name, s, e in kernels:
        st = stage_of(name)
        if st is None or st == "memops":
            if st is None and cur is not None:   # a foreign kernel ends the call
                calls.append(cur)
                cur, prev_stage = None, None
            continue
        new = st == "prep" or (st == "native" and prev_stage == "native") or cur is None
        if new and cur is not None:
            calls.append(cur)
        if new:
            cur = []
        cur.append((st, s, e))
        prev_stage = st
    if cur:
        calls.append(cur)
    return calls


def call_metrics(call):
    span = max(e for _, _, e in call) - min(s for _, s, _ in call)
    busy = union_length([(s, e) for _, s, e in call])
    m = {"kernels": len(call), "span_us": span / 1e3, "busy_us": busy / 1e3, "gap_us": (span - busy) / 1e3}
    for st in STAGES:
        m[st + "_us"] = union_length([(s, e) for k, s, e in call if k == st]) / 1e3
    return m


def kernel_table(kernels):
    """{short name: (stage, launches, avg_us, min_us, max_us)} over the library's kernels."""
    d = {}
    for name, s, e in kernels:
        st = stage_of(name)
        if st is None:
            continue
        d.setdefault(short_name(name), (st, []))[1].append((e - s) / 1e3)
    return {k: (st, len(v), statistics.fmean(v), min(v), max(v)) for k, (st, v) in d.items()}


def algorithmic(workload):
    """Per-launch algorithmic quantities of a uniform group: {stage: (amount, unit, peak)}."""
    G, m, n, k, N = (int(x) for x in workload[:5])
    beta = float(workload[5]) if len(workload) > 5 else 0.0
    kp = (k + 31) // 32 * 32
    planes = N + 1
    prep = G * (8.0 * (m * k + k * n) + planes * (m + n) * kp + 16.0 * (m + n))
    ops = G * planes * 2.0 * m * n * kp
    recon = G * ((N + 4.0) * m * n + 8.0 * m * n * (2 if beta != 0 else 1) + 16.0 * (m + n))
    return {"prep": (prep, "B", HBM_PEAK), "i8_gemm": (ops, "op", INT8_PEAK), "reconstruct": (recon, "B", HBM_PEAK)}


def read_counter(path, counter):
    """{short kernel name: [per-dispatch value]} of one counter."""
    d = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            d.setdefault(short_name(r["Kernel_Name"]), []).append(float(r["Counter_Value"]))
    return d


def copy_factor(path, counter, true_kib):
    """Counter reading per true KiB for the calibration copy (its largest dispatch)."""
    vals = [v for k, vs in read_counter(path, counter).items() if "copyBuffer" in k for v in vs]
    if not vals:
        raise SystemExit(f"{path}: no copy dispatch with {counter}")
    return max(vals) / true_kib


def traffic_detail(args):
    """{kernel: record} per dispatch: mean FETCH_SIZE / WRITE_SIZE (KiB), the copy factors and the
    calibrated read / write bytes; {} without counter files."""
    if not (args.fetch and args.write):
        return {}
    kib = args.copy_bytes / 1024.0
    ff = copy_factor(args.copy_fetch, "FETCH_SIZE", kib) if args.copy_fetch else 1.0
    fw = copy_factor(args.copy_write, "WRITE_SIZE", kib) if args.copy_write else 1.0
    fe, wr = read_counter(args.fetch, "FETCH_SIZE"), read_counter(args.write, "WRITE_SIZE")
    out = {}
    for k in fe:
        if stage_of(k) in (None, "memops") or k not in wr:
            continue
        f_kib, w_kib = statistics.fmean(fe[k]), statistics.fmean(wr[k])
        out[k] = {"fetch_kib": f_kib, "write_kib": w_kib, "fetch_factor": ff, "write_factor": fw,
                  "read_bytes": f_kib / ff * 1024.0, "write_bytes": w_kib / fw * 1024.0}
    return out


def traffic(args):
    """{kernel: (read_bytes, write_bytes)} per dispatch, or {} without counter files."""
    return {k: (r["read_bytes"], r["write_bytes"]) for k, r in traffic_detail(args).items()}


def write_traffic_json(args, kt):
    """Record the HBM bytes per launch of the busiest kernel of stage args.traffic_stage (the INT8
    GEMM by default, prep for a call whose dominant kernel is prep) under args.traffic_key in
    args.traffic_json (the figure bench.py reports as roofline.traffic); other keys of an existing
    file are kept."""
    det = traffic_detail(args)
    stage = getattr(args, "traffic_stage", None) or "i8_gemm"
    gemm = [k for k in det if stage_of(k) == stage]
    if not gemm:
        raise SystemExit(f"--traffic-json: no {stage} kernel with FETCH_SIZE and WRITE_SIZE counters")
    k = max(gemm, key=lambda g: kt[g][1] * kt[g][2] if g in kt else 0.0)   # most busy time
    r = det[k]
    rec = {"kernel": k, "fetch_kib": r["fetch_kib"], "write_kib": r["write_kib"], "fetch_factor": r["fetch_factor"],
           "write_factor": r["write_factor"], "traffic_bytes": int(round(r["read_bytes"] + r["write_bytes"]))}
    data = {}
    if os.path.exists(args.traffic_json):
        with open(args.traffic_json) as f:
            data = json.load(f)
    data[args.traffic_key] = rec
    with open(args.traffic_json, "w") as f:
        json.dump(data, f, indent=1)
        f.write("\n")
    return rec


def fmt(x, nd=1):
    return "-" if x is None else f"{x:.{nd}f}"


def report(args):
    kernels = read_trace(args.trace)
    calls = [call_metrics(c) for c in split_calls(kernels)]
    kt = kernel_table(kernels)
    alg = algorithmic(args.workload.split(",")) if args.workload else {}
    tr = traffic(args)
    lines = [f"# rocprofv3 report: {args.trace}", ""]
    if calls:
        med = {key: statistics.median(c[key] for c in calls) for key in calls[0]}
        lines += ["## Calls (median over %d)" % len(calls), "",
                  "| kernels | span (us) | busy (us) | gap (us) | " + " | ".join(f"{s} (us)" for s in STAGES) + " |",
                  "|---" * (4 + len(STAGES)) + "|",
                  f"| {med['kernels']:.0f} | {med['span_us']:.1f} | {med['busy_us']:.1f} | {med['gap_us']:.1f} | "
                  + " | ".join(f"{med[s + '_us']:.1f}" for s in STAGES) + " |", ""]
        if med["busy_us"] > 0:
            lines += ["Busy share: " + ", ".join(f"{s} {100 * med[s + '_us'] / med['busy_us']:.1f} %"
                                                for s in STAGES if med[s + "_us"] > 0), ""]
    lines += ["## Kernels", "", "| kernel | stage | launches | avg (us) | min (us) | max (us) | achieved | % of peak |"
              " HBM read / write per launch (GB) |", "|---|---|---|---|---|---|---|---|---|"]
    rows = []
    for k, (st, n, avg, mn, mx) in sorted(kt.items(), key=lambda kv: -kv[1][1] * kv[1][2]):
        ach = frac = None
        unit = ""
        if st in alg and re.search(ALG_KERNEL[st], k):
            amount, u, peak = alg[st]
            ach = amount / (avg * 1e-6)
            frac = ach / peak
            unit = "TB/s" if u == "B" else "TOP/s"
        rw = tr.get(k)
        rows.append({"kernel": k, "stage": st, "launches": n, "avg_us": avg, "min_us": mn, "max_us": mx,
                     "achieved": ach / 1e12 if ach else None, "unit": unit, "frac": frac,
                     "hbm_read_gb": rw[0] / 1e9 if rw else None, "hbm_write_gb": rw[1] / 1e9 if rw else None})
        lines.append(f"| {k} | {st} | {n} | {avg:.1f} | {mn:.1f} | {mx:.1f} | "
                     f"{fmt(ach / 1e12 if ach else None, 2)} {unit} | {fmt(100 * frac if frac else None)} | "
                     f"{fmt(rw[0] / 1e9 if rw else None, 3)} / {fmt(rw[1] / 1e9 if rw else None, 3)} |")
    if args.workload:
        lines += ["", f"Workload {args.workload} (G,m,n,k,N[,beta]); peaks: HBM {HBM_PEAK / 1e12:.0f} TB/s, "
                  f"INT8 {INT8_PEAK / 1e15:.1f} POP/s."]
    text = "\n".join(lines) + "\n"
    if args.out:
        with open(args.out, "w") as f:
            f.write(text)
    else:
        sys.stdout.write(text)
    if getattr(args, "traffic_json", None):
        write_traffic_json(args, kt)
    if args.csv:
        with open(args.csv, "w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=list(rows[0].keys()) if rows else ["kernel"])
            w.writeheader()
            w.writerows(rows)
    return calls, rows


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("trace", help="rocprofv3 <prefix>_kernel_trace.csv")
    ap.add_argument("--workload", help="G,m,n,k,N[,beta] of a uniform group")
    ap.add_argument("--fetch", help="counter_collection.csv of a FETCH_SIZE run")
    ap.add_argument("--write", help="counter_collection.csv of a WRITE_SIZE run")
    ap.add_argument("--copy-fetch", help="FETCH_SIZE over the calibration copy")
    ap.add_argument("--copy-write", help="WRITE_SIZE over the calibration copy")
    ap.add_argument("--copy-bytes", type=float, default=float(1 << 30), help="bytes read (= written) per copy")
    ap.add_argument("-o", "--out", help="markdown output (default stdout)")
    ap.add_argument("--csv", help="per-kernel CSV output")
    ap.add_argument("--traffic-json", help="record the INT8 GEMM's HBM bytes per launch in this JSON file")
    ap.add_argument("--traffic-key", default="uniform", help="workload key of that record")
    ap.add_argument("--traffic-stage", default="i8_gemm", choices=["i8_gemm", "prep"],
                    help="stage whose busiest kernel the record is for")
    report(ap.parse_args(argv))


if __name__ == "__main__":
    main()
