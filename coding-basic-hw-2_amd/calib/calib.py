"""Planner cost-model calibration on this GPU: measures, fits and writes params_<arch>.json.

The flow of the reference's bench/calib/calib.cu (microbenchmarks -> CSV rows) and
bench/calib/fit.py (CSV -> parameters), with this library's own kernels in place of cuBLAS and
cuBLASLt:
  dgemm  : the native FP64 path (ggemm_grouped_dgemm, NATIVE_GROUPED), one square problem;
  i8gemm : the INT8 GEMM stage of the emulation (EMU_GROUPED, in-process stage timing), one square
           problem with its N + 1 planes; value = planes * 2 m n Kp / stage time;
  bw_copy / bw_read : a plain device copy / a full reduction of doubles;
  launch_stream : back-to-back launches of a one-element kernel;
  h2d_pinned : pinned host -> device copies.
Cost model (fit.py:7-14): emu = 3 t_launch + bytes_emu / bw + N 2mnk / i8_peak,
native = t_launch + 2mnk / f64_peak; peaks from a least-squares line t = t0 + work / peak over
the sizes >= 1024, plus the per-size rate tables.  The planner reads f64_peak_flops, i8_peak_ops
and bw_Bps (GGEMM_CALIB_JSON, GGEMM_CALIB_DIR, or this directory next to the library).

Usage: python3 calib.py [-o OUTDIR] [--csv FILE] [--max-dim 8192]
"""
import argparse
import ctypes as C
import json
import os
import re
import sys
import time
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))


def median(v):
    v = sorted(v)
    return v[len(v) // 2] if v else None


def linfit(xs, ys):
    """Least squares y = a + b x -> (a, b)."""
    n = len(xs)
    mx, my = sum(xs) / n, sum(ys) / n
    sxx = sum((x - mx) ** 2 for x in xs)
    if sxx == 0:
        return my, 0.0
    b = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sxx
    return my - b * mx, b


def event_time_us(torch, fn, iters, reps=5):
    """Median over reps of the per-iteration time of iters back-to-back calls (HIP events)."""
    out = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out.append(e0.elapsed_time(e1) * 1e3 / iters)
    return median(out)


def measure(max_dim):
    import torch
    import ggemm as G

    dev = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(0)
    meta = {"gpu": props.gcnArchName.split(":")[0], "sm_count": props.multi_processor_count,
            "cc": f"{props.major}.{props.minor}", "name": props.name}
    rows = []

    def row(kind, param, m, n, k, nbytes, iters, t_us, value, unit):
        rows.append({"kind": kind, "param": param, "m": m, "n": n, "k": k, "bytes": nbytes, "iters": iters,
                     "time_us": t_us, "value": value, "unit": unit})

    # launches
    x = torch.zeros(1, device=dev)
    t = event_time_us(torch, lambda: x.add_(1.0), 2000)
    row("launch_stream", "", 0, 0, 0, 0, 2000, t, 0.0, "us")
    for _ in range(3):
        t0 = time.perf_counter()
        for _ in range(200):
            x.add_(1.0)
            torch.cuda.synchronize()
        row("launch_sync", "", 0, 0, 0, 0, 200, (time.perf_counter() - t0) * 1e6 / 200, 0.0, "us")
    # pinned H2D
    for sz in [1 << 12, 1 << 16, 1 << 20, 1 << 24, 1 << 26]:
        h = torch.empty(sz, dtype=torch.uint8, pin_memory=True)
        d = torch.empty(sz, dtype=torch.uint8, device=dev)

        def cp():
            d.copy_(h, non_blocking=True)
            torch.cuda.synchronize()
        cp()
        t0 = time.perf_counter()
        for _ in range(20):
            cp()
        row("h2d_pinned", "", 0, 0, 0, sz, 20, (time.perf_counter() - t0) * 1e6 / 20, 0.0, "us")
    # bandwidth
    n = 1 << 27   # 1 GiB of doubles
    a = torch.ones(n, dtype=torch.float64, device=dev)
    b = torch.empty_like(a)
    t = event_time_us(torch, lambda: b.copy_(a), 5)
    row("bw_copy", "", 0, 0, 0, 16 * n, 5, t, 16 * n / (t * 1e-6) / 1e9, "GB/s")
    t = event_time_us(torch, lambda: a.sum(), 5)
    row("bw_read", "", 0, 0, 0, 8 * n, 5, t, 8 * n / (t * 1e-6) / 1e9, "GB/s")
    del a, b
    torch.cuda.empty_cache()

    dims = [d for d in [64, 128, 256, 512, 1024, 2048, 4096, 8192, 16384] if d <= max_dim]
    cfg_nat = G.Config(0, 1e-15, 1, 0)
    cfg_emu = G.Config(0, 1e-15, 1, G.REPAIR_OFF)
    for d in dims:
        A = torch.rand(d * d, dtype=torch.float64, device=dev) - 0.5
        B = torch.rand(d * d, dtype=torch.float64, device=dev) - 0.5
        Cm = torch.zeros(d * d, dtype=torch.float64, device=dev)
        probs = G.problems_array([G.Problem(d, d, d, A.data_ptr(), d, B.data_ptr(), d, Cm.data_ptr(), d, 1.0, 0.0)])
        with G.Handle(1, d * d, d * d, d * d) as h:
            st = G.Stats()

            def call(path, cfg):
                rc = G.lib().ggemm_grouped_dgemm(h.h, path, C.byref(cfg), probs, 1, C.byref(st))
                if rc:
                    raise RuntimeError(f"ggemm_grouped_dgemm rc={rc}")
            iters = max(3, min(200, int(2e11 / (2.0 * d ** 3))))
            call(G.PATH_NATIVE_GROUPED, cfg_nat)
            t = event_time_us(torch, lambda: call(G.PATH_NATIVE_GROUPED, cfg_nat), iters, reps=3)
            row("dgemm", "", d, d, d, 0, iters, t, 2.0 * d ** 3 / (t * 1e-6) / 1e9, "GFLOP/s")
            # INT8 stage of the emulation, from the in-process stage timers
            call(G.PATH_EMU_GROUPED, cfg_emu)
            planes = st.moduli_max + 1
            G.lib().ggemm_profile_enable(1)
            G.lib().ggemm_profile_read(None, None, 1)
            for _ in range(iters):
                call(G.PATH_EMU_GROUPED, cfg_emu)
            torch.cuda.synchronize()
            ms = (C.c_double * 4)()
            cnt = C.c_longlong(0)
            G.lib().ggemm_profile_read(ms, C.byref(cnt), 1)
            G.lib().ggemm_profile_enable(0)
            t_i8 = ms[1] / max(cnt.value, 1) * 1e3   # us
            kp = (d + 31) // 32 * 32
            ops = planes * 2.0 * d * d * kp
            row("i8gemm", f"planes={planes}", d, d, d, 0, iters, t_i8, ops / (t_i8 * 1e-6) / 1e9, "GOP/s")
        del A, B, Cm
        torch.cuda.empty_cache()
        print(f"  calib d={d} done", file=sys.stderr, flush=True)
    return meta, rows


def fit_gemm(rows, kind):
    pts = []
    for r in rows:
        if r["kind"] != kind or r["time_us"] <= 0:
            continue
        d = int(r["m"])
        ops = r["value"] * 1e9 * r["time_us"] * 1e-6   # the work the row's rate refers to
        pts.append((d, r["time_us"] * 1e-6, ops))
    if not pts:
        return None
    pts.sort()
    table = [{"mnk": d, "time_s": t, "rate_ops": w / t} for d, t, w in pts]
    best = max(p["rate_ops"] for p in table)
    big = [(w, t) for d, t, w in pts if d >= 1024] or [(w, t) for d, t, w in pts[-3:]]
    a, b = linfit([w for w, _ in big], [t for _, t in big])
    return {"peak_ops": best, "peak_ops_linfit": 1.0 / b if b > 0 else best, "t0_linfit_s": a, "table": table}


def fit(meta, rows):
    def sel(kind):
        return [r for r in rows if r["kind"] == kind]
    t_launch = median([r["time_us"] for r in sel("launch_stream")]) * 1e-6
    h2d = sorted((r["bytes"], r["time_us"] * 1e-6) for r in sel("h2d_pinned"))
    h2d_lat, h2d_inv = linfit([b for b, _ in h2d], [t for _, t in h2d]) if len(h2d) > 1 else (None, 0.0)
    bw = max(r["value"] for r in sel("bw_copy")) * 1e9
    f64 = fit_gemm(rows, "dgemm")
    i8 = fit_gemm(rows, "i8gemm")
    out = {
        "schema": "ggemm-calib-v1",
        "gpu": meta["gpu"], "sm_count": meta["sm_count"], "cc": meta["cc"], "device_name": meta.get("name", ""),
        "t_launch_s": t_launch,
        "bw_Bps": bw,
        "f64_peak_flops": f64["peak_ops_linfit"] if f64 else None,
        "i8_peak_ops": i8["peak_ops_linfit"] if i8 else None,
        "extra": {
            "t_launch_sync_us": median([r["time_us"] for r in sel("launch_sync")]),
            "h2d_pinned_latency_s": h2d_lat,
            "h2d_pinned_Bps": 1.0 / h2d_inv if h2d_inv > 0 else None,
            "bw_read_Bps": max(r["value"] for r in sel("bw_read")) * 1e9,
            "f64_peak_flops_max": f64["peak_ops"] if f64 else None,
            "i8_peak_ops_max": i8["peak_ops"] if i8 else None,
            "f64_t0_s": f64["t0_linfit_s"] if f64 else None,
            "i8_t0_s": i8["t0_linfit_s"] if i8 else None,
        },
        "f64_table": f64["table"] if f64 else [],
        "i8_table": i8["table"] if i8 else [],
        "model": {
            "emu": "3*t_launch_s + bytes_emu/bw_Bps + N*2*m*n*k/i8_peak_ops",
            "native": "t_launch_s + 2*m*n*k/f64_peak_flops",
            "bytes_emu": "8*(m*k+k*n) + N*(m+n)*Kp + 8*N*m*n + 8*m*n*(2 if beta!=0 else 1)",
            "Kp": "round_up(k,32)",
        },
    }
    if out["f64_peak_flops"] and out["i8_peak_ops"]:
        def emu(d, N):
            kp = (d + 31) // 32 * 32
            by = 8 * 2 * d * d + N * 2 * d * kp + 8 * N * d * d + 8 * d * d
            return 3 * t_launch + by / bw + N * 2.0 * d ** 3 / out["i8_peak_ops"]

        def nat(d):
            return t_launch + 2.0 * d ** 3 / out["f64_peak_flops"]
        out["crossover_square_pow2_by_N"] = {
            str(N): next((d for d in [2 ** i for i in range(4, 16)] if emu(d, N) < nat(d)), None)
            for N in range(6, 21)}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("-o", "--outdir", default=str(HERE))
    ap.add_argument("--csv", help="also write the measured rows (calib.cu's CSV format) here")
    ap.add_argument("--max-dim", type=int, default=8192)
    args = ap.parse_args()
    meta, rows = measure(args.max_dim)
    if args.csv:
        with open(args.csv, "w") as f:
            for key in ("gpu", "sm_count", "cc"):
                f.write(f"# {key},{meta[key]}\n")
            f.write("kind,param,m,n,k,bytes,iters,time_us,value,unit\n")
            for r in rows:
                f.write(f"{r['kind']},{r['param']},{r['m']},{r['n']},{r['k']},{r['bytes']},{r['iters']},"
                        f"{r['time_us']:.4f},{r['value']:.4f},{r['unit']}\n")
    out = fit(meta, rows)
    slug = re.sub(r"[^A-Za-z0-9]+", "_", meta["gpu"]).strip("_").lower()
    path = Path(args.outdir) / f"params_{slug}.json"
    path.write_text(json.dumps(out, indent=2) + "\n")
    print(path)
    print(json.dumps({k: out[k] for k in ("gpu", "sm_count", "t_launch_s", "bw_Bps", "f64_peak_flops",
                                           "i8_peak_ops")}, indent=2))


if __name__ == "__main__":
    main()
