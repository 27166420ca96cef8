"""Benchmark: grouped Ozaki-II FP64 GEMM (INT8 MFMA emulation) on one MI355X.

Metric: effective FP64 TFLOP/s = sum_g 2 m_g n_g k_g / t, t = wall time of one
ggemm_grouped_dgemm call (hipEvent-bracketed over K back-to-back calls on the handle's stream,
inputs resident in HBM), reported with % of the INT8 MFMA peak, % of the FP64 MFMA peak and the
max certified error (sampled entries vs an 80-bit host reference).

Default workload = the uniform group G=64, m=n=k=1024, entries (U-0.5) exp(0.5 Z), alpha=1,
beta=0.5 with random C, adaptive moduli at 1e-15, fallback allowed, repair ON, through the
grouped emulation path (GGEMM_PATH_EMU_GROUPED).  --workload large runs G=8 x 8192 x 8192 x 16384.
Prints ONE JSON line.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "coding-basic-hw-2_amd"))

INT8_PEAK_TOPS = 5000.0     # MI355X dense INT8 MFMA, TOP/s
FP64_PEAK_TFLOPS = 78.6     # MI355X FP64 MFMA, TFLOP/s
HBM_PEAK_GBS = 8000.0

WORKLOADS = {
    # name: (G, m, n, k, phi, alpha, beta, seed offset, path)
    "uniform": dict(G=64, m=1024, n=1024, k=1024, phi=0.5, alpha=1.0, beta=0.5, seed=1,
                    desc="uniform group G=64, m=n=k=1024, (U-0.5)exp(0.5Z), alpha=1, beta=0.5, adaptive N at 1e-15"),
    "large": dict(G=8, m=8192, n=8192, k=16384, phi=0.0, alpha=1.0, beta=0.0, seed=3, graph=True,
                  desc="large group G=8, m=n=8192, k=16384, U(-1,1), alpha=1, beta=0, adaptive N at 1e-15, "
                       "repeated via plan/execute (hipGraph) with pointer updates between runs"),
    "plumbing": dict(G=1, m=256, n=256, k=256, phi=0.0, alpha=1.0, beta=0.0, seed=0,
                     desc="single 256^3, U(-0.5,0.5), fixed N=14"),
}


def splitmix_uniform(torch, seed, count, device, salt):
    """Counter-based SplitMix64 on the device: u[i] = (mix(seed + (3 i + salt) gamma) >> 11) 2^-53."""
    g = 0x9E3779B97F4A7C15 - (1 << 64)   # as int64
    i = torch.arange(count, dtype=torch.int64, device=device)
    z = (seed + (3 * i + salt) * g)

    def srl(x, s):
        return (x >> s) & ((1 << (64 - s)) - 1)

    z = (z ^ srl(z, 30)) * (0xBF58476D1CE4E5B9 - (1 << 64))
    z = (z ^ srl(z, 27)) * (0x94D049BB133111EB - (1 << 64))
    z = z ^ srl(z, 31)
    return srl(z, 11).to(torch.float64) * 2.0 ** -53


def fill(torch, out, phi, seed, salt, lo_hi=None):
    """(U - 0.5) exp(phi Z) with Z from Box-Muller; lo_hi=(a, b) gives U(a, b) instead."""
    n = out.numel()
    step = 1 << 26
    for s0 in range(0, n, step):
        cnt = min(step, n - s0)
        u = splitmix_uniform(torch, seed + s0 * 7, cnt, out.device, salt)
        if lo_hi is not None:
            v = lo_hi[0] + (lo_hi[1] - lo_hi[0]) * u
        else:
            v = u - 0.5
            if phi:
                u1 = 1.0 - splitmix_uniform(torch, seed + s0 * 7, cnt, out.device, salt + 1)
                u2 = splitmix_uniform(torch, seed + s0 * 7, cnt, out.device, salt + 2)
                z = torch.sqrt(-2.0 * torch.log(u1)) * torch.cos(2 * np.pi * u2)
                v = v * torch.exp(phi * z)
        out.view(-1)[s0:s0 + cnt] = v


def measured_traffic(workload, kernel):
    """HBM bytes per launch of the INT8 GEMM kernel from the committed rocprofv3 counter summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by its plain-copy calibration), or None
    when no summary exists for this workload and kernel."""
    f = REPO / "profiles" / "hbm_traffic.json"
    try:
        rec = json.loads(f.read_text()).get(workload)
    except (OSError, ValueError):
        return None
    if not rec or rec.get("kernel") != kernel:
        return None
    return rec.get("traffic_bytes")


def kp_of(k):
    return (k + 31) // 32 * 32


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="uniform", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-native", action="store_true")
    ap.add_argument("--probe-copy", action="store_true",
                    help="only run a plain 1 GiB device copy 5 times (calibrates the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import torch
    if args.probe_copy:
        # 5 timed copies (the counter calibration reads the copy dispatches only), then the stream
        # rates a memory-bound kernel can reach on this GPU: read-only (a sum) and write-only (a fill)
        src = torch.ones(1 << 30, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

        def rate(f, reps, nbytes):
            e0.record()
            for _ in range(reps):
                f()
            e1.record()
            torch.cuda.synchronize()
            return round(nbytes * reps / (e0.elapsed_time(e1) * 1e9), 3)

        dst.copy_(src)
        torch.cuda.synchronize()
        copy_tb = rate(lambda: dst.copy_(src), 4, 2 << 30)
        x = src.view(torch.float64)
        y = dst.view(torch.float64)
        x.sum()
        read_tb = rate(lambda: x.sum(), 10, 1 << 30)
        write_tb = rate(lambda: y.fill_(1.0), 10, 1 << 30)
        print(json.dumps({"probe": "copy", "bytes_read": 1 << 30, "bytes_written": 1 << 30, "launches": 5,
                          "copy_TB_s": copy_tb, "read_TB_s": read_tb, "write_TB_s": write_tb}))
        return
    import ggemm as G

    W = WORKLOADS[args.workload]
    Gp, m, n, k = W["G"], W["m"], W["n"], W["k"]
    dev = torch.device("cuda:0")
    seed = 20261201 + W["seed"]
    lda, ldb, ldc = m, k, m
    A = torch.empty((Gp, k, m), dtype=torch.float64, device=dev)   # per problem column-major m x k
    B = torch.empty((Gp, n, k), dtype=torch.float64, device=dev)
    Cm = torch.empty((Gp, n, m), dtype=torch.float64, device=dev)
    lo_hi = (-1.0, 1.0) if args.workload == "large" else None
    fill(torch, A, W["phi"], seed, 0, lo_hi)
    fill(torch, B, W["phi"], seed + 1, 10, lo_hi)
    fill(torch, Cm, 0.0, seed + 2, 20)
    C0 = Cm.clone() if W["beta"] != 0.0 else None
    torch.cuda.synchronize()

    def problems(Cbuf):
        return [G.Problem(m, n, k, A[g].data_ptr(), lda, B[g].data_ptr(), ldb, Cbuf[g].data_ptr(), ldc,
                          W["alpha"], W["beta"]) for g in range(Gp)]

    fixed_n = 14 if args.workload == "plumbing" else 0
    cfg = G.Config(fixed_n, 1e-15, 1, G.REPAIR_ON)
    path = G.PATH_EMU_GROUPED
    flops = 2.0 * Gp * m * n * k
    h = G.Handle(Gp, Gp * m * k, Gp * k * n, Gp * m * n)
    probs = G.problems_array(problems(Cm))
    st = G.Stats()

    def call():
        rc = G.lib().ggemm_grouped_dgemm(h.h, path, C.byref(cfg), probs, Gp, C.byref(st))
        if rc:
            raise RuntimeError(f"ggemm_grouped_dgemm rc={rc}")

    plan = None
    timed = call
    if W.get("graph"):
        # the call planned once (ggemm_make_plan: a hipGraph), then per step the output pointers are
        # updated -- alternating between two C buffers -- and the plan executed on the same stream
        Cm2 = torch.empty_like(Cm)
        err = C.c_int(0)
        plan = G.lib().ggemm_make_plan_ex(h.h, path, C.byref(cfg), probs, Gp, C.byref(err))
        if not plan:
            raise RuntimeError(f"ggemm_make_plan_ex failed: {err.value}")
        if G.lib().ggemm_plan_get_stats(plan, C.byref(st)):
            raise RuntimeError("ggemm_plan_get_stats failed")
        ptrs = lambda T: (C.c_void_p * Gp)(*[T[g].data_ptr() for g in range(Gp)])
        PA, PB, PC = ptrs(A), ptrs(B), (ptrs(Cm), ptrs(Cm2))
        step = [0]

        def timed():
            rc = G.lib().ggemm_plan_update_pointers(plan, PA, PB, PC[step[0] & 1])
            if rc == 0:
                rc = G.lib().ggemm_execute_plan(plan, None)
            if rc:
                raise RuntimeError(f"plan update / execute rc={rc}")
            step[0] += 1

    def reset_c():
        if C0 is not None:
            Cm.copy_(C0)

    # ---- timed region: K back-to-back calls (beta != 0 makes C drift; values are not checked here)
    for _ in range(args.warmup):
        timed()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        timed()
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ms = e0.elapsed_time(e1) / args.steps
    N = st.moduli_max
    planes = N + 1
    int8_ops = planes * 2.0 * Gp * m * n * kp_of(k)

    # ---- per-stage kernel durations (HIP events around each launch on the handle's stream)
    G.lib().ggemm_profile_enable(1)
    G.lib().ggemm_profile_read(None, None, 1)
    for _ in range(args.steps):
        call()
    torch.cuda.synchronize()
    stage = (C.c_double * 4)()
    ncalls = C.c_longlong(0)
    G.lib().ggemm_profile_read(stage, C.byref(ncalls), 1)
    G.lib().ggemm_profile_enable(0)
    i8_kernel = G.lib().ggemm_profile_i8_kernel().decode()
    st_ms = [stage[q] / max(ncalls.value, 1) for q in range(4)]
    i8_ms = st_ms[1]
    achieved = int8_ops / (i8_ms * 1e-3) / 1e12 if i8_ms > 0 else 0.0
    prep_bytes = Gp * (8.0 * (m * k + n * k) + planes * (m + n) * kp_of(k) + 16.0 * (m + n))
    # reconstruct: N digit bytes + the int32 abs-plane product per entry, C0 (beta != 0), C, shifts
    recon_bytes = Gp * ((N + 4.0) * m * n + 8.0 * m * n * (2 if W["beta"] != 0 else 1) + 16.0 * (m + n))

    if plan is not None:
        G.lib().ggemm_destroy_plan(plan)
        del Cm2
    h.close()   # free the timing workspace before the validation handle allocates its own

    # ---- validation call with device counters on (separate handle; syncs per call)
    os.environ["GGEMM_STATS_REPAIR"] = "1"
    hv = G.Handle(Gp, Gp * m * k, Gp * k * n, Gp * m * n)
    del os.environ["GGEMM_STATS_REPAIR"]
    reset_c()
    torch.cuda.synchronize()
    stv = G.Stats()
    rc = G.lib().ggemm_grouped_dgemm(hv.h, path, C.byref(cfg), probs, Gp, C.byref(stv))
    torch.cuda.synchronize()
    assert rc == 0
    # sampled componentwise error vs an 80-bit host reference
    rng = np.random.default_rng(7)
    ns = 256 if args.workload != "large" else 64
    worst_gamma = worst_norm = 0.0
    u = 2.0 ** -53
    nt = k + (W["alpha"] != 1.0) + (W["beta"] != 0.0)
    gam = nt * u / (1 - nt * u)
    for g in range(Gp):
        ii = rng.integers(0, m, ns)
        jj = rng.integers(0, n, ns)
        a = A[g][:, torch.from_numpy(ii).to(dev)].cpu().numpy().T.astype(np.longdouble)   # ns x k
        b = B[g][torch.from_numpy(jj).to(dev), :].cpu().numpy().astype(np.longdouble)     # ns x k
        ref = W["alpha"] * (a * b).sum(axis=1)
        den = abs(W["alpha"]) * np.abs(a * b).sum(axis=1)
        if C0 is not None:
            c0 = C0[g][torch.from_numpy(jj).to(dev), torch.from_numpy(ii).to(dev)].cpu().numpy().astype(np.longdouble)
            ref = ref + W["beta"] * c0
            den = den + abs(W["beta"]) * np.abs(c0)
        got = Cm[g][torch.from_numpy(jj).to(dev), torch.from_numpy(ii).to(dev)].cpu().numpy().astype(np.longdouble)
        err = np.abs(got - ref)
        worst_gamma = max(worst_gamma, float(np.max(err / (gam * den))))
        nrm = np.sqrt((a * a).sum(axis=1) * (b * b).sum(axis=1))
        worst_norm = max(worst_norm, float(np.max(err / (abs(W["alpha"]) * nrm))))

    # ---- native FP64 MFMA path on the same workload (context: the emulation must beat this)
    native_tflops = None
    if not args.no_native:
        cfgn = G.Config(0, 1e-15, 1, 0)
        for _ in range(2):
            G.lib().ggemm_grouped_dgemm(hv.h, G.PATH_NATIVE_GROUPED, C.byref(cfgn), probs, Gp, None)
        torch.cuda.synchronize()
        reps = max(2, min(args.steps, 10))
        e0.record()
        for _ in range(reps):
            G.lib().ggemm_grouped_dgemm(hv.h, G.PATH_NATIVE_GROUPED, C.byref(cfgn), probs, Gp, None)
        e1.record()
        torch.cuda.synchronize()
        native_tflops = flops / (e0.elapsed_time(e1) / reps * 1e-3) / 1e12
    hv.close()

    # ---- CPU baseline: the host FP64 GEMM (OpenMP) on a bounded sample of the same problems
    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, str(REPO / "tests"))
        import oracle_lib as O
        ora = O.oracle()
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        done, t_cpu, budget = 0, 0.0, 15.0
        for g in range(Gp):
            ha = A[g].cpu().numpy().reshape(-1)
            hb = B[g].cpu().numpy().reshape(-1)
            hc = np.zeros(m * n)
            t1 = time.perf_counter()
            ora.oz2o_dgemm(m, n, k, W["alpha"], ha, lda, hb, ldb, 0.0, hc, ldc)
            t_cpu += time.perf_counter() - t1
            done += 1
            if t_cpu > budget or (args.workload == "large"):
                break
        cpu = {"value": round(2.0 * m * n * k * done / t_cpu / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
               "kind": "port",
               "sample": f"{done} of {Gp} problems ({m}x{n}x{k}) through the host blocked FP64 GEMM "
                         f"(oracle/oz2_dgemm.c, OpenMP, {threads} threads), {t_cpu:.1f} s"}

    value = flops / (ms * 1e-3) / 1e12
    out = {
        "metric": "effective FP64 TFLOP/s (2*sum mnk/t), % INT8 MFMA peak, max certified rel err",
        "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "wall_ms_per_step": round(wall_ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f64", "data": "synthetic",
        "config": {"workload": W["desc"], "G": Gp, "m": m, "n": n, "k": k, "path": "EMU_GROUPED",
                   "execution": "plan/execute (hipGraph), pointers updated per run" if plan is not None
                   else "ggemm_grouped_dgemm per run",
                   "num_moduli": N, "planes": planes, "repair": "ON"},
        "int8_mfma_frac_end_to_end": round(int8_ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
        "fp64_mfma_frac": round(value / FP64_PEAK_TFLOPS, 4),
        "native_fp64_tflops": None if native_tflops is None else round(native_tflops, 3),
        "max_err_over_gamma_sampled": worst_gamma, "max_normwise_rel_err_sampled": worst_norm,
        "stats": {"num_fallback": stv.num_fallback, "num_repaired": stv.num_repaired,
                  "num_uncertified": stv.num_uncertified, "num_safety_fallback": stv.num_safety_fallback,
                  "kernel_launches": stv.kernel_launches, "moduli": [stv.moduli_min, stv.moduli_max]},
        "stage_ms": {"prep": round(st_ms[0], 4), "int8_gemm": round(st_ms[1], 4), "reconstruct": round(st_ms[2], 4),
                     "native": round(st_ms[3], 4)},
        "stage_hbm_gbs": {"prep": round(prep_bytes / (st_ms[0] * 1e-3) / 1e9, 1) if st_ms[0] else None,
                          "reconstruct": round(recon_bytes / (st_ms[2] * 1e-3) / 1e9, 1) if st_ms[2] else None},
        "roofline": {"bound": "mfma", "kernel": i8_kernel, "achieved": round(achieved, 2),
                     "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s", "frac": round(achieved / INT8_PEAK_TOPS, 4),
                     "traffic": measured_traffic(args.workload, i8_kernel)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
