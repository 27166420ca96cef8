"""Times the ROCm vendor INT8 GEMM (hipBLASLt, through torch._int_mm) at given shapes.

A point of comparison for the library's INT8 grouped GEMM: the same product shapes with both
operands K-contiguous (A m x k row-major, B stored n x k), int32 output.  Prints one JSON line per
shape with the average time of back-to-back calls (HIP events) and the INT8 rate: at least `reps`
calls and at least `min_seconds` of them, so that the GPU runs at its sustained clock (as during a
long library call) rather than in a short burst.

Usage: python3 vendor_int8_gemm.py [--shape M,N,K ...] [--reps R] [--min-seconds S]
"""
import argparse
import json

import torch


def time_int_mm(m, n, k, reps, min_seconds):
    g = torch.Generator(device="cuda").manual_seed(1)
    a = torch.randint(-128, 128, (m, k), dtype=torch.int8, device="cuda", generator=g)
    b = torch.randint(-128, 128, (n, k), dtype=torch.int8, device="cuda", generator=g).t()   # k x n, K-contiguous
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(count):
        e0.record()
        for _ in range(count):
            torch._int_mm(a, b)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / count

    timed(3)         # warm-up (the first calls include the library's setup)
    est = timed(3)   # first estimate (ms per call)
    count = max(reps, int(min_seconds * 1e3 / max(est, 1e-3)) + 1)
    if min_seconds > 0:
        timed(count)   # bring the clock to its sustained level first
    return timed(count), count


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--shape", action="append", default=None, help="M,N,K (repeatable)")
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--min-seconds", type=float, default=0.0)
    args = ap.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit("vendor_int8_gemm: no GPU visible")
    shapes = args.shape or ["1024,1024,1024", "8192,8192,1024", "16384,16384,1024", "8192,8192,16384"]
    for s in shapes:
        m, n, k = (int(x) for x in s.split(","))
        ms, count = time_int_mm(m, n, k, args.reps, args.min_seconds)
        print(json.dumps({"op": "torch._int_mm", "device": torch.cuda.get_device_name(0), "m": m, "n": n, "k": k,
                          "calls": count, "ms": round(ms, 4), "top_s": round(2.0 * m * n * k / ms / 1e9, 1)}),
              flush=True)


if __name__ == "__main__":
    main()
