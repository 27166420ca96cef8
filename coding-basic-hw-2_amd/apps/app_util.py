"""Shared pieces of the application benchmarks: the ABI paths, grouped calls through the library,
stage timing with device events, and the CSV record.

The applications are downstream consumers of the C ABI (include/ggemm.h) through the ctypes
binding; every GEMM they run is a ggemm_grouped_dgemm call.  torch supplies device memory and the
non-GEMM elementwise / gather steps on the same (default) stream as the library's handle."""
import csv
import ctypes as C
import os
import sys
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parents[1]
if str(PKG) not in sys.path:
    sys.path.insert(0, str(PKG))

import ggemm as G   # noqa: E402

PATHS = {"native_loop": G.PATH_NATIVE_LOOP, "native_grouped": G.PATH_NATIVE_GROUPED,
         "emu_loop": G.PATH_EMU_LOOP, "emu_grouped": G.PATH_EMU_GROUPED, "auto": G.PATH_AUTO,
         "emu_grouped_reuse": G.PATH_EMU_GROUPED_REUSE, "emu_loop_batched": G.PATH_EMU_LOOP_BATCHED}
EMULATED = ("emu_loop", "emu_grouped", "emu_grouped_reuse", "emu_loop_batched")
U = 2.0 ** -53


def parse_paths(spec):
    """'all' or a comma list of PATHS keys -> list of names (ValueError on an unknown name)."""
    if spec == "all":
        return list(PATHS)
    names = [s.strip() for s in spec.split(",") if s.strip()]
    bad = [s for s in names if s not in PATHS]
    if bad or not names:
        raise ValueError(f"unknown path(s) {bad or spec!r}; choose from {', '.join(PATHS)} or all")
    return names


def gamma(n):
    return n * U / (1.0 - n * U)


def phi_values(rng, shape, phi):
    """(U(0,1) - 0.5) exp(phi N(0,1)): the Ozaki-scheme test distribution (phi = 0: uniform)."""
    v = rng.random(shape) - 0.5
    if phi:
        v *= np.exp(phi * rng.standard_normal(shape))
    return v


class Grouped:
    """One handle sized for a fixed set of problem shapes, and the calls on it."""

    def __init__(self, shapes, min_k=None):
        self.max_problems = max(1, len(shapes))
        self.sizes = (sum(m * k for m, n, k in shapes) + 1, sum(k * n for m, n, k in shapes) + 1,
                      sum(m * n for m, n, k in shapes) + 1)
        self.h = G.Handle(self.max_problems, *self.sizes, min_k=min_k)

    def run(self, path, cfg, problems):
        """One ggemm_grouped_dgemm call on a Problems set (or a list of G.Problem)."""
        ps = problems if isinstance(problems, Problems) else Problems(problems)
        st = G.Stats()
        rc = G.lib().ggemm_grouped_dgemm(self.h.h, PATHS[path], C.byref(cfg), ps.arr, ps.n, C.byref(st))
        if rc != G.GGEMM_OK:
            raise RuntimeError(f"ggemm_grouped_dgemm({path}) returned {rc}")
        return st

    def close(self):
        self.h.close()


class Problems:
    """A fixed list of problems and its ctypes array, built once (calls in loops reuse it)."""

    def __init__(self, probs):
        self.list = list(probs)
        self.n = len(self.list)
        self.arr = G.problems_array(self.list)


def problem(m, n, k, A, lda, B, ldb, C, ldc, alpha=1.0, beta=0.0):
    """A ggemm_problem_t from device addresses (integers) and leading dimensions."""
    return G.Problem(m, n, k, A, max(1, lda), B, max(1, ldb), C, max(1, ldc), alpha, beta)


class StageTimer:
    """Device-event timing of named stages over repeated runs on the current stream."""

    def __init__(self, torch, stages):
        self.torch = torch
        self.stages = list(stages)
        self.ms = {s: [] for s in self.stages + ["total"]}
        self.ev = None

    def start(self):
        t = self.torch
        self.ev = [t.cuda.Event(enable_timing=True) for _ in range(len(self.stages) + 1)]
        self.ev[0].record()

    def mark(self, i):
        """End of stage i (0-based)."""
        self.ev[i + 1].record()

    def stop(self):
        self.torch.cuda.synchronize()
        for i, s in enumerate(self.stages):
            self.ms[s].append(self.ev[i].elapsed_time(self.ev[i + 1]))
        self.ms["total"].append(self.ev[0].elapsed_time(self.ev[-1]))

    def mean(self):
        return {s: float(np.mean(v)) if v else 0.0 for s, v in self.ms.items()}


def write_csv(path, rows, append):
    """rows: list of dicts with the same keys; header written unless appending to an existing file."""
    if not path or not rows:
        return
    exists = os.path.exists(path) and os.path.getsize(path) > 0
    with open(path, "a" if append else "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0].keys()))
        if not (append and exists):
            w.writeheader()
        w.writerows(rows)
