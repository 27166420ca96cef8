"""FP64 block-sparse (BSR, variable block sizes) times dense multi-vector, Y = A X, on the grouped
Ozaki-II DGEMM: an application benchmark of the C ABI (the reference's counterpart:
bench/app/block_sparse_fp64.cu).

Instance (fixed seed): atoms uniform in a periodic cube at number density --density; each atom an
element H / C / O (probabilities 0.5 / 0.35 / 0.15) with the basis-function count of the chosen
correlation-consistent basis (cc-pVDZ 5 / 14 / 14, cc-pVTZ 14 / 30 / 30, cc-pVQZ 30 / 55 / 55); block
(I, J) is stored when the minimum-image distance of atoms I and J is at most --cutoff (the diagonal
always), with entries of the phi distribution damped by exp(-r_IJ / 2).  A block row I is stored as
one column-major panel r_I x K_I (its blocks side by side, ascending J), so block (I, J) is the
panel's column range of J.  X is N x nrhs column-major (N = total basis functions).

Formulations (--mode panel|waves|both):
  panel  one problem per block row: the rows of X of the row's block columns are gathered into a
         K_I x nrhs panel Xp_I (one device gather for all rows), then Y_I = A_I Xp_I in one grouped
         call -- the sum over the row's blocks happens inside each problem's inner dimension;
  waves  no gather and no reduction buffer: call w takes block w of every row that has one,
         Y_I = A_IJw X_Jw + beta Y_I with beta = 0 for w = 0 and 1 after, the B operand being the
         rows of X itself (ldb = N).  Calls = the longest block row; every call a grouped call.
Timing: device events per stage over --reps runs after --warmup; descriptors are built once.
Error (per path and mode): --samples rows of Y recomputed on the host in 80-bit arithmetic;
err = max |Y - Y*| / (gamma_n |A| |X|), n = max K_I + max blocks per row + 1 (the waves
formulation rounds each block product once more); <= 1 means FP64-accurate (a diagnostic).

Usage: python3 block_sparse.py [--atoms 1024] [--density 0.1] [--cutoff 6] [--basis dz|tz|qz]
                               [--nrhs 128] [--mode both] [--phi 0.5] [--seed 11] [--moduli 0]
                               [--paths all|name,...] [--reps 5] [--warmup 2] [--samples 64]
                               [--csv FILE] [--append]
Prints one JSON line per (mode, path).
"""
import argparse
import json
import sys

import numpy as np

import app_util as AU

BASIS = {"dz": (5, 14, 14), "tz": (14, 30, 30), "qz": (30, 55, 55)}   # H, C, O
ELEMENT_P = (0.5, 0.35, 0.15)


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--atoms", type=int, default=1024)
    ap.add_argument("--density", type=float, default=0.1)
    ap.add_argument("--cutoff", type=float, default=6.0)
    ap.add_argument("--basis", choices=sorted(BASIS), default="dz")
    ap.add_argument("--nrhs", type=int, default=128)
    ap.add_argument("--mode", choices=("panel", "waves", "both"), default="both")
    ap.add_argument("--phi", type=float, default=0.5)
    ap.add_argument("--seed", type=int, default=11)
    ap.add_argument("--moduli", type=int, default=0)
    ap.add_argument("--paths", default="all")
    ap.add_argument("--reps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--samples", type=int, default=64)
    ap.add_argument("--csv", default=None)
    ap.add_argument("--append", action="store_true")
    a = ap.parse_args(argv)
    if a.atoms < 1 or a.nrhs < 1 or a.density <= 0 or a.cutoff < 0:
        ap.error("--atoms and --nrhs must be positive, --density positive, --cutoff non-negative")
    if a.reps < 1 or a.warmup < 0 or a.samples < 0:
        ap.error("--reps must be positive, --warmup and --samples non-negative")
    try:
        a.path_list = AU.parse_paths(a.paths)
    except ValueError as e:
        ap.error(str(e))
    a.modes = ["panel", "waves"] if a.mode == "both" else [a.mode]
    return a


def structure(atoms, density, cutoff, basis, rng):
    """Block sizes per atom, and per block row the (ascending) neighbour columns and distances."""
    side = (atoms / density) ** (1.0 / 3.0)
    pos = rng.random((atoms, 3)) * side
    elem = rng.choice(3, size=atoms, p=ELEMENT_P)
    size = np.asarray(BASIS[basis])[elem]
    cols, dist = [], []
    for i in range(atoms):
        d = pos - pos[i]
        d -= side * np.round(d / side)                 # minimum image
        r = np.sqrt((d * d).sum(axis=1))
        j = np.nonzero(r <= cutoff)[0]                 # ascending, includes i (r = 0)
        cols.append(j)
        dist.append(r[j])
    return size, cols, dist


class Matrix:
    """The BSR matrix, X, Y and the problem lists of both formulations."""

    def __init__(self, a, torch):
        self.a, self.torch = a, torch
        rng = np.random.default_rng(a.seed)
        self.size, self.cols, self.dist = structure(a.atoms, a.density, a.cutoff, a.basis, rng)
        self.off = np.concatenate([[0], np.cumsum(self.size)[:-1]])   # first basis function per atom
        self.N = int(self.size.sum())
        nb = a.nrhs
        # row panels, column-major r_I x K_I, back to back in one buffer
        self.K = np.array([int(self.size[c].sum()) for c in self.cols])
        self.poff = np.concatenate([[0], np.cumsum(self.size * self.K)[:-1]])
        vals = np.empty(int((self.size * self.K).sum()))
        for i, (c, r) in enumerate(zip(self.cols, self.dist)):
            ri, Ki = int(self.size[i]), int(self.K[i])
            p = AU.phi_values(rng, (Ki, ri), a.phi)    # (K_I, r_I) row-major = column-major r_I x K_I
            p *= np.repeat(np.exp(-r / 2.0), self.size[c])[:, None]
            vals[self.poff[i]:self.poff[i] + ri * Ki] = p.reshape(-1)
        self.vals_h = vals
        self.X_h = AU.phi_values(rng, (nb, self.N), a.phi)             # (nrhs, N) = column-major N x nrhs
        dev = "cuda"
        self.vals = torch.from_numpy(vals).to(dev)
        self.X = torch.from_numpy(self.X_h).to(dev)
        self.Y = torch.empty(nb, self.N, dtype=torch.float64, device=dev)
        w = 8
        # panel: gathered X rows of every row's block columns, rows back to back (K_I rows each)
        gidx = np.concatenate([np.concatenate([np.arange(self.off[j], self.off[j] + self.size[j]) for j in c])
                               for c in self.cols])
        self.gidx = torch.from_numpy(gidx).to(dev)
        self.KT = int(self.K.sum())
        self.Xp = torch.empty(nb, self.KT, dtype=torch.float64, device=dev)
        koff = np.concatenate([[0], np.cumsum(self.K)[:-1]])
        self.panel = [AU.problem(int(self.size[i]), nb, int(self.K[i]), self.vals.data_ptr() + w * int(self.poff[i]),
                                 int(self.size[i]), self.Xp.data_ptr() + w * int(koff[i]), self.KT,
                                 self.Y.data_ptr() + w * int(self.off[i]), self.N)
                      for i in range(a.atoms)]
        # waves: call w holds block w of every row with more than w blocks
        self.nwaves = max(len(c) for c in self.cols)
        self.waves = []
        for wv in range(self.nwaves):
            probs = []
            for i, c in enumerate(self.cols):
                if wv >= len(c):
                    continue
                j = int(c[wv])
                ri, cj = int(self.size[i]), int(self.size[j])
                col0 = int(self.size[c[:wv]].sum())     # the block's first column inside the panel
                probs.append(AU.problem(ri, nb, cj, self.vals.data_ptr() + w * (int(self.poff[i]) + col0 * ri), ri,
                                        self.X.data_ptr() + w * int(self.off[j]), self.N,
                                        self.Y.data_ptr() + w * int(self.off[i]), self.N, 1.0, 0.0 if wv == 0 else 1.0))
            self.waves.append(AU.Problems(probs))
        self.panel = AU.Problems(self.panel)
        # one handle for both: a wave's sums of m k, k n and m n are at most the panel call's
        self.grouped = AU.Grouped([(int(self.size[i]), nb, int(self.K[i])) for i in range(a.atoms)],
                                  min_k=int(self.size.min()))
        self.cfg = AU.G.Config(a.moduli, 1e-15, 1, 0)

    def run(self, mode, path, timer=None):
        """Y = A X in one formulation; returns the stats of its grouped calls."""
        t = self.torch
        if timer:
            timer.start()
        sts = []
        if mode == "panel":
            t.index_select(self.X, 1, self.gidx, out=self.Xp)
            if timer:
                timer.mark(0)
            sts.append(self.grouped.run(path, self.cfg, self.panel))
            if timer:
                timer.mark(1)
        else:
            if timer:
                timer.mark(0)
            for probs in self.waves:
                sts.append(self.grouped.run(path, self.cfg, probs))
            if timer:
                timer.mark(1)
        if timer:
            timer.stop()
        return sts

    def reference(self, rows):
        """80-bit host Y* and |A| |X| for the given global rows: (row, y (nrhs,), den (nrhs,))."""
        atom = np.searchsorted(self.off, rows, side="right") - 1
        out = []
        for r, i in zip(rows, atom):
            ri, Ki = int(self.size[i]), int(self.K[i])
            panel = self.vals_h[self.poff[i]:self.poff[i] + ri * Ki].reshape(Ki, ri)   # (K_I, r_I)
            arow = panel[:, r - self.off[i]].astype(np.longdouble)                   # row of A_I (K_I,)
            xr = np.concatenate([np.arange(self.off[j], self.off[j] + self.size[j]) for j in self.cols[i]])
            Xk = self.X_h[:, xr].astype(np.longdouble)                              # (nrhs, K_I)
            out.append((int(r), Xk @ arow, np.abs(Xk) @ np.abs(arow)))
        return out

    def error(self, refs):
        Y = self.Y.cpu().numpy()
        n = int(self.K.max()) + self.nwaves + 1
        g = AU.gamma(n)
        e = 0.0
        for r, y, den in refs:
            d = g * den
            m = d > 0
            if m.any():
                e = max(e, float(np.max(np.abs(Y[:, r].astype(np.longdouble) - y)[m] / d[m])))
        return e

    def close(self):
        self.grouped.close()


def main(argv=None):
    a = parse_args(argv)
    import torch
    if not torch.cuda.is_available():
        sys.exit("block_sparse: no GPU")
    mat = Matrix(a, torch)
    rng = np.random.default_rng(a.seed + 1)
    rows = np.sort(rng.choice(mat.N, min(a.samples, mat.N), replace=False)) if a.samples else []
    refs = mat.reference(rows)
    nblocks = sum(len(c) for c in mat.cols)
    flops = 2.0 * a.nrhs * float(sum(int(mat.size[i]) * int(mat.K[i]) for i in range(a.atoms)))
    out = []
    for mode in a.modes:
        for path in a.path_list:
            stages = ("gather", "gemm")   # the waves formulation gathers nothing: its gather stage is empty
            for _ in range(a.warmup):
                mat.run(mode, path)
            timer = AU.StageTimer(torch, stages)
            for _ in range(a.reps):
                sts = mat.run(mode, path, timer)
            ms = timer.mean()
            rec = {"app": "block_sparse", "mode": mode, "path": path, "atoms": a.atoms, "basis": a.basis,
                   "cutoff": a.cutoff, "nrhs": a.nrhs, "N": mat.N, "blocks": nblocks, "calls": len(sts),
                   "problems": sum(s.num_problems for s in sts), "total_ms": round(ms["total"], 4),
                   **{f"{s}_ms": round(ms[s], 4) for s in stages},
                   "gemm_tflops": round(flops / (ms["gemm"] * 1e-3) / 1e12, 3),
                   "err_over_bound": mat.error(refs),
                   "fallback": sum(s.num_fallback for s in sts), "launches": sum(s.kernel_launches for s in sts)}
            print(json.dumps(rec), flush=True)
            out.append(rec)
    AU.write_csv(a.csv, out, a.append)
    mat.close()
    return out


if __name__ == "__main__":
    main()
