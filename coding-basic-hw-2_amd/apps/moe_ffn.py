"""FP64 mixture-of-experts feed-forward layer on the grouped Ozaki-II DGEMM: an application
benchmark of the C ABI (the reference's counterpart: bench/app/moe_ffn_fp64.cu).

Layer, column-major throughout (T tokens, model width d, hidden width f, E experts, k per token):
  route    expert popularity p_e ~ (e + 1)^-s; every token takes k distinct experts by one
           Gumbel-top-k draw over log p_e, with gate weights = uniform draws normalised per token.
           The routing is fixed for the run (computed once on the host), like the descriptors.
  dispatch the (token, slot) pairs sorted by expert (stable in token order) form the rows of
           Xd (M x d, M = T k); expert e owns rows off_e .. off_e + m_e - 1; gathered on the GPU
  up       one grouped GEMM, a problem per expert:   H_e  = Xd_e W1_e   (m_e x f, inner d)
  act      tanh, or the tanh form of GELU, elementwise on the GPU
  down     one grouped GEMM:                         Yd_e = Ha_e W2_e   (m_e x d, inner f)
  combine  Y[t] = sum over slots j (in order) of g[t, j] Yd[pos(t, j)]  (deterministic)
Experts that receive no token stay in the group as m = 0 problems (the library skips them).

Timing: device events around dispatch, up, act, down and combine over --reps runs after --warmup.
Error (per path): for --samples tokens the layer is recomputed on the host in 80-bit arithmetic
from the same inputs.  err_up = max |H - H*| / (gamma_d |x| |W1|) over those tokens' rows of H;
err_y = max |Y - Y*| / (gamma_n den), den = sum_j |g_j| (|act(h_j)| |W2_j| + L (|x| |W1_j|) |W2_j|),
the first-order componentwise sensitivity of the layer to both GEMMs (L = sup |act'|), with
n = max(d, f) + k + 4 covering the combine sum and a few ulps of the activation.  Both are <= 1
for an FP64-accurate layer; they are diagnostics, not proofs.

Usage: python3 moe_ffn.py [--tokens 4096] [--experts 16] [--topk 2] [--d-model 1024] [--d-ff 2048]
                          [--zipf 1.0] [--phi 0.5] [--act tanh|gelu] [--seed 7] [--moduli 0]
                          [--paths all|name,...] [--reps 10] [--warmup 3] [--samples 32]
                          [--csv FILE] [--append]
Prints one JSON line per path.
"""
import argparse
import json
import math
import sys

import numpy as np

import app_util as AU

GELU_C = math.sqrt(2.0 / math.pi)
STAGES = ("dispatch", "up", "act", "down", "combine")


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--tokens", type=int, default=4096)
    ap.add_argument("--experts", type=int, default=16)
    ap.add_argument("--topk", type=int, default=2)
    ap.add_argument("--d-model", type=int, default=1024)
    ap.add_argument("--d-ff", type=int, default=2048)
    ap.add_argument("--zipf", type=float, default=1.0)
    ap.add_argument("--phi", type=float, default=0.5)
    ap.add_argument("--act", choices=("tanh", "gelu"), default="tanh")
    ap.add_argument("--seed", type=int, default=7)
    ap.add_argument("--moduli", type=int, default=0)
    ap.add_argument("--paths", default="all")
    ap.add_argument("--reps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--samples", type=int, default=32)
    ap.add_argument("--csv", default=None)
    ap.add_argument("--append", action="store_true")
    a = ap.parse_args(argv)
    if a.tokens < 1 or a.experts < 1 or a.d_model < 1 or a.d_ff < 1:
        ap.error("--tokens, --experts, --d-model and --d-ff must be positive")
    if not 1 <= a.topk <= a.experts:
        ap.error("--topk must lie in [1, --experts]")
    if a.reps < 1 or a.warmup < 0 or a.samples < 0:
        ap.error("--reps must be positive, --warmup and --samples non-negative")
    try:
        a.path_list = AU.parse_paths(a.paths)
    except ValueError as e:
        ap.error(str(e))
    return a


def route(tokens, experts, topk, zipf, rng):
    """(experts per token (T, k) in descending key order, gates (T, k) summing to 1 per token)."""
    logp = -zipf * np.log(np.arange(1, experts + 1, dtype=np.float64))
    keys = logp[None, :] - np.log(-np.log(rng.random((tokens, experts))))   # Gumbel perturbation
    top = np.argpartition(-keys, topk - 1, axis=1)[:, :topk]
    order = np.argsort(-np.take_along_axis(keys, top, axis=1), axis=1)
    ex = np.take_along_axis(top, order, axis=1)
    g = rng.random((tokens, topk)) + 0.25
    return ex, g / g.sum(axis=1, keepdims=True)


def dispatch_plan(ex, experts):
    """Pairs (token, slot) sorted by expert: token index per row, row of each pair (T, k), and the
    per-expert row counts and offsets."""
    T, k = ex.shape
    flat = ex.reshape(-1)
    order = np.argsort(flat, kind="stable")          # rows in expert order, tokens ascending
    counts = np.bincount(flat, minlength=experts)
    offs = np.concatenate([[0], np.cumsum(counts)[:-1]])
    pos = np.empty(T * k, dtype=np.int64)
    pos[order] = np.arange(T * k)
    return order // k, pos.reshape(T, k), counts, offs


class Layer:
    """Inputs, routing, device buffers and the two groups of problems of one MoE layer."""

    def __init__(self, a, torch):
        self.a, self.torch = a, torch
        rng = np.random.default_rng(a.seed)
        T, E, d, f, k = a.tokens, a.experts, a.d_model, a.d_ff, a.topk
        self.ex, self.g = route(T, E, k, a.zipf, rng)
        tok, self.pos, self.counts, self.offs = dispatch_plan(self.ex, E)
        self.M = T * k
        # host copies in torch layouts: X (d, T) = column-major T x d; W1[e] (f, d) = d x f; W2[e] (d, f) = f x d
        self.X_h = AU.phi_values(rng, (d, T), a.phi)
        self.W1_h = AU.phi_values(rng, (E, f, d), a.phi) / math.sqrt(d)
        self.W2_h = AU.phi_values(rng, (E, d, f), a.phi) / math.sqrt(f)
        dev = "cuda"
        self.X = torch.from_numpy(self.X_h).to(dev)
        self.W1 = torch.from_numpy(self.W1_h).to(dev)
        self.W2 = torch.from_numpy(self.W2_h).to(dev)
        self.tok = torch.from_numpy(tok).to(dev)
        self.pos_d = torch.from_numpy(np.ascontiguousarray(self.pos.T)).to(dev)   # (k, T)
        self.gate = torch.from_numpy(self.g.T.copy()).to(dev)   # (k, T)
        z = lambda *s: torch.empty(*s, dtype=torch.float64, device=dev)
        self.Xd, self.H, self.Ha, self.Yd, self.Y = z(d, self.M), z(f, self.M), z(f, self.M), z(d, self.M), z(d, T)
        w = 8
        self.up = [AU.problem(int(self.counts[e]), f, d, self.Xd.data_ptr() + w * int(self.offs[e]), self.M,
                              self.W1[e].data_ptr(), d, self.H.data_ptr() + w * int(self.offs[e]), self.M)
                   for e in range(E)]
        self.down = [AU.problem(int(self.counts[e]), d, f, self.Ha.data_ptr() + w * int(self.offs[e]), self.M,
                                self.W2[e].data_ptr(), f, self.Yd.data_ptr() + w * int(self.offs[e]), self.M)
                     for e in range(E)]
        self.up, self.down = AU.Problems(self.up), AU.Problems(self.down)
        shapes = [(int(self.counts[e]), f, d) for e in range(E)] + [(int(self.counts[e]), d, f) for e in range(E)]
        self.grouped = AU.Grouped(shapes)
        self.cfg = AU.G.Config(a.moduli, 1e-15, 1, 0)

    def act(self, x):
        t = self.torch
        if self.a.act == "tanh":
            return t.tanh(x)
        return 0.5 * x * (1.0 + t.tanh(GELU_C * (x + 0.044715 * x * x * x)))

    def forward(self, path, timer=None):
        """One layer forward on the given ABI path; returns the stats of the two grouped calls."""
        t = self.torch
        mark = (lambda i: timer.mark(i)) if timer else (lambda i: None)
        if timer:
            timer.start()
        t.index_select(self.X, 1, self.tok, out=self.Xd)
        mark(0)
        st_up = self.grouped.run(path, self.cfg, self.up)
        mark(1)
        self.Ha.copy_(self.act(self.H))
        mark(2)
        st_down = self.grouped.run(path, self.cfg, self.down)
        mark(3)
        self.Y.zero_()
        for j in range(self.a.topk):
            self.Y.add_(t.index_select(self.Yd, 1, self.pos_d[j]) * self.gate[j])
        mark(4)
        if timer:
            timer.stop()
        return st_up, st_down

    def reference(self, tokens):
        """80-bit host evaluation for the given tokens: per token its output row Y*, the sensitivity
        den and, per slot, (row of H, hidden row h, its sensitivity |x| |W1|).  Each expert's
        matrices are converted once."""
        a = self.a
        L = 1.0 if a.act == "tanh" else 1.13   # sup |act'|
        res = {int(tk): [np.zeros(a.d_model, dtype=np.longdouble), np.zeros(a.d_model, dtype=np.longdouble), []]
               for tk in tokens}
        pairs = [(int(tk), j, int(self.ex[tk, j])) for tk in tokens for j in range(a.topk)]
        for e in sorted({p[2] for p in pairs}):
            W1 = self.W1_h[e].T.astype(np.longdouble)           # d x f
            W2 = self.W2_h[e].T.astype(np.longdouble)           # f x d
            aW1, aW2 = np.abs(W1), np.abs(W2)
            for tk, j, ee in pairs:
                if ee != e:
                    continue
                x = self.X_h[:, tk].astype(np.longdouble)
                h = x @ W1
                hden = np.abs(x) @ aW1
                if a.act == "tanh":
                    ha = np.tanh(h)
                else:
                    ha = 0.5 * h * (1.0 + np.tanh(np.longdouble(GELU_C) * (h + np.longdouble(0.044715) * h ** 3)))
                gj = np.longdouble(self.g[tk, j])
                r = res[tk]
                r[0] += gj * (ha @ W2)
                r[1] += abs(gj) * (np.abs(ha) @ aW2 + L * (hden @ aW2))
                r[2].append((int(self.pos[tk, j]), h, hden))
        return [(tk, y, den, rows) for tk, (y, den, rows) in res.items()]

    def errors(self, refs):
        """(err_up, err_y) over the reference tokens, in units of their bounds."""
        a = self.a
        H = self.H.cpu().numpy()
        Y = self.Y.cpu().numpy()
        gd = AU.gamma(a.d_model)
        gn = AU.gamma(max(a.d_model, a.d_ff) + a.topk + 4)
        eu = ey = 0.0
        for tk, y, den, rows in refs:
            for p, h, hden in rows:
                dd = gd * hden
                m = dd > 0
                if m.any():
                    eu = max(eu, float(np.max(np.abs(H[:, p].astype(np.longdouble) - h)[m] / dd[m])))
            dy = gn * den
            m = dy > 0
            if m.any():
                ey = max(ey, float(np.max(np.abs(Y[:, tk].astype(np.longdouble) - y)[m] / dy[m])))
        return eu, ey

    def close(self):
        self.grouped.close()


def main(argv=None):
    a = parse_args(argv)
    import torch
    if not torch.cuda.is_available():
        sys.exit("moe_ffn: no GPU")
    lay = Layer(a, torch)
    rng = np.random.default_rng(a.seed + 1)
    sample = np.sort(rng.choice(a.tokens, min(a.samples, a.tokens), replace=False)) if a.samples else []
    refs = lay.reference(sample)
    flops = 2.0 * lay.M * a.d_model * a.d_ff * 2
    rows = []
    for path in a.path_list:
        for _ in range(a.warmup):
            lay.forward(path)
        timer = AU.StageTimer(torch, STAGES)
        for _ in range(a.reps):
            st_up, st_down = lay.forward(path, timer)
        ms = timer.mean()
        eu, ey = lay.errors(refs)
        rec = {"app": "moe_ffn", "path": path, "tokens": a.tokens, "experts": a.experts, "topk": a.topk,
               "d_model": a.d_model, "d_ff": a.d_ff, "act": a.act, "zipf": a.zipf, "phi": a.phi,
               "total_ms": round(ms["total"], 4), **{f"{s}_ms": round(ms[s], 4) for s in STAGES},
               "gemm_tflops": round(flops / ((ms["up"] + ms["down"]) * 1e-3) / 1e12, 3),
               "err_up_over_bound": eu, "err_y_over_bound": ey,
               "moduli": f"{min(st_up.moduli_min, st_down.moduli_min)}-{max(st_up.moduli_max, st_down.moduli_max)}",
               "fallback": st_up.num_fallback + st_down.num_fallback,
               "launches": st_up.kernel_launches + st_down.kernel_launches}
        print(json.dumps(rec), flush=True)
        rows.append(rec)
    AU.write_csv(a.csv, rows, a.append)
    lay.close()
    return rows


if __name__ == "__main__":
    main()
