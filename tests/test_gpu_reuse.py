"""GGEMM_PATH_EMU_GROUPED_REUSE end to end (tests/test_reuse_e2e.cu semantics, --small shapes).

Three sharing patterns: LoRA shrink (one shared B, distinct A), tensor parallel (one shared A,
distinct B) and a no-sharing control.  Gates: REUSE output bit-identical to EMU_GROUPED (same N
under EXACT_N, so identical numerics) and to the oracle; EMU_LOOP_BATCHED bit-identical too;
unique-operand counts, reuse flag and launch count in the stats; AUTO never reuses.  A handle
created with GGEMM_REUSE_PROMOTE=1 gives the same bits (N depends only on k here, so nothing is
promoted)."""
import os

import numpy as np
import pytest
import torch

os.environ["GGEMM_STATS_REPAIR"] = "1"

import ggemm as G
import oracle_lib as O
from gpu_util import dev, host, same_bits, say

pytestmark = pytest.mark.gpu

CFG_EMU = G.Config(0, 1e-15, 0, 0)
CFG_AUTO = G.Config(0, 1e-15, 1, 0)

#              name    G   m   n    k  shareA shareB uA uB
WORKLOADS = [("lora", 4, 16, 64, 256, False, True, 4, 1),
             ("tp", 4, 64, 48, 256, True, False, 1, 4),
             ("none", 4, 48, 64, 128, False, False, 4, 4)]


def mixed(rng, n):
    """Normal entries times 2^e, e uniform in [-8, 8]: exercises the per-row / column scaling."""
    return np.ldexp(rng.standard_normal(n), rng.integers(-8, 9, n))


class Workload:
    def __init__(self, name, Gp, m, n, k, share_a, share_b, ua, ub, seed):
        rng = np.random.default_rng(seed)
        self.name, self.G, self.m, self.n, self.k = name, Gp, m, n, k
        self.expect = (ua, ub)
        nA = 1 if share_a else Gp
        nB = 1 if share_b else Gp
        self.hA = [mixed(rng, m * k) for _ in range(nA)]
        self.hB = [mixed(rng, k * n) for _ in range(nB)]
        self.hC0 = [mixed(rng, m * n) for _ in range(Gp)]
        self.dA = [dev(a) for a in self.hA]
        self.dB = [dev(b) for b in self.hB]
        self.dC = [dev(c) for c in self.hC0]
        self.ia = [0 if share_a else g for g in range(Gp)]
        self.ib = [0 if share_b else g for g in range(Gp)]
        self.alpha = [1.0 + 0.25 * (g % 3) for g in range(Gp)]
        self.beta = [0.5 if g % 2 else 0.0 for g in range(Gp)]

    def problems(self):
        return [G.Problem(self.m, self.n, self.k, self.dA[self.ia[g]].data_ptr(), self.m,
                          self.dB[self.ib[g]].data_ptr(), self.k, self.dC[g].data_ptr(), self.m,
                          self.alpha[g], self.beta[g]) for g in range(self.G)]

    def run(self, handle, path, cfg):
        for d, c in zip(self.dC, self.hC0):
            d.copy_(torch.from_numpy(c))
        torch.cuda.synchronize()
        rc, st = handle.dgemm(path, cfg, self.problems())
        torch.cuda.synchronize()
        return rc, st, [host(d) for d in self.dC]

    def oracle(self, g, N):
        h = O.HostProb(self.m, self.n, self.k, 0, 0.0, self.alpha[g], self.beta[g])
        h.lda, h.ldb, h.ldc = self.m, self.k, self.m
        h.A, h.B, h.C0 = self.hA[self.ia[g]].copy(), self.hB[self.ib[g]].copy(), self.hC0[g].copy()
        return h.emulate(O.REPAIR_COUNT, N)[0]

    def sizes(self):
        return self.G * self.m * self.k, self.G * self.k * self.n, self.G * self.m * self.n


@pytest.mark.parametrize("wl", WORKLOADS, ids=[w[0] for w in WORKLOADS])
def test_reuse_matches_grouped_and_oracle(wl):
    w = Workload(*wl, seed=1234 + WORKLOADS.index(wl))
    say(f"reuse {w.name}")
    with G.Handle(w.G, *w.sizes()) as h:
        rb, sb, cb = w.run(h, G.PATH_EMU_GROUPED, CFG_EMU)
        rr, sr, cr = w.run(h, G.PATH_EMU_GROUPED_REUSE, CFG_EMU)
        rl, sl, cl = w.run(h, G.PATH_EMU_LOOP_BATCHED, CFG_EMU)
        ra, sa, _ = w.run(h, G.PATH_AUTO, CFG_AUTO)
    assert rb == rr == rl == ra == 0, (rb, rr, rl, ra)
    for g in range(w.G):
        assert same_bits(cr[g], cb[g]), f"{w.name}: REUSE != EMU_GROUPED in problem {g}"
        assert same_bits(cl[g], cb[g]), f"{w.name}: EMU_LOOP_BATCHED != EMU_GROUPED in problem {g}"
        assert same_bits(cr[g], w.oracle(g, sr.moduli_max)), f"{w.name}: REUSE != oracle in problem {g}"
    assert (sb.reuse_enabled, sr.reuse_enabled, sa.reuse_enabled) == (0, 1, 0)
    assert (sb.num_unique_A, sb.num_unique_B) == (w.G, w.G)
    assert (sr.num_unique_A, sr.num_unique_B) == w.expect
    assert sr.kernel_launches == sb.kernel_launches == 6
    assert sr.num_promoted == 0
    assert (sr.num_uncertified, sr.num_repaired, sr.num_safety_fallback) == \
           (sb.num_uncertified, sb.num_repaired, sb.num_safety_fallback)


def test_reuse_promote_policy_same_bits():
    w = Workload(*WORKLOADS[0], seed=77)
    with G.Handle(w.G, *w.sizes()) as h:
        _, _, cb = w.run(h, G.PATH_EMU_GROUPED, CFG_EMU)
    os.environ["GGEMM_REUSE_PROMOTE"] = "1"
    try:
        h = G.Handle(w.G, *w.sizes())
    finally:
        del os.environ["GGEMM_REUSE_PROMOTE"]
    with h:
        rr, sr, cr = w.run(h, G.PATH_EMU_GROUPED_REUSE, CFG_EMU)
    assert rr == 0 and sr.reuse_enabled == 1 and sr.num_promoted == 0
    assert (sr.num_unique_A, sr.num_unique_B) == w.expect
    for g in range(w.G):
        assert same_bits(cr[g], cb[g])
