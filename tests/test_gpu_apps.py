"""The application benchmarks on the GPU (coding-basic-hw-2_amd/apps), every ABI path.

Each path's layer / product must be FP64-accurate against the apps' 80-bit host reference on
sampled rows (err / bound <= 1).  On the emulated paths the GEMMs inside the apps are compared bit
for bit with the oracle: sampled 8 x 8 blocks of the up and down projections of several experts
(MoE) and of several block-row panels (block sparse), each problem's inputs taken from the app's own
device buffers (the oracle needs only the sampled rows of A and columns of B)."""
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import ggemm as G
import oracle_lib as O
from gpu_util import gpu_block, oracle_block, same_bits, say

APPS = Path(__file__).resolve().parents[1] / "coding-basic-hw-2_amd" / "apps"
sys.path.insert(0, str(APPS))
import app_util as AU      # noqa: E402
import block_sparse as BS  # noqa: E402
import moe_ffn as MOE      # noqa: E402

pytestmark = pytest.mark.gpu


def _sample(rng, n, cnt):
    return np.sort(rng.choice(n, min(cnt, n), replace=False))


def test_moe_every_path():
    a = MOE.parse_args(["--tokens", "200", "--experts", "5", "--topk", "2", "--d-model", "72", "--d-ff", "120",
                        "--phi", "1.0", "--act", "gelu", "--seed", "3"])
    lay = MOE.Layer(a, torch)
    lay.cfg = G.Config(0, 1e-15, 1, G.REPAIR_ON)
    refs = lay.reference(np.arange(0, a.tokens, 9))
    rng = np.random.default_rng(1)
    try:
        for path in AU.PATHS:
            say(f"moe path={path}")
            st_up, st_down = lay.forward(path)
            eu, ey = lay.errors(refs)
            assert eu <= 1.0 and ey <= 1.0, (path, eu, ey)
            if path not in AU.EMULATED:
                continue
            for st, probs, (At, Bt, Ct), k in ((st_up, lay.up.list, (lay.Xd, lay.W1, lay.H), a.d_model),
                                               (st_down, lay.down.list, (lay.Ha, lay.W2, lay.Yd), a.d_ff)):
                assert st.moduli_min == st.moduli_max > 0
                N = st.moduli_max
                for e in np.argsort(-lay.counts)[:3]:          # the three busiest experts
                    m, o = int(lay.counts[e]), int(lay.offs[e])
                    pr = probs[e]
                    I, J = _sample(rng, m, 8), _sample(rng, pr.n, 8)
                    want, _ = oracle_block(At[:, o:o + m], Bt[e], None, k, 1.0, 0.0, N, O.REPAIR_ON, I, J)
                    assert same_bits(gpu_block(Ct[:, o:o + m], I, J), want), (path, int(e))
    finally:
        lay.close()


def test_block_sparse_every_path_and_mode():
    a = BS.parse_args(["--atoms", "48", "--density", "0.1", "--cutoff", "4.5", "--basis", "dz", "--nrhs", "24",
                       "--phi", "1.0", "--seed", "5"])
    mat = BS.Matrix(a, torch)
    mat.cfg = G.Config(0, 1e-15, 1, G.REPAIR_ON)
    refs = mat.reference(np.arange(0, mat.N, 7))
    rng = np.random.default_rng(2)
    koff = np.concatenate([[0], np.cumsum(mat.K)[:-1]])
    try:
        for mode in ("panel", "waves"):
            for path in AU.PATHS:
                say(f"block_sparse mode={mode} path={path}")
                sts = mat.run(mode, path)
                err = mat.error(refs)
                assert err <= 1.0, (mode, path, err)
                if mode != "panel" or path not in AU.EMULATED:
                    continue
                st = sts[0]
                for i in rng.choice(a.atoms, 4, replace=False):
                    r, K = int(mat.size[i]), int(mat.K[i])
                    A_t = mat.vals[int(mat.poff[i]):int(mat.poff[i]) + r * K].view(K, r)
                    B_t = mat.Xp[:, int(koff[i]):int(koff[i]) + K]
                    C_t = mat.Y[:, int(mat.off[i]):int(mat.off[i]) + r]
                    N = O.oracle().oz2o_choose_num_moduli(K, 1e-15)
                    assert st.moduli_min <= N <= st.moduli_max
                    I, J = np.arange(r), _sample(rng, a.nrhs, 8)
                    want, _ = oracle_block(A_t, B_t, None, K, 1.0, 0.0, N, O.REPAIR_ON, I, J)
                    assert same_bits(gpu_block(C_t, I, J), want), (path, int(i))
    finally:
        mat.close()


def test_apps_command_line(tmp_path):
    """Both programs end to end through their command lines: one record per path (and mode),
    printed and written to the CSV file."""
    f1, f2 = tmp_path / "moe.csv", tmp_path / "bsr.csv"
    rows = MOE.main(["--tokens", "64", "--experts", "4", "--d-model", "40", "--d-ff", "56", "--paths",
                     "emu_grouped,auto", "--reps", "1", "--warmup", "0", "--samples", "4", "--csv", str(f1)])
    assert [r["path"] for r in rows] == ["emu_grouped", "auto"]
    assert all(r["err_y_over_bound"] <= 1.0 and r["launches"] > 0 for r in rows)
    rows = BS.main(["--atoms", "24", "--cutoff", "4", "--nrhs", "8", "--paths", "native_grouped,emu_grouped",
                    "--reps", "1", "--warmup", "0", "--samples", "8", "--csv", str(f2)])
    assert [(r["mode"], r["path"]) for r in rows] == [("panel", "native_grouped"), ("panel", "emu_grouped"),
                                                    ("waves", "native_grouped"), ("waves", "emu_grouped")]
    assert all(r["err_over_bound"] <= 1.0 for r in rows)
    assert len(f1.read_text().splitlines()) == 3 and len(f2.read_text().splitlines()) == 5
