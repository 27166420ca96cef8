"""Random ragged groups through the production paths, bitwise against the oracle (GPU).

A fixed-seed sweep over what the hand-written tests pin one case at a time: groups of 1-4 problems
with m, n in [1, 260] (every tile configuration, ragged 256 x 256 tiles) and k in [32, 1100] (both
sides of the one-read limit of the B prep at k = 1024, kp = 0 and 32 mod 64), adaptive N or a fixed
N on both sides of the digit-width switch (8 .. 20), EMU_GROUPED and EMU_LOOP, the default,
general or large-tile INT8 kernel, four input spreads, beta 0 or 0.5, and B columns scaled by
2^650 or 2^-700 (the prep's rescale path).  Each emulated problem must equal the oracle bit for
bit with equal counters (the checks of test_gpu_grouped.check_case); a second sweep runs repair ON
with NaN / Inf entries, so the FP64 dot products are compared too."""
import numpy as np
import pytest

import ggemm as G
import oracle_lib as O
from gpu_util import say
from test_gpu_grouped import Case, check_case, kernel_handle, run

pytestmark = pytest.mark.gpu

CASES = 150
CASES_REPAIR = 60


def _draw(rng):
    shapes = [(int(rng.integers(1, 261)), int(rng.integers(1, 261)), int(rng.integers(32, 1101)))
              for _ in range(int(rng.integers(1, 5)))]
    return dict(shapes=shapes, N=int(rng.choice([0, 8, 12, 15, 16, 17, 20])),
                path=[G.PATH_EMU_GROUPED, G.PATH_EMU_LOOP][int(rng.integers(0, 2))],
                kernel=[None, "general", "large"][int(rng.integers(0, 3))],
                phi=float(rng.choice([0.0, 0.5, 1.0, 2.0])), beta=float(rng.choice([0.0, 0.5])),
                seed=int(rng.integers(0, 1 << 30)), scale=int(rng.choice([0, 0, 650, -700])),
                pick=(int(rng.integers(0, 1 << 30)), int(rng.integers(0, 1 << 30))))


def test_random_groups_bitwise():
    rng = np.random.default_rng(20261230)
    for i in range(CASES):
        d = _draw(rng)
        say(f"random group {i}: {d}")
        case = Case(d["shapes"], d["seed"], phi=d["phi"], beta=d["beta"])
        if d["scale"]:
            h = case.hp[d["pick"][0] % len(case.hp)]
            c = d["pick"][1] % h.n
            col = slice(c * h.ldb, c * h.ldb + h.k)
            h.B[col] = np.ldexp(h.B[col], d["scale"])
            case.alloc()
        cfg = G.Config(d["N"], 1e-15, 0, 0)
        if d["kernel"]:
            with kernel_handle(case, d["kernel"]) as hd:
                rc, st = run(case, d["path"], cfg, handle=hd)
        else:
            rc, st = run(case, d["path"], cfg)
        assert rc == 0, (i, rc)
        check_case(case, d["path"], cfg, st, O.REPAIR_COUNT)


def test_random_groups_repair_on_bitwise():
    """The same generator with repair ON, wider spreads (phi 1-3) and NaN / Inf entries in half of
    the groups: the entries that fail the certificate (repair) or meet a non-finite row or column
    (safety) take the FP64 dot products -- per lane, per wave block or per workgroup tile -- and
    must equal the oracle's sequential fma chains bit for bit, with equal counters."""
    rng = np.random.default_rng(20261231)
    for i in range(CASES_REPAIR):
        d = _draw(rng)
        d["phi"] = float(rng.choice([1.0, 2.0, 3.0]))
        say(f"random group (repair ON) {i}: {d}")
        case = Case(d["shapes"], d["seed"], phi=d["phi"], beta=d["beta"])
        if rng.random() < 0.5:
            for h in case.hp:
                for _ in range(int(rng.integers(1, 4))):
                    bad = float(rng.choice([np.nan, np.inf, -np.inf]))
                    if rng.random() < 0.5:
                        h.A[int(rng.integers(0, h.m)) + int(rng.integers(0, h.k)) * h.lda] = bad
                    else:
                        h.B[int(rng.integers(0, h.k)) + int(rng.integers(0, h.n)) * h.ldb] = bad
            case.alloc()
        cfg = G.Config(d["N"], 1e-15, 0, G.REPAIR_ON)
        if d["kernel"]:
            with kernel_handle(case, d["kernel"]) as hd:
                rc, st = run(case, d["path"], cfg, handle=hd)
        else:
            rc, st = run(case, d["path"], cfg)
        assert rc == 0, (i, rc)
        check_case(case, d["path"], cfg, st, O.REPAIR_ON)
