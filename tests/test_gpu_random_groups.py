"""Random ragged groups through the production paths, bitwise against the oracle (GPU).

A fixed-seed sweep over what the hand-written tests pin one case at a time: groups of 1-4 problems
with m, n in [1, 260] (every tile configuration, ragged 256 x 256 tiles) and k in [32, 1100] (both
sides of the one-read limit of the B prep at k = 1024, kp = 0 and 32 mod 64), adaptive N or a fixed
N on both sides of the digit-width switch (8 .. 20), EMU_GROUPED and EMU_LOOP, the default,
general or large-tile INT8 kernel, four input spreads, beta 0 or 0.5, and B columns scaled by
2^650 or 2^-700 (the prep's rescale path).  Each emulated problem must equal the oracle bit for
bit with equal counters (the checks of test_gpu_grouped.check_case)."""
import numpy as np
import pytest

import ggemm as G
import oracle_lib as O
from gpu_util import say
from test_gpu_grouped import Case, check_case, kernel_handle, run

pytestmark = pytest.mark.gpu

CASES = 150


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
