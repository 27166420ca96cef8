"""Host-side logic of the application benchmarks (coding-basic-hw-2_amd/apps): MoE routing and
dispatch, the block-sparse structure, argument checking (CPU only)."""
import sys
from pathlib import Path

import numpy as np
import pytest

APPS = Path(__file__).resolve().parents[1] / "coding-basic-hw-2_amd" / "apps"
sys.path.insert(0, str(APPS))

import app_util as AU      # noqa: E402
import block_sparse as BS  # noqa: E402
import moe_ffn as MOE      # noqa: E402


@pytest.mark.parametrize("topk", [1, 2, 4])
def test_moe_routing_and_dispatch(topk):
    rng = np.random.default_rng(topk)
    T, E = 300, 7
    ex, g = MOE.route(T, E, topk, 1.2, rng)
    assert ex.shape == (T, topk) and g.shape == (T, topk)
    assert all(len(set(r)) == topk for r in ex)                 # distinct experts per token
    assert np.allclose(g.sum(axis=1), 1.0) and (g > 0).all()
    tok, pos, counts, offs = MOE.dispatch_plan(ex, E)
    assert counts.sum() == T * topk and (offs == np.concatenate([[0], np.cumsum(counts)[:-1]])).all()
    # row pos[t, j] holds token t and lies in the block of expert ex[t, j]
    assert (tok[pos] == np.arange(T)[:, None]).all()
    e_of_row = np.repeat(np.arange(E), counts)
    assert (e_of_row[pos] == ex).all()
    # inside an expert's block, tokens ascend
    for e in range(E):
        blk = tok[offs[e]:offs[e] + counts[e]]
        assert (np.diff(blk) > 0).all()


def test_moe_zipf_skew():
    """Popularity falls with the expert index (Zipf): the first expert is picked most often."""
    ex, _ = MOE.route(20000, 8, 1, 1.0, np.random.default_rng(0))
    c = np.bincount(ex.reshape(-1), minlength=8)
    assert c[0] == c.max() and c[0] > 2 * c[-1]


def test_block_sparse_structure():
    rng = np.random.default_rng(5)
    size, cols, dist = BS.structure(80, 0.1, 4.0, "tz", rng)
    assert set(size.tolist()) <= {14, 30}
    S = [set(c.tolist()) for c in cols]
    for i in range(80):
        assert i in S[i]                                         # diagonal block
        assert (np.diff(cols[i]) > 0).all()                      # ascending block columns
        assert (dist[i] <= 4.0).all() and dist[i][list(cols[i]).index(i)] == 0.0
        for j in S[i]:
            assert i in S[j]                                     # symmetric pattern (minimum image)


@pytest.mark.parametrize("mod,argv", [(MOE, ["--topk", "0"]), (MOE, ["--topk", "9", "--experts", "8"]),
                                      (MOE, ["--paths", "emu_groupd"]), (MOE, ["--reps", "0"]),
                                      (BS, ["--nrhs", "0"]), (BS, ["--paths", "x"]), (BS, ["--density", "0"])])
def test_argument_errors(mod, argv):
    with pytest.raises(SystemExit):
        mod.parse_args(argv)


def test_paths_and_csv(tmp_path):
    assert AU.parse_paths("all") == list(AU.PATHS)
    assert AU.parse_paths("auto, emu_grouped") == ["auto", "emu_grouped"]
    f = tmp_path / "r.csv"
    AU.write_csv(str(f), [{"a": 1, "b": 2}], append=False)
    AU.write_csv(str(f), [{"a": 3, "b": 4}], append=True)
    assert f.read_text().splitlines() == ["a,b", "1,2", "3,4"]
