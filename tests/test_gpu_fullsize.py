"""The reference's ragged group (G=128: m, n log-uniform in [64, 4096], k log-uniform in [16, 8192],
(U-0.5)exp(Z), alpha ~ U(-2, 2) with 8 problems alpha = 0, beta ~ U(-1, 1), adaptive N at 1e-15,
create_ex(min_k = 16)) at its full size, checked through properties that do not need the oracle's
full emulation (minutes per problem at these sizes; the same shapes at reduced size are checked
bit for bit against the oracle in test_gpu_grouped.py):
  * routes: num_fallback and the moduli range equal the oracle planner's plan for the same shapes;
  * 64 sampled entries per problem against an 80-bit host dot product: every entry within
    gamma_n (|alpha| |A||B| + |beta C0|), the bound the componentwise certificate (or the
    FP64 repair / native route) guarantees; alpha = 0 problems equal beta C0 exactly;
  * repair ON leaves no entry uncertified, and a second call reproduces every bit.
Data are generated on the GPU (torch generator, fixed seeds); shapes from numpy (fixed seed)."""
import ctypes as C

import numpy as np
import pytest
import torch

import ggemm as G
import oracle_lib as O
from gpu_util import say

pytestmark = pytest.mark.gpu


def ragged_shapes(seed=20261203, count=128, nalpha0=8):
    rng = np.random.default_rng(seed)
    lu = lambda lo, hi: int(np.exp(rng.uniform(np.log(lo), np.log(hi))))
    shapes = []
    zero = set(rng.choice(count, nalpha0, replace=False).tolist())
    for g in range(count):
        m, n, k = lu(64, 4096), lu(64, 4096), lu(16, 8192)
        a = 0.0 if g in zero else float(rng.uniform(-2, 2))
        shapes.append((m, n, k, a, float(rng.uniform(-1, 1))))
    return shapes


def gen(shape, gen_, phi):
    u = torch.rand(shape, dtype=torch.float64, device="cuda", generator=gen_) - 0.5
    if phi:
        u *= torch.exp(phi * torch.randn(shape, dtype=torch.float64, device="cuda", generator=gen_))
    return u


def oracle_plan(shapes, cfg, path):
    props = torch.cuda.get_device_properties(0)
    dm = G.DeviceModel()
    G.lib().ggemm_device_model_init(C.byref(dm), props.gcnArchName.encode(), 9, 5, props.multi_processor_count)
    arr = (O.Shape * len(shapes))(*[O.Shape(m, n, k, a, b) for (m, n, k, a, b) in shapes])
    odm = O.DeviceModel(dm.num_sms, dm.fp64_flops, dm.int8_ops, dm.mem_bw, dm.tiny_mnk)
    out = (O.PlanEntry * len(shapes))()
    rc = O.oracle().oz2o_plan(arr, len(shapes), cfg.num_moduli, cfg.target_rel_err, cfg.allow_fallback, path,
                              C.byref(odm), 16.0, out)
    assert rc == 0
    return list(out)


@pytest.mark.parametrize("path", [G.PATH_AUTO, G.PATH_EMU_GROUPED])
def test_ragged_group_full_size(path):
    shapes = ragged_shapes()
    g_ = torch.Generator(device="cuda")
    g_.manual_seed(3)
    A = [gen((k, m), g_, 1.0) for (m, n, k, a, b) in shapes]    # column-major m x k, lda = m
    B = [gen((n, k), g_, 1.0) for (m, n, k, a, b) in shapes]    # column-major k x n, ldb = k
    C0 = [gen((n, m), g_, 0.0) for (m, n, k, a, b) in shapes]   # column-major m x n, ldc = m
    Cw = [c.clone() for c in C0]
    probs = G.problems_array([G.Problem(m, n, k, A[g].data_ptr(), m, B[g].data_ptr(), k, Cw[g].data_ptr(), m, a, b)
                              for g, (m, n, k, a, b) in enumerate(shapes)])
    tot = [sum(s[0] * s[2] for s in shapes), sum(s[2] * s[1] for s in shapes), sum(s[0] * s[1] for s in shapes)]
    cfg = G.Config(0, 1e-15, 1, G.REPAIR_ON)
    say(f"ragged G=128 full size path={path}: {tot[0] / 1e6:.0f}M + {tot[1] / 1e6:.0f}M + {tot[2] / 1e6:.0f}M elements")
    with G.Handle(len(shapes), *tot, min_k=16) as h:
        os_ = G.Stats()
        rc = G.lib().ggemm_grouped_dgemm(h.h, path, C.byref(cfg), probs, len(shapes), C.byref(os_))
        torch.cuda.synchronize()
        assert rc == 0
        first = [c.clone() for c in Cw]
        for g in range(len(shapes)):
            Cw[g].copy_(C0[g])
        st = G.Stats()
        rc = G.lib().ggemm_grouped_dgemm(h.h, path, C.byref(cfg), probs, len(shapes), C.byref(st))
        torch.cuda.synchronize()
        assert rc == 0
    for g in range(len(shapes)):
        assert torch.equal(first[g].view(torch.int64), Cw[g].view(torch.int64)), f"call 2 differs (problem {g})"

    plan = oracle_plan(shapes, cfg, path)
    emu = [e.num_moduli for e in plan if e.route == 0]
    assert st.num_fallback == sum(O.oracle().oz2o_route_is_fallback(e.route) for e in plan)
    if emu:
        assert (st.moduli_min, st.moduli_max) == (min(emu), max(emu))
    assert st.num_uncertified in (0, -1)

    rng = np.random.default_rng(11)
    u = 2.0 ** -53
    worst = 0.0
    for g, (m, n, k, a, b) in enumerate(shapes):
        if a == 0.0:   # BLAS: beta C0 exactly, A and B not referenced
            assert torch.equal(Cw[g], b * C0[g]), g
            continue
        ii = torch.from_numpy(rng.integers(0, m, 64)).cuda()
        jj = torch.from_numpy(rng.integers(0, n, 64)).cuda()
        av = A[g][:, ii].T.cpu().numpy().astype(np.longdouble)   # 64 x k
        bv = B[g][jj, :].cpu().numpy().astype(np.longdouble)     # 64 x k
        c0 = C0[g][jj, ii].cpu().numpy().astype(np.longdouble)
        got = Cw[g][jj, ii].cpu().numpy().astype(np.longdouble)
        ref = a * (av * bv).sum(axis=1) + b * c0
        den = abs(a) * np.abs(av * bv).sum(axis=1) + abs(b) * np.abs(c0)
        nt = k + (a != 1.0) + (b != 0.0)
        gam = nt * u / (1 - nt * u)
        r = float(np.max(np.abs(got - ref) / (gam * den)))
        assert r <= 1.0, (g, shapes[g], plan[g].route, r)
        worst = max(worst, r)
    say(f"  worst sampled err / gamma_n = {worst:.3g}; routes {sorted(set(e.route for e in plan))}, "
        f"moduli {st.moduli_min}..{st.moduli_max}, fallback {st.num_fallback}, repaired {st.num_repaired}")


def with_nonfinite(x, gen_, rate=1e-3):
    bad = torch.rand(x.shape, device="cuda", generator=gen_) < rate
    kind = torch.randint(0, 3, x.shape, device="cuda", generator=gen_)
    vals = torch.tensor([float("nan"), float("inf"), float("-inf")], dtype=torch.float64, device="cuda")
    return torch.where(bad, vals[kind], x)


def test_hard_numerics_full_size():
    """The reference's hard-numerics group at full size: G = 32 of 2048^3 plus 4 of 2048 x 2048 x
    65536, (U-0.5)exp(4Z), 0.1 % of A and B entries NaN / +-Inf at seeded positions, AUTO with
    repair ON.  Almost every row and column is non-finite, so nearly all entries take the FP64
    safety path.  Checked on every entry: C is non-finite exactly where row i of A or column j of
    B is (a NaN/Inf input makes its products non-finite and the class -- NaN, +Inf, -Inf -- does
    not depend on the summation order); the safety-fallback count equals the number of such
    entries of the emulated problems.  Sampled: the class of non-finite entries matches a host
    dot, finite entries are within gamma_n of an 80-bit dot; routes as the oracle planner's;
    bitwise reproducible."""
    shapes = [(2048, 2048, 2048, 1.0, 0.0)] * 32 + [(2048, 2048, 65536, 1.0, 0.0)] * 4
    g_ = torch.Generator(device="cuda")
    g_.manual_seed(5)
    A = [with_nonfinite(gen((k, m), g_, 4.0), g_) for (m, n, k, a, b) in shapes]
    B = [with_nonfinite(gen((n, k), g_, 4.0), g_) for (m, n, k, a, b) in shapes]
    Cw = [torch.zeros((n, m), dtype=torch.float64, device="cuda") for (m, n, k, a, b) in shapes]
    probs = G.problems_array([G.Problem(m, n, k, A[g].data_ptr(), m, B[g].data_ptr(), k, Cw[g].data_ptr(), m, a, b)
                              for g, (m, n, k, a, b) in enumerate(shapes)])
    tot = [sum(s[0] * s[2] for s in shapes), sum(s[2] * s[1] for s in shapes), sum(s[0] * s[1] for s in shapes)]
    cfg = G.Config(0, 1e-15, 1, G.REPAIR_ON)
    say("hard numerics full size (G = 32 x 2048^3 + 4 x 2048^2 x 65536, 0.1 % NaN/Inf)")
    import os
    saved = os.environ.get("GGEMM_STATS_REPAIR")
    os.environ["GGEMM_STATS_REPAIR"] = "1"   # device counters in the stats (read at creation)
    try:
        h = G.Handle(len(shapes), *tot)
    finally:
        if saved is None:
            os.environ.pop("GGEMM_STATS_REPAIR")
        else:
            os.environ["GGEMM_STATS_REPAIR"] = saved
    with h:
        st = G.Stats()
        rc = G.lib().ggemm_grouped_dgemm(h.h, G.PATH_AUTO, C.byref(cfg), probs, len(shapes), C.byref(st))
        torch.cuda.synchronize()
        assert rc == 0
        first = [c.clone() for c in Cw]
        st2 = G.Stats()
        rc = G.lib().ggemm_grouped_dgemm(h.h, G.PATH_AUTO, C.byref(cfg), probs, len(shapes), C.byref(st2))
        torch.cuda.synchronize()
        assert rc == 0
    for g in range(len(shapes)):
        same = (first[g].view(torch.int64) == Cw[g].view(torch.int64)) | (torch.isnan(first[g]) & torch.isnan(Cw[g]))
        assert bool(same.all()), f"call 2 differs (problem {g})"

    plan = oracle_plan(shapes, cfg, G.PATH_AUTO)
    emu = [e.num_moduli for e in plan if e.route == 0]
    assert st.num_fallback == sum(O.oracle().oz2o_route_is_fallback(e.route) for e in plan)
    if emu:
        assert (st.moduli_min, st.moduli_max) == (min(emu), max(emu))
    assert st.num_uncertified == 0

    safety = 0
    rng = np.random.default_rng(13)
    u = 2.0 ** -53
    for g, (m, n, k, a, b) in enumerate(shapes):
        row_ok = torch.isfinite(A[g]).all(dim=0)   # rows of A (A[g] is k x m)
        col_ok = torch.isfinite(B[g]).all(dim=1)   # columns of B (B[g] is n x k)
        fin = torch.isfinite(Cw[g])                # n x m
        want = col_ok[:, None] & row_ok[None, :]
        assert torch.equal(fin, want), f"non-finite pattern differs (problem {g})"
        if plan[g].route == 0:
            safety += m * n - int(row_ok.sum()) * int(col_ok.sum())
        ii = rng.integers(0, m, 64)
        jj = rng.integers(0, n, 64)
        av = A[g][:, torch.from_numpy(ii).cuda()].T.cpu().numpy()
        bv = B[g][torch.from_numpy(jj).cuda(), :].cpu().numpy()
        got = Cw[g][torch.from_numpy(jj).cuda(), torch.from_numpy(ii).cuda()].cpu().numpy()
        with np.errstate(invalid="ignore", over="ignore"):
            d = (av * bv).sum(axis=1)   # float64: only its class is used for non-finite entries
        for s in range(64):
            if not np.isfinite(got[s]) or not np.isfinite(d[s]):
                assert (np.isnan(got[s]) and np.isnan(d[s])) or got[s] == d[s], (g, s, got[s], d[s])
                continue
            al, bl = av[s].astype(np.longdouble), bv[s].astype(np.longdouble)
            ref = (al * bl).sum()
            den = np.abs(al * bl).sum()
            gam = k * u / (1 - k * u)
            assert abs(got[s] - ref) <= gam * den, (g, s)
    assert st.num_safety_fallback == safety
    say(f"  safety {safety}, repaired {st.num_repaired}, fallback {st.num_fallback}, "
        f"routes {sorted(set(e.route for e in plan))}, moduli {st.moduli_min}..{st.moduli_max}")
