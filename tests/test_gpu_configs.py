"""The reference's benchmark configurations at full size, emulated problems checked bit for bit
against the oracle: every entry of every emulated problem (uniform and ragged configs), every entry
of the finite-row x finite-column block of every problem plus sampled entries elsewhere (hard
config), sampled entries (large config, whose 1.5e14 multiply-adds the CPU oracle cannot redo).

Each output entry of the Ozaki-II pipeline depends only on its row of A, its column of B and its C0
entry (shifts, abs shifts and norm bounds are per row / column; CRT, certificate and repair per
entry), so the oracle run on the sub-problem (rows I of A, columns J of B, C0(I, J)) gives the exact
bits of those entries (tests/gpu_util.oracle_block).  Calls are checked in COUNT mode (uncertified
entries keep their emulated value, so an error in any stage shows) and in ON mode (repaired entries
take the FP64 dot, whose bits the oracle also gives).  Where the oracle covers every entry that can be
uncertified or repaired, the device counters must EQUAL the oracle's counts (num_uncertified in COUNT
mode, num_repaired in ON mode, num_safety_fallback), as the reference's numerics test requires
(tests/test_numerics_standalone.cu:400-433); on the large config they must be at least the sampled
counts.  Native-route problems (own FP64 MFMA GEMM, whose order differs from the reference's closed
vendor GEMM) are checked by the componentwise gamma_n gate against an 80-bit dot on sampled entries;
alpha = 0 problems must equal beta C0 exactly.  Stats (fallback count, moduli range) must equal the
oracle planner's, and a repeated call must reproduce every bit.

  uniform : G = 64 x 1024^3, (U-0.5)exp(0.5Z), alpha 1, beta 0.5            (EMU_GROUPED and AUTO)
  ragged  : G = 128, m, n log-U[64, 4096], k log-U[16, 8192], 8 alpha = 0    (AUTO and EMU_GROUPED)
  large   : G = 8 x 8192^2 x 16384, U(-1, 1), plan / execute with pointer updates over two data sets
  hard    : G = 32 x 2048^3 + 4 x 2048^2 x 65536, (U-0.5)exp(4Z), 0.1 % NaN / +-Inf, AUTO
Data are generated on the GPU with torch generators (fixed seeds), shapes with numpy (fixed seed)."""
import ctypes as C
import os

import numpy as np
import pytest
import torch

import ggemm as G
import oracle_lib as O
from gpu_util import gpu_block, oracle_block, oracle_full_many, read_counters, same_bits, say

pytestmark = pytest.mark.gpu
U53 = 2.0 ** -53


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


def gen(shape, gen_, phi, lo_hi=None):
    u = torch.rand(shape, dtype=torch.float64, device="cuda", generator=gen_)
    if lo_hi is not None:
        return lo_hi[0] + (lo_hi[1] - lo_hi[0]) * u
    u -= 0.5
    if phi:
        u *= torch.exp(phi * torch.randn(shape, dtype=torch.float64, device="cuda", generator=gen_))
    return u


def with_nonfinite(x, gen_, rate=1e-3):
    bad = torch.rand(x.shape, device="cuda", generator=gen_) < rate
    kind = torch.randint(0, 3, x.shape, device="cuda", generator=gen_)
    vals = torch.tensor([float("nan"), float("inf"), float("-inf")], dtype=torch.float64, device="cuda")
    return torch.where(bad, vals[kind], x)


def stats_handle(*args, **kw):
    """A handle whose calls report the device counters (GGEMM_STATS_REPAIR is read at creation)."""
    saved = os.environ.get("GGEMM_STATS_REPAIR")
    os.environ["GGEMM_STATS_REPAIR"] = "1"
    try:
        return G.Handle(*args, **kw)
    finally:
        if saved is None:
            os.environ.pop("GGEMM_STATS_REPAIR")
        else:
            os.environ["GGEMM_STATS_REPAIR"] = saved


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


def oz2_mode(repair):
    return {G.REPAIR_OFF: O.REPAIR_OFF, G.REPAIR_COUNT: O.REPAIR_COUNT, G.REPAIR_ON: O.REPAIR_ON}[repair]


def pick(rng, size, count, prefer=None):
    """count distinct indices below size; half of them from `prefer` (a boolean mask) when given."""
    count = min(count, size)
    if prefer is not None:
        good = np.flatnonzero(prefer)
        take = rng.choice(good, min(len(good), count // 2), replace=False) if len(good) else np.array([], dtype=int)
        rest = np.setdiff1d(np.arange(size), take)
        return np.sort(np.concatenate([take, rng.choice(rest, count - len(take), replace=False)]))
    return np.sort(rng.choice(size, count, replace=False))


def check_full(shapes, A, B, C0, Cw, plan, repair, blocks=None):
    """Every entry of every emulated problem bitwise against the oracle -- or, with blocks, the entries
    of rows I x columns J of problem g, blocks[g] = (I, J) -- on a thread pool.  Returns the oracle's
    counters [nonfinite vectors, uncertified, repaired, safety] summed over the entries covered."""
    jobs = []
    for g, (m, n, k, a, b) in enumerate(shapes):
        e = plan[g]
        if a == 0.0 or e.route != 0:
            continue
        I, J = blocks[g] if blocks is not None else (None, None)
        if I is None:
            assert tuple(A[g].shape) == (k, m) and tuple(B[g].shape) == (n, k) and tuple(Cw[g].shape) == (n, m)
            got = Cw[g].cpu().numpy()
        elif len(I) == 0 or len(J) == 0:
            continue
        else:
            got = gpu_block(Cw[g], I, J)
        jobs.append((g, A[g], B[g], C0[g], k, a, b, e.num_moduli, oz2_mode(repair), I, J, got))
    tot = np.zeros(4, dtype=np.int64)
    for g, eq, cnt, where in oracle_full_many(jobs):
        assert eq, f"problem {g} {shapes[g][:3]} N={plan[g].num_moduli}: entry (column, row) {where} differs"
        tot += cnt
    return tot


def check_problems(shapes, A, B, C0, Cw, plan, repair, rng, n_side=8, finite_masks=None, emulated=True):
    """Sampled entries of every problem against the oracle (emulated routes, bitwise; skipped with
    emulated=False), the gamma_n gate (native routes) or beta C0 (alpha = 0).  Returns the oracle
    counters summed over the samples and the worst native err / gamma_n."""
    tot = np.zeros(4, dtype=np.int64)
    worst = 0.0
    for g, (m, n, k, a, b) in enumerate(shapes):
        e = plan[g]
        if a == 0.0:   # BLAS: beta C0 exactly, A and B not referenced
            assert torch.equal(Cw[g], b * C0[g]), g
            continue
        if e.route == 0 and not emulated:
            continue
        pr, pc = (finite_masks[g] if finite_masks else (None, None))
        I = pick(rng, m, n_side, pr)
        J = pick(rng, n, n_side, pc)
        got = gpu_block(Cw[g], I, J)
        if e.route == 0:
            want, cnt = oracle_block(A[g], B[g], C0[g], k, a, b, e.num_moduli, oz2_mode(repair), I, J)
            assert same_bits(got, want), f"problem {g} {shapes[g][:3]} N={e.num_moduli}: sampled entries differ"
            tot += cnt
        else:
            ii, jj = torch.as_tensor(I, device="cuda"), torch.as_tensor(J, device="cuda")
            av = A[g][:k][:, ii].T.cpu().numpy().astype(np.longdouble)        # |I| x k
            bv = B[g][jj][:, :k].cpu().numpy().astype(np.longdouble)          # |J| x k
            c0 = (np.zeros((len(J), len(I))) if C0[g] is None else
                  C0[g][jj][:, ii].cpu().numpy()).astype(np.longdouble)         # |J| x |I|
            ref = a * (bv @ av.T) + b * c0
            den = abs(a) * (np.abs(bv) @ np.abs(av).T) + abs(b) * np.abs(c0)
            nt = k + (a != 1.0) + (b != 0.0)
            gam = nt * U53 / (1 - nt * U53)
            r = float(np.max(np.abs(got.astype(np.longdouble) - ref) / (gam * den)))
            assert r <= 1.0, (g, shapes[g], G.ROUTES[e.route], r)
            worst = max(worst, r)
    return tot, worst


def check_stats(st, shapes, plan, counts, exact):
    """Routes and moduli as the oracle planner's; device counters equal to the oracle's counts
    (exact: the oracle covered every entry that can be uncertified, repaired or safety) or at least
    the sampled ones."""
    emu = [e.num_moduli for e in plan if e.route == 0]
    assert st.num_fallback == sum(O.oracle().oz2o_route_is_fallback(e.route) for e in plan)
    if emu:
        assert (st.moduli_min, st.moduli_max) == (min(emu), max(emu))
    got = (st.num_uncertified, st.num_repaired, st.num_safety_fallback)
    want = (int(counts[1]), int(counts[2]), int(counts[3]))
    if exact:
        assert got == want, f"device counters (uncertified, repaired, safety) {got} != oracle {want}"
    else:
        assert all(x >= y for x, y in zip(got, want)), (got, want)


def run_call(h, path, cfg, probs, n):
    st = G.Stats()
    rc = G.lib().ggemm_grouped_dgemm(h.h, path, C.byref(cfg), probs, n, C.byref(st))
    torch.cuda.synchronize()
    assert rc == 0, rc
    return st


def problems(shapes, A, B, Cw):
    return G.problems_array([G.Problem(m, n, k, A[g].data_ptr(), A[g].shape[1], B[g].data_ptr(), B[g].shape[1],
                                       Cw[g].data_ptr(), Cw[g].shape[1], a, b)
                             for g, (m, n, k, a, b) in enumerate(shapes)])


def sizes(shapes):
    return [sum(s[0] * s[2] for s in shapes), sum(s[2] * s[1] for s in shapes), sum(s[0] * s[1] for s in shapes)]


@pytest.mark.parametrize("path", [G.PATH_EMU_GROUPED, G.PATH_AUTO])
def test_uniform_config_sampled_bitwise(path):
    shapes = [(1024, 1024, 1024, 1.0, 0.5)] * 64
    g_ = torch.Generator(device="cuda")
    g_.manual_seed(2)
    A = [gen((k, m), g_, 0.5) for (m, n, k, a, b) in shapes]
    B = [gen((n, k), g_, 0.5) for (m, n, k, a, b) in shapes]
    C0 = [gen((n, m), g_, 0.0) for (m, n, k, a, b) in shapes]
    Cw = [c.clone() for c in C0]
    probs = problems(shapes, A, B, Cw)
    rng = np.random.default_rng(21)
    with stats_handle(len(shapes), *sizes(shapes)) as h:
        for repair in (G.REPAIR_COUNT, G.REPAIR_ON):
            cfg = G.Config(0, 1e-15, 1, repair)
            say(f"uniform G=64 x 1024^3 path={path} repair={repair}")
            for g in range(len(shapes)):
                Cw[g].copy_(C0[g])
            st = run_call(h, path, cfg, probs, len(shapes))
            plan = oracle_plan(shapes, cfg, path)
            counts = check_full(shapes, A, B, C0, Cw, plan, repair)
            _, worst = check_problems(shapes, A, B, C0, Cw, plan, repair, rng, emulated=False)
            check_stats(st, shapes, plan, counts, exact=True)
            say(f"  routes {sorted({G.ROUTES[e.route] for e in plan})}, moduli {st.moduli_min}..{st.moduli_max}, "
                f"uncertified {st.num_uncertified}, repaired {st.num_repaired} (oracle, every entry: "
                f"{counts.tolist()}), native worst err/gamma {worst:.3g}")


@pytest.mark.parametrize("path", [G.PATH_AUTO, G.PATH_EMU_GROUPED])
def test_ragged_config_sampled_bitwise(path):
    shapes = ragged_shapes()
    g_ = torch.Generator(device="cuda")
    g_.manual_seed(3)
    A = [gen((k, m), g_, 1.0) for (m, n, k, a, b) in shapes]    # column-major m x k, lda = m
    B = [gen((n, k), g_, 1.0) for (m, n, k, a, b) in shapes]    # column-major k x n, ldb = k
    C0 = [gen((n, m), g_, 0.0) for (m, n, k, a, b) in shapes]   # column-major m x n, ldc = m
    Cw = [c.clone() for c in C0]
    probs = problems(shapes, A, B, Cw)
    tot = sizes(shapes)
    rng = np.random.default_rng(31)
    say(f"ragged G=128 full size path={path}: {tot[0] / 1e6:.0f}M + {tot[1] / 1e6:.0f}M + {tot[2] / 1e6:.0f}M elements")
    with stats_handle(len(shapes), *tot, min_k=16) as h:
        for repair in (G.REPAIR_COUNT, G.REPAIR_ON):
            cfg = G.Config(0, 1e-15, 1, repair)
            for g in range(len(shapes)):
                Cw[g].copy_(C0[g])
            st = run_call(h, path, cfg, probs, len(shapes))
            first = [c.clone() for c in Cw]
            for g in range(len(shapes)):
                Cw[g].copy_(C0[g])
            run_call(h, path, cfg, probs, len(shapes))
            for g in range(len(shapes)):
                assert torch.equal(first[g].view(torch.int64), Cw[g].view(torch.int64)), f"call 2 differs ({g})"
            del first
            plan = oracle_plan(shapes, cfg, path)
            counts = check_full(shapes, A, B, C0, Cw, plan, repair)
            _, worst = check_problems(shapes, A, B, C0, Cw, plan, repair, rng, emulated=False)
            check_stats(st, shapes, plan, counts, exact=True)
            say(f"  repair={repair}: routes {sorted({G.ROUTES[e.route] for e in plan})}, moduli "
                f"{st.moduli_min}..{st.moduli_max}, fallback {st.num_fallback}, uncertified {st.num_uncertified}, "
                f"repaired {st.num_repaired}, oracle counts over every entry {counts.tolist()}, native worst {worst:.3g}")


def test_large_config_plan_execute_pointer_updates_sampled_bitwise():
    """G = 8 x 8192^2 x 16384, U(-1, 1), alpha 1, beta 0, EMU_GROUPED at 1e-15 (N = 16), as the
    benchmark runs it: a plan made once (hipGraph), then per run ggemm_plan_update_pointers and
    ggemm_execute_plan.  Two data sets X, Y and two output buffers: plan on X -> C1, update to
    Y -> C2, back to X -> C2; every result sampled bitwise against the oracle on its own data,
    REPAIR_ON and (a second plan) REPAIR_COUNT.  Row-major residues, the 256 x 256 INT8 kernel and
    blocked digits are the production choices at this size."""
    shapes = [(8192, 8192, 16384, 1.0, 0.0)] * 8
    Gp = len(shapes)
    m, n, k = shapes[0][:3]
    g_ = torch.Generator(device="cuda")
    g_.manual_seed(4)
    X = ([gen((k, m), g_, 0.0, (-1.0, 1.0)) for _ in range(Gp)], [gen((n, k), g_, 0.0, (-1.0, 1.0)) for _ in range(Gp)])
    Y = ([gen((k, m), g_, 0.0, (-1.0, 1.0)) for _ in range(Gp)], [gen((n, k), g_, 0.0, (-1.0, 1.0)) for _ in range(Gp)])
    C1 = [torch.zeros((n, m), dtype=torch.float64, device="cuda") for _ in range(Gp)]
    C2 = [torch.zeros((n, m), dtype=torch.float64, device="cuda") for _ in range(Gp)]
    rng = np.random.default_rng(41)
    ptrs = lambda T: (C.c_void_p * Gp)(*[t.data_ptr() for t in T])
    say("large G=8 x 8192^2 x 16384 via plan / update_pointers / execute")
    try:
        with stats_handle(Gp, *sizes(shapes)) as h:
            for repair in (G.REPAIR_ON, G.REPAIR_COUNT):
                cfg = G.Config(0, 1e-15, 1, repair)
                probs = problems(shapes, X[0], X[1], C1)
                err = C.c_int(0)
                plan = G.lib().ggemm_make_plan_ex(h.h, G.PATH_EMU_GROUPED, C.byref(cfg), probs, Gp, C.byref(err))
                assert plan, err.value
                try:
                    st = G.Stats()
                    assert G.lib().ggemm_plan_get_stats(plan, C.byref(st)) == 0
                    oplan = oracle_plan(shapes, cfg, G.PATH_EMU_GROUPED)
                    assert (st.num_fallback, st.moduli_min, st.moduli_max, st.kernel_launches) == (0, 16, 16, 6)
                    assert all(e.route == 0 and e.num_moduli == 16 for e in oplan)
                    for (data, out, tag) in ((X, C1, "X -> C1"), (Y, C2, "Y -> C2"), (X, C2, "X -> C2")):
                        if tag != "X -> C1":
                            assert G.lib().ggemm_plan_update_pointers(plan, ptrs(data[0]), ptrs(data[1]), ptrs(out)) == 0
                        read_counters(reset=True)
                        assert G.lib().ggemm_execute_plan(plan, None) == 0
                        torch.cuda.synchronize()
                        dev = read_counters(reset=True)   # the device counters of this execution
                        sampled, _ = check_problems(shapes, data[0], data[1], [None] * Gp, out, oplan, repair, rng)
                        st.num_uncertified, st.num_repaired = dev.uncertified, dev.repaired
                        st.num_safety_fallback = dev.safety_fallback
                        check_stats(st, shapes, oplan, sampled, exact=False)
                        say(f"  repair={repair} {tag}: sampled oracle counts {sampled.tolist()}, device uncertified "
                            f"{dev.uncertified}, repaired {dev.repaired}, safety {dev.safety_fallback}")
                finally:
                    G.lib().ggemm_destroy_plan(plan)
    finally:
        del X, Y, C1, C2
        torch.cuda.empty_cache()


def test_hard_numerics_config_sampled_bitwise():
    """G = 32 x 2048^3 + 4 x 2048^2 x 65536, (U-0.5)exp(4Z), 0.1 % of A and B entries NaN / +-Inf,
    AUTO with repair ON (then COUNT).  Almost every row and column holds a non-finite value, so
    nearly all entries take the FP64 safety path.  Checked: every entry of each problem's
    finite-row x finite-column block bitwise against the oracle -- the only entries that can be
    certified, uncertified or repaired -- so num_repaired (ON) and num_uncertified (COUNT) must
    equal the oracle's counts; sampled entries elsewhere bitwise too (safety entries); on every entry
    C is non-finite exactly where row i of A or column j of B is; the safety count equals the number
    of such entries of the emulated problems; routes as the oracle planner's; a repeated call
    reproduces every bit."""
    shapes = [(2048, 2048, 2048, 1.0, 0.0)] * 32 + [(2048, 2048, 65536, 1.0, 0.0)] * 4
    g_ = torch.Generator(device="cuda")
    g_.manual_seed(5)
    A = [with_nonfinite(gen((k, m), g_, 4.0), g_) for (m, n, k, a, b) in shapes]
    B = [with_nonfinite(gen((n, k), g_, 4.0), g_) for (m, n, k, a, b) in shapes]
    Cw = [torch.zeros((n, m), dtype=torch.float64, device="cuda") for (m, n, k, a, b) in shapes]
    probs = problems(shapes, A, B, Cw)
    rows_ok = [torch.isfinite(A[g]).all(dim=0).cpu().numpy() for g in range(len(shapes))]
    cols_ok = [torch.isfinite(B[g]).all(dim=1).cpu().numpy() for g in range(len(shapes))]
    rng = np.random.default_rng(51)
    say("hard numerics full size (G = 32 x 2048^3 + 4 x 2048^2 x 65536, 0.1 % NaN/Inf)")
    with stats_handle(len(shapes), *sizes(shapes)) as h:
        for repair in (G.REPAIR_ON, G.REPAIR_COUNT):
            cfg = G.Config(0, 1e-15, 1, repair)
            st = run_call(h, G.PATH_AUTO, cfg, probs, len(shapes))
            first = [c.clone() for c in Cw]
            run_call(h, G.PATH_AUTO, cfg, probs, len(shapes))
            for g in range(len(shapes)):
                same = (first[g].view(torch.int64) == Cw[g].view(torch.int64)) | (torch.isnan(first[g]) &
                                                                                   torch.isnan(Cw[g]))
                assert bool(same.all()), f"call 2 differs (problem {g})"
            del first
            plan = oracle_plan(shapes, cfg, G.PATH_AUTO)
            safety = 0
            for g, (m, n, k, a, b) in enumerate(shapes):
                fin = torch.isfinite(Cw[g])                # n x m
                want = torch.from_numpy(cols_ok[g]).cuda()[:, None] & torch.from_numpy(rows_ok[g]).cuda()[None, :]
                assert torch.equal(fin, want), f"non-finite pattern differs (problem {g})"
                if plan[g].route == 0:
                    safety += m * n - int(rows_ok[g].sum()) * int(cols_ok[g].sum())
            sampled, worst = check_problems(shapes, A, B, [None] * len(shapes), Cw, plan, repair, rng,
                                            finite_masks=list(zip(rows_ok, cols_ok)))
            blocks = [(np.flatnonzero(r), np.flatnonzero(c)) for r, c in zip(rows_ok, cols_ok)]
            counts = check_full(shapes, A, B, [None] * len(shapes), Cw, plan, repair, blocks=blocks)
            assert counts[3] == 0
            counts[3] = safety
            check_stats(st, shapes, plan, counts, exact=True)
            if repair == G.REPAIR_ON:
                assert st.num_uncertified == 0
            say(f"  repair={repair}: safety {safety}, repaired {st.num_repaired}, uncertified {st.num_uncertified}, "
                f"fallback {st.num_fallback}, routes {sorted({G.ROUTES[e.route] for e in plan})}, moduli "
                f"{st.moduli_min}..{st.moduli_max}, oracle counts over the finite blocks {counts.tolist()}, "
                f"sampled {sampled.tolist()}")
