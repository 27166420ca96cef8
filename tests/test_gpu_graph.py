"""Plan / execute as a hipGraph (tests/test_graph.cu T1-T3 semantics): the planned call equals
the direct call bit for bit with equal stats, on the handle's stream and on another stream
interleaved with direct calls, and after pointer updates there and back."""
import ctypes as C

import numpy as np
import pytest
import torch

import ggemm as G
import oracle_lib as O
from gpu_util import host, same_bits, say
from test_gpu_grouped import CFG_AUTO, Case, oracle_plan

pytestmark = pytest.mark.gpu

WORKLOADS = {
    "tiny64": [(32, 32, 64)] * 64,
    "moe": [(int(m), 256, 512) for m in np.random.default_rng(3).integers(16, 513, 16)],
    "mixed": [(int(a), int(b), int(c)) for a, b, c in np.random.default_rng(4).integers(8, 385, (14, 3))]
             + [(0, 64, 64), (48, 40, 0)],
}


def _problems(case, Cs, alpha, beta):
    return [G.Problem(h.m, h.n, h.k, a.data_ptr(), h.lda, b.data_ptr(), h.ldb, c.data_ptr(), h.ldc, alpha, beta)
            for h, a, b, c in zip(case.hp, case.dA, case.dB, Cs)]


def _copy(dst, case):
    for d, h in zip(dst, case.hp):
        d.copy_(torch.from_numpy(h.C0))


@pytest.mark.parametrize("name", sorted(WORKLOADS))
@pytest.mark.parametrize("path", [G.PATH_EMU_GROUPED, G.PATH_AUTO])
def test_plan_matches_direct(name, path):
    shapes = WORKLOADS[name]
    X = Case(shapes, 11, phi=1.0)
    Y = Case(shapes, 22, phi=1.0)
    cfg = CFG_AUTO if path == G.PATH_AUTO else G.Config(0, 1e-15, 0, 0)
    hs = torch.cuda.Stream()
    s2 = torch.cuda.Stream()
    sizes = X.sizes()
    h = G.Handle(len(shapes), 4 * sizes[0], 4 * sizes[1], sizes[2], stream=hs.cuda_stream)
    mk = lambda case: [torch.empty_like(d) for d in case.dC]
    Cref, Cg, Cref2, Cg2 = mk(X), mk(X), mk(Y), mk(Y)
    alpha, beta = 1.5, 0.5
    _copy(Cref, X)
    _copy(Cg, X)
    torch.cuda.synchronize()
    say(f"graph T1 {name} path={path}")
    rc, st_d = h.dgemm(path, cfg, _problems(X, Cref, alpha, beta))
    assert rc == 0
    arr = G.problems_array(_problems(X, Cg, alpha, beta))
    err = C.c_int(0)
    plan = G.lib().ggemm_make_plan_ex(h.h, path, C.byref(cfg), arr, len(shapes), C.byref(err))
    assert plan, err.value
    st_p = G.Stats()
    assert G.lib().ggemm_plan_get_stats(plan, C.byref(st_p)) == 0
    assert G.lib().ggemm_execute_plan(plan, hs.cuda_stream) == 0
    torch.cuda.synchronize()
    ref = np.concatenate([host(t) for t in Cref])
    assert same_bits(np.concatenate([host(t) for t in Cg]), ref)
    assert (st_p.num_fallback, st_p.moduli_min, st_p.moduli_max) == (st_d.num_fallback, st_d.moduli_min,
                                                                     st_d.moduli_max)
    assert st_p.kernel_launches == st_d.kernel_launches

    say(f"graph T2 {name}")
    py = G.problems_array(_problems(Y, Y.dC, alpha, 0.0))
    for _ in range(4):
        with torch.cuda.stream(s2):
            _copy(Cg, X)
        assert G.lib().ggemm_execute_plan(plan, s2.cuda_stream) == 0
        st = G.Stats()
        assert G.lib().ggemm_grouped_dgemm(h.h, path, C.byref(cfg), py, len(shapes), C.byref(st)) == 0
    torch.cuda.synchronize()
    assert same_bits(np.concatenate([host(t) for t in Cg]), ref)

    say(f"graph T3 {name}")
    _copy(Cref2, Y)
    _copy(Cg2, Y)
    torch.cuda.synchronize()
    st = G.Stats()
    assert G.lib().ggemm_grouped_dgemm(h.h, path, C.byref(cfg), G.problems_array(_problems(Y, Cref2, alpha, beta)),
                                       len(shapes), C.byref(st)) == 0
    PA = (C.c_void_p * len(shapes))(*[t.data_ptr() for t in Y.dA])
    PB = (C.c_void_p * len(shapes))(*[t.data_ptr() for t in Y.dB])
    PC = (C.c_void_p * len(shapes))(*[t.data_ptr() for t in Cg2])
    assert G.lib().ggemm_plan_update_pointers(plan, PA, PB, PC) == 0
    assert G.lib().ggemm_execute_plan(plan, s2.cuda_stream) == 0
    torch.cuda.synchronize()
    assert same_bits(np.concatenate([host(t) for t in Cg2]), np.concatenate([host(t) for t in Cref2]))
    _copy(Cg, X)
    torch.cuda.synchronize()
    PA = (C.c_void_p * len(shapes))(*[t.data_ptr() for t in X.dA])
    PB = (C.c_void_p * len(shapes))(*[t.data_ptr() for t in X.dB])
    PC = (C.c_void_p * len(shapes))(*[t.data_ptr() for t in Cg])
    assert G.lib().ggemm_plan_update_pointers(plan, PA, PB, PC) == 0
    assert G.lib().ggemm_execute_plan(plan, hs.cuda_stream) == 0
    torch.cuda.synchronize()
    assert same_bits(np.concatenate([host(t) for t in Cg]), ref)
    G.lib().ggemm_destroy_plan(plan)
    h.close()


def test_plan_rejects_other_paths_and_bad_pointers():
    X = Case([(16, 16, 16)], 1, phi=0.0)
    h = G.Handle(1, *X.sizes())
    arr = G.problems_array(X.problems())
    err = C.c_int(0)
    for path in (G.PATH_NATIVE_LOOP, G.PATH_EMU_LOOP, G.PATH_EMU_LOOP_BATCHED):
        assert not G.lib().ggemm_make_plan_ex(h.h, path, None, arr, 1, C.byref(err))
        assert err.value == G.GGEMM_ERR_INVALID
    plan = G.lib().ggemm_make_plan(h.h, G.PATH_AUTO, None, arr, 1)
    assert plan
    null = (C.c_void_p * 1)(None)
    assert G.lib().ggemm_plan_update_pointers(plan, None, None, null) == G.GGEMM_ERR_INVALID
    G.lib().ggemm_destroy_plan(plan)
    h.close()


def test_plan_update_pointers_long_k_matches_oracle():
    """A plan whose calls take the long-k production layout (row-major residues, blocked digits;
    largest Kp > 4096), executed on data set X, re-pointed to Y (ggemm_plan_update_pointers) and
    executed again: both outputs bitwise equal to the oracle's in COUNT mode."""
    shapes = [(256, 256, 4160)] * 2 + [(128, 96, 16384)]
    X = Case(shapes, 61, phi=1.0, beta=0.5)
    Y = Case(shapes, 62, phi=1.0, beta=0.5)
    cfg = G.Config(0, 1e-15, 0, G.REPAIR_COUNT)
    rc, plan_o = oracle_plan(X, cfg, G.PATH_EMU_GROUPED)
    assert rc == 0
    h = G.Handle(len(shapes), *[max(a, b) for a, b in zip(X.sizes(), Y.sizes())])
    X.reset_C()
    Y.reset_C()
    arr = G.problems_array(X.problems())
    err = C.c_int(0)
    plan = G.lib().ggemm_make_plan_ex(h.h, G.PATH_EMU_GROUPED, C.byref(cfg), arr, len(shapes), C.byref(err))
    assert plan, err.value
    try:
        say("long-k plan on X")
        assert G.lib().ggemm_execute_plan(plan, None) == 0
        torch.cuda.synchronize()
        ptr = lambda ts: (C.c_void_p * len(shapes))(*[t.data_ptr() for t in ts])
        assert G.lib().ggemm_plan_update_pointers(plan, ptr(Y.dA), ptr(Y.dB), ptr(Y.dC)) == 0
        say("long-k plan re-pointed to Y")
        assert G.lib().ggemm_execute_plan(plan, None) == 0
        torch.cuda.synchronize()
        for case in (X, Y):
            for g, (hp, e) in enumerate(zip(case.hp, plan_o)):
                Co, _ = hp.emulate(O.REPAIR_COUNT, e.num_moduli)
                assert same_bits(case.C(g), Co), f"problem {g} differs"
    finally:
        G.lib().ggemm_destroy_plan(plan)
        h.close()


def test_persistent_plan_replays_match_oracle():
    """A plan captured with the persistent work-stealing INT8 kernel (GGEMM_I8_SCHED=persistent at
    handle creation) replayed four times, alternating two data sets, with eager work between the
    replays: the queue counters live in the plan's schedule image and reset themselves, so every
    replay is bitwise equal to the oracle (COUNT mode)."""
    import os
    shapes = [(300, 260, 700)] * 3 + [(96, 130, 2000), (520, 64, 90)]
    X = Case(shapes, 71, phi=1.0, beta=0.5)
    Y = Case(shapes, 72, phi=1.0, beta=0.5)
    cfg = G.Config(0, 1e-15, 0, G.REPAIR_COUNT)
    rc, plan_o = oracle_plan(X, cfg, G.PATH_EMU_GROUPED)
    assert rc == 0
    saved = dict(os.environ)
    os.environ["GGEMM_I8_SCHED"] = "persistent"
    try:
        h = G.Handle(len(shapes), *[max(a, b) for a, b in zip(X.sizes(), Y.sizes())])
    finally:
        os.environ.clear()
        os.environ.update(saved)
    arr = G.problems_array(X.problems())
    err = C.c_int(0)
    plan = G.lib().ggemm_make_plan_ex(h.h, G.PATH_EMU_GROUPED, C.byref(cfg), arr, len(shapes), C.byref(err))
    assert plan, err.value
    ptr = lambda ts: (C.c_void_p * len(shapes))(*[t.data_ptr() for t in ts])
    try:
        for rep in range(4):
            case = X if rep % 2 == 0 else Y
            case.reset_C()
            assert G.lib().ggemm_plan_update_pointers(plan, ptr(case.dA), ptr(case.dB), ptr(case.dC)) == 0
            say(f"persistent plan replay {rep}")
            assert G.lib().ggemm_execute_plan(plan, None) == 0
            torch.cuda.synchronize()
            torch.zeros(1 << 20, device="cuda").sum().item()   # eager work between replays
            for g, (hp, e) in enumerate(zip(case.hp, plan_o)):
                Co, _ = hp.emulate(O.REPAIR_COUNT, e.num_moduli)
                assert same_bits(case.C(g), Co), f"replay {rep}: problem {g} differs"
    finally:
        G.lib().ggemm_destroy_plan(plan)
        h.close()


@pytest.mark.parametrize("kernel", ["auto", "large"])
def test_plan_replays_alternate_nonfinite_and_finite_data(kernel):
    """One plan replayed on a data set with NaN / Inf entries and on a finite one, alternately
    (ggemm_plan_update_pointers between the runs), repair ON.  Prep marks problems with non-finite
    rows / columns and the reconstruct marks problems with flagged entries in the plan's device
    descriptors; a replay on finite data after one on non-finite data sees those marks still set
    and must take the general paths, so every run is compared with the oracle bit for bit.  In X
    every A row of problem 0 and every B column of problem 2 holds a non-finite value, so the INT8
    GEMM skips their tiles there; on Y, with the marks still set, it must compute them.  kernel
    large (GGEMM_I8_KERNEL at handle creation): the 256 x 256 kernel, whose packed products run in
    its tail workgroups as compacted tiles over prep's finite-row / finite-column lists (on Y every
    row and column, the marks still set) with the tail's queue counters reset by each replay."""
    shapes = [(200, 150, 300)] * 2 + [(64, 96, 1200), (130, 70, 40)]
    X = Case(shapes, 81, phi=2.0, alpha=1.5, beta=0.5)
    Y = Case(shapes, 82, phi=1.0, alpha=1.5, beta=0.5)
    rng = np.random.default_rng(83)
    bad = [np.nan, np.inf, -np.inf]
    for hp in X.hp:
        for arr, rows, cols, ld in ((hp.A, hp.m, hp.k, hp.lda), (hp.B, hp.k, hp.n, hp.ldb)):
            nbad = max(1, rows * cols // 1500)
            arr[rng.integers(0, rows, nbad) + rng.integers(0, cols, nbad) * ld] = rng.choice(bad, nbad)
    h0, h2 = X.hp[0], X.hp[2]
    for i in range(h0.m):
        h0.A[i + rng.integers(0, h0.k) * h0.lda] = bad[i % 3]
    for j in range(h2.n):
        h2.B[rng.integers(0, h2.k) + j * h2.ldb] = bad[j % 3]
    X.alloc()
    cfg = G.Config(0, 1e-15, 0, G.REPAIR_ON)
    rc, plan_o = oracle_plan(X, cfg, G.PATH_EMU_GROUPED)
    assert rc == 0
    want = {}
    for name, case in (("X", X), ("Y", Y)):
        want[name] = [hp.emulate(O.REPAIR_ON, e.num_moduli) for hp, e in zip(case.hp, plan_o)]
    assert sum(int(c[3]) for _, c in want["X"]) > 0 and sum(int(c[3]) for _, c in want["Y"]) == 0
    import os
    saved = dict(os.environ)
    if kernel == "large":
        os.environ["GGEMM_I8_KERNEL"] = "large"
    try:
        h = G.Handle(len(shapes), *[max(a, b) for a, b in zip(X.sizes(), Y.sizes())])
    finally:
        os.environ.clear()
        os.environ.update(saved)
    arr = G.problems_array(X.problems())
    err = C.c_int(0)
    plan = G.lib().ggemm_make_plan_ex(h.h, G.PATH_EMU_GROUPED, C.byref(cfg), arr, len(shapes), C.byref(err))
    assert plan, err.value
    ptr = lambda ts: (C.c_void_p * len(shapes))(*[t.data_ptr() for t in ts])
    try:
        for rep, name in enumerate(("X", "Y", "Y", "X", "Y")):
            case = X if name == "X" else Y
            case.reset_C()
            assert G.lib().ggemm_plan_update_pointers(plan, ptr(case.dA), ptr(case.dB), ptr(case.dC)) == 0
            say(f"plan replay {rep} on {name}, {kernel} kernel")
            assert G.lib().ggemm_execute_plan(plan, None) == 0
            torch.cuda.synchronize()
            if kernel == "large":
                assert G.lib().ggemm_profile_i8_kernel().decode() == "i8_large_kernel"
            for g, (Co, _) in enumerate(want[name]):
                assert same_bits(case.C(g), Co), f"replay {rep} ({name}): problem {g} differs"
    finally:
        G.lib().ggemm_destroy_plan(plan)
        h.close()
