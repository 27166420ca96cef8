"""The planner -- the library's ggemm_plan and the oracle's oz2o_plan -- against what the reference's
own planner unit test (tests/test_planner.cpp) asserts and printed on its run
(results/planner_unit_590223/test_planner.log, transcribed to tests/golden/planner_unit_log.json by
tests/golden/extract_planner_log.py).  Device model: tests/testdata/planner/valid.json with 132 SMs
(fp64 5e13, int8 1e15, bw 3e12, tiny 32^3), exactly the test's model_h200().

What the log pins beyond the route table:
  * the tile chosen for 8 shapes in large groups (padding efficiency),
  * the wave-quantisation shrink of 4 small groups (tile and N),
  * for 4 shapes planned alone and in a group of 4000: tile, route and t_emu to 3 significant
    digits -- t_emu is the cost model's sum of prep, INT8 GEMM (with its C32 write) and
    reconstruct terms, so a dropped or mis-weighted term changes the printed digits,
  * the route histograms of a 65535-problem generated group on AUTO and EMU_GROUPED.
Plus the test's own assertions: UNSAFE for an offending problem at index 2, PRECISION for an
unreachable target, N = clamp(choose_cw(k, 16)) on AUTO, fixed N on tile 0 for EMU_GROUPED, the
cost / route consistency after re-evaluation, determinism, and no heap allocation inside
ggemm_plan (an interposing C++ harness, tests/planner_alloc/count_allocs.cpp)."""
import ctypes as C
import json
import math
import os
import subprocess
from pathlib import Path

import numpy as np
import pytest

import ggemm as G
import oracle_lib as O

REPO = Path(__file__).resolve().parents[1]
GOLDEN = REPO / "tests" / "golden"
LOG = json.loads((GOLDEN / "planner_unit_log.json").read_text())
ROUTES = ["EMU", "EMPTY", "K_ZERO", "K_TOO_LARGE", "TINY", "UNPROFITABLE", "PRECISION", "SMALL_K", "ALPHA_ZERO"]
TILE = {0: 128, 1: 64, 2: 32}
KMAX = G.MAX_K_EXACT


def valid_dm():
    old = os.environ.get("GGEMM_CALIB_JSON")
    os.environ["GGEMM_CALIB_JSON"] = str(GOLDEN / "planner_valid.json")
    try:
        dm = G.DeviceModel()
        G.lib().ggemm_device_model_init(C.byref(dm), b"NVIDIA H200", 9, 0, 132)
    finally:
        if old is None:
            os.environ.pop("GGEMM_CALIB_JSON", None)
        else:
            os.environ["GGEMM_CALIB_JSON"] = old
    m = LOG["model"]
    assert (dm.num_sms, dm.fp64_flops, dm.int8_ops, dm.mem_bw, dm.tiny_mnk) == \
        (m["num_sms"], m["fp64"], m["i8"], m["bw"], m["tiny_mnk"])
    return dm


DM = None


def dm():
    global DM
    if DM is None:
        DM = valid_dm()
    return DM


def P(m, n, k, alpha=1.0, beta=0.0):
    return (m, n, k, alpha, beta)


def plan_lib(shapes, nm, fb, path, tgt=1e-15):
    arr = G.problems_array([G.Problem(m, n, k, None, max(1, m), None, max(1, k), None, max(1, m), a, b)
                            for (m, n, k, a, b) in shapes])
    out = (G.PlanEntry * max(len(shapes), 1))()
    cfg = G.Config(nm, tgt, fb, 0)
    rc = G.lib().ggemm_plan(arr, len(shapes), C.byref(cfg), path, C.byref(dm()), out)
    return rc, list(out)[:len(shapes)]


def plan_oracle(shapes, nm, fb, path, tgt=1e-15):
    arr = (O.Shape * max(len(shapes), 1))(*[O.Shape(*s) for s in shapes])
    d = dm()
    odm = O.DeviceModel(d.num_sms, d.fp64_flops, d.int8_ops, d.mem_bw, d.tiny_mnk)
    out = (O.PlanEntry * max(len(shapes), 1))()
    rc = O.oracle().oz2o_plan(arr, len(shapes), nm, tgt, fb, path, C.byref(odm), 16.0, out)
    return rc, list(out)[:len(shapes)]


PLANNERS = {"library": plan_lib, "oracle": plan_oracle}


def make_group(G_, seed):
    """tests/test_planner.cpp:371-386 (LCG s = 1664525 s + 1013904223 mod 2^32)."""
    s = seed
    out = []

    def nxt(lo, hi):
        nonlocal s
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        return lo + ((s >> 8) % (hi - lo + 1))

    for _ in range(G_):
        r = nxt(0, 99)
        m, n, k = nxt(1, 2048), nxt(1, 2048), nxt(1, 8192)
        if r < 3:
            k = 0
        elif r < 5:
            m = 0
        elif r < 7:
            k = KMAX + nxt(1, 1000)
        elif r < 12:
            k = nxt(1, 16)
        out.append(P(m, n, k, 0.0 if r == 50 else 1.0, 1.0 if r & 1 else 0.0))
    return out


@pytest.mark.parametrize("who", sorted(PLANNERS))
def test_route_assertions_of_the_reference_test(who):
    plan = PLANNERS[who]
    # tests/test_planner.cpp:164-170: fb = 0 error reported for an offending problem at index 2
    rc, _ = plan([P(128, 128, 128), P(64, 64, 64), P(128, 128, KMAX + 32)], 0, 0, G.PATH_AUTO)
    assert rc == G.GGEMM_ERR_UNSAFE
    # :172-186: unreachable target 1e-40 on the fixed-target path: fb = 0 -> UNSAFE, fb = 1 -> PRECISION
    assert O.oracle().oz2o_choose_num_moduli(100000, 1e-40) < 0
    rc, _ = plan([P(1024, 1024, 100000)], 0, 0, G.PATH_EMU_GROUPED, tgt=1e-40)
    assert rc == G.GGEMM_ERR_UNSAFE
    rc, e = plan([P(1024, 1024, 100000)], 0, 1, G.PATH_EMU_GROUPED, tgt=1e-40)
    assert rc == 0 and ROUTES[e[0].route] == "PRECISION"
    # :189-208: AUTO adaptive N = clamp(choose_cw(k, 16), 2, 20); fixed N = 7 kept, tile 0 on EMU_GROUPED
    for k in (17, 32, 100, 512, 1024, 4096, 16384, 65536, KMAX):
        rc, e = plan([P(4096, 4096, k)], 0, 0, G.PATH_AUTO)
        want = min(max(O.oracle().oz2o_choose_num_moduli_cw(k, 16.0), 2), 20)
        assert rc == 0 and ROUTES[e[0].route] == "EMU" and e[0].num_moduli == want, k
        rc, e = plan([P(4096, 4096, k)], 7, 0, G.PATH_AUTO)
        assert rc == 0 and e[0].num_moduli == 7, k
        rc, e = plan([P(4096, 4096, k)], 7, 0, G.PATH_EMU_GROUPED)
        assert rc == 0 and e[0].num_moduli == 7 and e[0].tile_cfg == 0, k


@pytest.mark.parametrize("who", sorted(PLANNERS))
def test_tile_choice_and_shrink_match_the_log(who):
    plan = PLANNERS[who]
    for c in LOG["tiles"]:   # 4a: no fallback, every problem emulated
        rc, e = plan([P(c["m"], c["n"], 4096)] * c["G"], 0, 0, G.PATH_AUTO)
        assert rc == 0
        assert {x.tile_cfg for x in e} == {e[0].tile_cfg}, "identical problems got different tiles"
        assert TILE[e[0].tile_cfg] == c["tile"], c
    for c in LOG["shrink"]:  # 4b
        rc, e = plan([P(c["m"], c["n"], c["k"])] * c["G"], 0, 0, G.PATH_AUTO)
        assert rc == 0
        tiles128 = c["G"] * (e[0].num_moduli + 1) * math.ceil(c["m"] / 128) * math.ceil(c["n"] / 128)
        assert (e[0].num_moduli, tiles128, TILE[e[0].tile_cfg]) == (c["N"], c["tiles128"], c["tile"]), c


@pytest.mark.parametrize("who", sorted(PLANNERS))
def test_reevaluated_costs_match_the_log(who):
    """4c-ii: a shape planned alone (tile shrunk by the wave quantisation) and in a group of 4000
    (tile kept): tile, route and t_emu as printed by the reference (%.3g)."""
    plan = PLANNERS[who]
    for c in LOG["reeval"]:
        p = P(c["m"], c["m"], c["k"])
        for key, G_ in (("alone", 1), ("group", 4000)):
            rc, e = plan([p] * G_, 0, 1, G.PATH_AUTO)
            assert rc == 0
            got = [TILE[e[0].tile_cfg], ROUTES[e[0].route], f"{e[0].t_emu_s:.3g}"]
            assert got == c[key], (c["m"], key, got)


@pytest.mark.parametrize("who", sorted(PLANNERS))
def test_costs_consistent_with_routes_after_reevaluation(who):
    """4c-i (tests/test_planner.cpp:315-346): every EMU entry has t_emu <= t_native and every
    UNPROFITABLE one t_emu > t_native, for groups of 1, 8 and 726 mixed shapes."""
    plan = PLANNERS[who]
    sz = [24, 48, 96, 160, 224, 256, 384, 512, 768, 1024, 2048]
    kk = [17, 64, 256, 1024, 4096, 16384]
    mix = [P(m, n, k, 1.0, 0.0 if (m + n) % 3 else 1.0) for m in sz for n in sz for k in kk]
    for G_ in (1, 8, len(mix)):
        start = 0
        while start + G_ <= len(mix):
            rc, e = plan(mix[start:start + G_], 0, 1, G.PATH_AUTO)
            assert rc == 0
            for x in e:
                if ROUTES[x.route] == "EMU":
                    assert x.t_emu_s <= x.t_native_s
                if ROUTES[x.route] == "UNPROFITABLE":
                    assert x.t_emu_s > x.t_native_s
            start += 37 if G_ == 1 else G_


@pytest.mark.parametrize("who", sorted(PLANNERS))
def test_route_histograms_of_the_generated_group_match_the_log(who):
    plan = PLANNERS[who]
    ps = make_group(65535, 777)
    for path, want in LOG["routes"].items():
        rc, e = plan(ps, 0, 1, int(path))
        assert rc == 0
        hist = {}
        for x in e:
            hist[ROUTES[x.route]] = hist.get(ROUTES[x.route], 0) + 1
        assert hist == {k: v for k, v in want.items() if k != "G"}, path
        # determinism (tests/test_planner.cpp:367-400): a second plan gives the same entries
        rc2, e2 = plan(ps, 0, 1, int(path))
        assert rc2 == 0
        assert all((a.route, a.num_moduli, a.tile_cfg, a.t_emu_s, a.t_native_s) ==
                   (b.route, b.num_moduli, b.tile_cfg, b.t_emu_s, b.t_native_s) for a, b in zip(e, e2))


def test_library_and_oracle_agree_bitwise_on_the_generated_groups():
    for seed in (777, 999 + 17, 999 + 1000):
        ps = make_group(4000, seed)
        for path in (G.PATH_AUTO, G.PATH_EMU_GROUPED, G.PATH_EMU_LOOP):
            for fb in (0, 1):
                rl, el = plan_lib(ps, 0, fb, path)
                ro, eo = plan_oracle(ps, 0, fb, path)
                assert rl == ro
                if rl == 0:
                    for a, b in zip(el, eo):
                        assert (a.route, a.num_moduli, a.tile_cfg) == (b.route, b.num_moduli, b.tile_cfg)
                        assert np.float64(a.t_emu_s).view(np.int64) == np.float64(b.t_emu_s).view(np.int64)
                        assert np.float64(a.t_native_s).view(np.int64) == np.float64(b.t_native_s).view(np.int64)


def test_plan_allocates_nothing(tmp_path):
    """tests/test_planner.cpp:429-464: no heap allocation inside ggemm_plan (operator new and the C
    allocator interposed for the whole process), first call included."""
    exe = tmp_path / "count_allocs"
    lib_dir = REPO / "coding-basic-hw-2_amd" / "ggemm"
    subprocess.run(["g++", "-O1", "-std=c++17", "-D__HIP_PLATFORM_AMD__", f"-I{REPO / 'include'}",
                    "-I/opt/rocm/include", str(REPO / "tests" / "planner_alloc" / "count_allocs.cpp"), "-o", str(exe),
                    f"-L{lib_dir}", "-lggemm_mi355x", f"-Wl,-rpath,{lib_dir}", "-L/opt/rocm/lib", "-lamdhip64"],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    lines = [l for l in r.stdout.splitlines() if l.startswith("path=")]
    assert len(lines) == 2, r.stdout
    for l in lines:
        kv = dict(x.split("=") for x in l.split())
        assert kv["first"] == "0" and kv["steady"] == "0", l
