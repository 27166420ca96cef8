"""ggemm_grouped_dgemm_noalloc (the allocation-free entry point) against ggemm_grouped_dgemm through a
handle: two calls in a row on the static workspace -- the second on a smaller group, so it runs on
scratch the first call left behind -- each bitwise equal to the handle call on the same problems with
equal stats and device counters; no call takes device memory of its own (free memory unchanged on
every call after the first; the first loads the code object holding the static
workspace); sizes beyond the limits and other paths are rejected."""
import ctypes as C
import os

import numpy as np
import pytest
import torch

os.environ["GGEMM_STATS_REPAIR"] = "1"   # read at handle creation and at the entry point's set-up

import ggemm as G
from gpu_util import say, same_bits
from test_gpu_grouped import Case

pytestmark = pytest.mark.gpu


def free_device_bytes():
    hip = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(0), C.c_size_t(0)
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def noalloc(path, cfg, case, mem=None):
    """One call of the entry point; mem (a list) receives the device bytes it took (free memory just
    before minus just after)."""
    st = G.Stats()
    case.reset_C()
    arr = G.problems_array(case.problems())
    torch.cuda.synchronize()
    before = free_device_bytes()
    rc = G.lib().ggemm_grouped_dgemm_noalloc(path, C.byref(cfg), arr, len(case.hp), None, C.byref(st))
    torch.cuda.synchronize()
    if mem is not None:
        mem.append(before - free_device_bytes())
    return rc, st, [case.C(g).copy() for g in range(len(case.hp))]


def with_handle(path, cfg, case):
    with G.Handle(len(case.hp), *case.sizes()) as h:
        case.reset_C()
        rc, st = h.dgemm(path, cfg, case.problems())
        torch.cuda.synchronize()
    return rc, st, [case.C(g).copy() for g in range(len(case.hp))]


def same_stats(a, b):
    keys = ["num_problems", "num_fallback", "kernel_launches", "moduli_min", "moduli_max", "num_repaired",
            "num_uncertified", "num_safety_fallback"]
    return {k: getattr(a, k) for k in keys} == {k: getattr(b, k) for k in keys}


def test_noalloc_matches_handle_two_calls_then_smaller():
    big = Case([(200, 150, 500), (96, 80, 160), (300, 1, 129), (64, 64, 33), (128, 256, 100), (130, 66, 512)],
               20261241, phi=2.0, beta=0.5)
    small = Case([(40, 33, 300), (17, 9, 64)], 20261242, phi=1.0, alpha=-1.5, beta=0.25)
    assert sum(h.m * h.k for h in big.hp) <= G.NOALLOC_MAX_ELEMS
    cfg_emu = G.Config(0, 1e-15, 0, G.REPAIR_COUNT)
    cfg_auto = G.Config(0, 1e-15, 1, G.REPAIR_ON)
    assert sum(h.k * h.n for h in big.hp) <= G.NOALLOC_MAX_ELEMS and sum(h.m * h.n for h in big.hp) <= G.NOALLOC_MAX_ELEMS
    # handle calls first load the library's other code objects (each source file is one, loaded on
    # first use: prep, INT8 GEMM, reconstruct, native FP64 GEMM, device state) on this device
    for path, cfg in ((G.PATH_EMU_GROUPED, cfg_emu), (G.PATH_AUTO, cfg_auto)):
        rc, _, _ = with_handle(path, cfg, small)
        assert rc == 0
    say("noalloc call 1: 6 problems, EMU_GROUPED, COUNT")
    mem = []
    rc, st1, out1 = noalloc(G.PATH_EMU_GROUPED, cfg_emu, big, mem)
    assert rc == 0, rc
    # the first call on a device loads the entry point's own code object, for which the loader places
    # the static workspace: at most the array plus the code object; later calls take nothing
    assert mem[0] <= G.NOALLOC_SCRATCH_BYTES + (8 << 20), mem[0]
    rc, sh1, ref1 = with_handle(G.PATH_EMU_GROUPED, cfg_emu, big)
    assert rc == 0
    for g, (a, b) in enumerate(zip(out1, ref1)):
        assert same_bits(a, b), f"call 1, problem {g} differs from the handle call"
    assert same_stats(st1, sh1), (st1.as_dict(), sh1.as_dict())
    assert st1.kernel_launches == 6 and st1.num_uncertified >= 0

    for path, cfg, tag in ((G.PATH_AUTO, cfg_auto, "AUTO, ON"), (G.PATH_EMU_GROUPED, cfg_emu, "EMU_GROUPED, COUNT")):
        say(f"noalloc call 2: 2 problems, {tag}")
        mem = []
        rc, st2, out2 = noalloc(path, cfg, small, mem)
        assert rc == 0, rc
        assert mem[0] == 0, f"the call took {mem[0]} bytes of device memory"
        rc, sh2, ref2 = with_handle(path, cfg, small)
        assert rc == 0
        for g, (a, b) in enumerate(zip(out2, ref2)):
            assert same_bits(a, b), f"call 2 ({tag}), problem {g} differs from the handle call"
        assert same_stats(st2, sh2), (st2.as_dict(), sh2.as_dict())


def test_noalloc_rejects_beyond_limits():
    cfg = G.Config(0, 1e-15, 1, G.REPAIR_ON)
    side = int(np.sqrt(G.NOALLOC_MAX_ELEMS)) + 16          # one square problem over every element budget
    big = Case([(side, side, side)], 5, phi=0.0)
    say("noalloc beyond the element budget")
    rc, _, _ = noalloc(G.PATH_EMU_GROUPED, cfg, big)
    assert rc == G.GGEMM_ERR_WORKSPACE
    many = Case([(8, 8, 8)] * (G.NOALLOC_MAX_PROBLEMS + 1), 6, phi=0.0)
    rc, _, _ = noalloc(G.PATH_EMU_GROUPED, cfg, many)
    assert rc == G.GGEMM_ERR_INVALID
    ok = Case([(8, 8, 8)] * 2, 7, phi=0.0)
    for path in (G.PATH_NATIVE_LOOP, G.PATH_NATIVE_GROUPED, G.PATH_EMU_LOOP, G.PATH_EMU_GROUPED_REUSE,
                 G.PATH_EMU_LOOP_BATCHED):
        rc, _, _ = noalloc(path, cfg, ok)
        assert rc == G.GGEMM_ERR_INVALID, path
    rc, st, _ = noalloc(G.PATH_EMU_GROUPED, cfg, ok)   # still usable after the rejections
    assert rc == 0 and st.kernel_launches == 6


def test_noalloc_refuses_a_capturing_stream():
    """The entry point synchronises its stream, so it cannot be captured: on a stream under capture it
    returns GGEMM_ERR_INVALID without touching the capture, which then ends normally (an empty graph);
    the same stream then runs the call and matches a handle call bit for bit."""
    hip = C.CDLL("libamdhip64.so")
    case = Case([(64, 48, 100), (37, 29, 257)], 20261243, phi=1.0, beta=0.5)
    cfg = G.Config(0, 1e-15, 1, G.REPAIR_ON)
    stream = C.c_void_p()
    assert hip.hipStreamCreate(C.byref(stream)) == 0
    try:
        say("noalloc under stream capture (global mode)")
        case.reset_C()
        arr = G.problems_array(case.problems())
        torch.cuda.synchronize()
        assert hip.hipStreamBeginCapture(stream, 0) == 0
        st = G.Stats()
        rc = G.lib().ggemm_grouped_dgemm_noalloc(G.PATH_AUTO, C.byref(cfg), arr, len(case.hp), stream, C.byref(st))
        graph = C.c_void_p()
        end = hip.hipStreamEndCapture(stream, C.byref(graph))
        assert rc == G.GGEMM_ERR_INVALID, rc
        assert end == 0 and graph.value, end
        assert hip.hipGraphDestroy(graph) == 0
        rc = G.lib().ggemm_grouped_dgemm_noalloc(G.PATH_AUTO, C.byref(cfg), arr, len(case.hp), stream, C.byref(st))
        assert rc == 0, rc
        assert hip.hipStreamSynchronize(stream) == 0
        out = [case.C(g).copy() for g in range(len(case.hp))]
        rc, sh, ref = with_handle(G.PATH_AUTO, cfg, case)
        assert rc == 0
        for g, (a, b) in enumerate(zip(out, ref)):
            assert same_bits(a, b), f"problem {g} differs from the handle call"
        assert same_stats(st, sh), (st.as_dict(), sh.as_dict())
    finally:
        hip.hipStreamDestroy(stream)
