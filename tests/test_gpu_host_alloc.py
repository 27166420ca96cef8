"""No host heap allocation inside the library's calls (the reference's contracts: no operator new
inside ggemm_plan, tests/test_planner.cpp:429-464; no growth of the INT8 schedule builder's host
scratch after a reserve, tests/test_i8_grouped.cu:348-352).

tests/planner_alloc/count_allocs (built by __graft_entry__.build()) interposes operator new and the
C allocator for its whole process and counts the allocations whose caller lies in the library's
code (the HIP runtime's own command objects are not the library's), over a mixed group -- emulated
problems and k = 0, alpha = 0 and k <= 16 problems on native routes -- through ggemm_grouped_dgemm on
every path, ggemm_execute_plan, ggemm_plan_update_pointers + ggemm_execute_plan, ggemm_plan_get_stats
and ggemm_grouped_dgemm_noalloc.  Handle and plan calls allocate nothing from their first call on
(the handle reserves everything at creation); the allocation-free entry point sizes its host
scratch once, on its first call, and allocates nothing after it."""
import subprocess
from pathlib import Path

import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu

REPO = Path(__file__).resolve().parents[1]
EXE = REPO / "tests" / "planner_alloc" / "count_allocs"


def test_calls_allocate_no_host_memory():
    assert EXE.exists(), f"{EXE} missing: run __graft_entry__.build() first"
    say("count_allocs gpu: every path, plan execute / update, noalloc")
    r = subprocess.run([str(EXE), "gpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("call=")]
    kinds = {}
    for ln in lines:
        kv = dict(x.split("=") for x in ln.split())
        name = kv.pop("call")
        kinds[name] = {k: int(v) for k, v in kv.items()}
    say(kinds)
    assert set(kinds) == {"native_loop", "native_grouped", "emu_loop", "emu_grouped", "auto", "emu_grouped_reuse",
                          "emu_loop_batched", "execute_plan", "update_pointers_execute", "plan_get_stats", "noalloc"}
    for name, c in kinds.items():
        assert c["steady"] == 0, (name, c)
        if name != "noalloc":
            assert c["first"] == 0, (name, c)
