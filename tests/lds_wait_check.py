"""Checks a kernel's AMDGPU assembly for uses of VGPRs whose LDS load (ds_read*) or vector-memory
load (global_ / buffer_ / flat_ / scratch_ loads, returning atomics) may still be pending.

The INT8 GEMM issues its fragment reads, and the shift loads of its tile check, as inline assembly
and waits for them with an explicit s_waitcnt, so the compiler cannot see the dependency: a
register copy it placed between a load and its wait would read stale data.  Dataflow over the
control-flow graph: state = the pending LDS-load destination register sets and the pending
vector-memory operations (their destination sets, empty for stores and LDS DMA), oldest first;
s_waitcnt lgkmcnt(N) keeps only the newest N LDS entries (LDS completes in order; scalar loads do
not, so the N outstanding may all be LDS), vmcnt(N) the newest N vector-memory entries (they
complete in order).  Any other instruction that names a pending register is reported.
Usage: python3 lds_wait_check.py file.s kernel_symbol_substring   (exit status 1 on a finding)
"""
import re
import sys


def _regs(text):
    out = set()
    for m in re.finditer(r"\bv\[(\d+):(\d+)\]", text):
        out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    for m in re.finditer(r"\bv(\d+)\b", text):
        out.add(int(m.group(1)))
    return out


def _merge(a, b):
    n = max(len(a), len(b))
    a = [set()] * (n - len(a)) + a
    b = [set()] * (n - len(b)) + b
    return [x | y for x, y in zip(a, b)]


def _blocks(lines):
    """Instructions per branch-target label (blocks labelled only by a comment stay merged into the
    preceding one: their branches are followed where they stand)."""
    blocks, order, cur = {"__entry": []}, ["__entry"], "__entry"
    for ln in lines:
        m = re.match(r"^(\.LBB\w+|\S+):", ln)
        if m and not ln.startswith("\t"):
            cur = m.group(1)
            blocks[cur] = []
            order.append(cur)
            continue
        t = ln.split(";")[0].strip()
        if t and not t.startswith("."):
            blocks[cur].append(t)
    return blocks, order


def _vmem(op, t):
    """(is a vector-memory operation, its destination text or None)."""
    if not op.startswith(("global_", "buffer_", "flat_", "scratch_")):
        return False, None
    parts = t[len(op):].split(",")
    if "_load" in op and "_lds" not in op:
        return True, parts[0]
    if "_atomic" in op and re.search(r"\b(sc0|glc)\b", t):   # returns the old value
        return True, parts[0]
    return True, None


# counter widths on gfx9: at most this many operations outstanding, so older entries have completed
# (the cap also bounds the dataflow state in loops that never drain)
kVmMax, kLgkmMax = 63, 15


def _keep(st, n):
    return [] if n == 0 else st[max(0, len(st) - n):]


def check_lines(src, want):
    """[(block, instruction, pending registers)] for the kernel whose symbol contains want."""
    start = next(i for i, ln in enumerate(src)
                 if not ln.startswith("\t") and re.match(r"^\S*" + re.escape(want) + r"\S*:", ln))
    end = next(i for i in range(start, len(src)) if "s_endpgm" in src[i])
    blocks, order = _blocks(src[start + 1:end + 1])
    state_in = {b: None for b in order}
    state_in["__entry"] = ([], [])
    work, reports = ["__entry"], set()

    def flow(target, lg, vm):   # the state reaching target along one edge
        if target not in state_in:
            return
        old = state_in[target]
        new = (lg, vm) if old is None else (_merge(old[0], lg), _merge(old[1], vm))
        if old is None or new != old:
            state_in[target] = new
            work.append(target)

    while work:
        b = work.pop()
        lg = [set(x) for x in state_in[b][0]]
        vm = [set(x) for x in state_in[b][1]]
        live = True
        for t in blocks[b]:
            op = t.split()[0]
            rest = t[len(op):]
            if op == "s_waitcnt":
                m = re.search(r"lgkmcnt\((\d+)\)", t)
                if m:
                    lg = _keep(lg, int(m.group(1)))
                m = re.search(r"vmcnt\((\d+)\)", t)
                if m:
                    vm = _keep(vm, int(m.group(1)))
                continue
            if op.startswith("s_cbranch"):
                flow(t.split()[1], lg, vm)
                continue
            if op == "s_branch":
                flow(t.split()[1], lg, vm)
                live = False
                break
            if op in ("s_endpgm", "s_setpc_b64"):
                live = False
                break
            pend = set().union(*lg, *vm)
            if op.startswith("ds_read") or op.startswith("ds_load"):
                parts = rest.split(",")
                srcs = _regs(",".join(parts[1:]))
                if srcs & pend:
                    reports.add((b, t, tuple(sorted(srcs & pend))))
                lg = _keep(lg + [_regs(parts[0])], kLgkmMax)
                continue
            is_vm, dst = _vmem(op, t)
            if is_vm:
                parts = rest.split(",")
                srcs = _regs(",".join(parts[1:]) if dst is not None else rest)
                if srcs & pend:
                    reports.add((b, t, tuple(sorted(srcs & pend))))
                vm = _keep(vm + [_regs(dst) if dst is not None else set()], kVmMax)
                continue
            used = _regs(rest)
            if used & pend:
                reports.add((b, t, tuple(sorted(used & pend))))
        bi = order.index(b)
        if live and bi + 1 < len(order):
            flow(order[bi + 1], lg, vm)
    return sorted(reports)


def check(path, want):
    with open(path) as f:
        return check_lines(f.read().splitlines(), want)


if __name__ == "__main__":
    found = check(sys.argv[1], sys.argv[2])
    for b, t, r in found:
        print(f"{b}: {t}   pending {r[:8]}")
    print(f"{len(found)} uses of pending load destinations")
    sys.exit(1 if found else 0)
