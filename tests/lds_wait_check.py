"""Checks a kernel's AMDGPU assembly for uses of VGPRs whose LDS load (ds_read*) may still be pending.

The INT8 GEMM issues its fragment reads as inline assembly and waits for them with an explicit
s_waitcnt, so the compiler cannot see the dependency: a register copy it placed between a read
and its wait would read stale data.  Dataflow over the control-flow graph: state = the pending
LDS-load destination register sets, oldest first; s_waitcnt lgkmcnt(N) keeps only the newest N
(LDS completes in order; scalar loads do not, so the N outstanding may all be LDS).  Any other
instruction that names a pending register is reported.
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
    succ = {}
    for bi, b in enumerate(order):
        s, fall = [], True
        for t in blocks[b]:
            op = t.split()[0]
            if op == "s_branch":
                s.append(t.split()[1])
                fall = False
            elif op.startswith("s_cbranch"):
                s.append(t.split()[1])
            elif op in ("s_endpgm", "s_setpc_b64"):
                fall = False
        if fall and bi + 1 < len(order):
            s.append(order[bi + 1])
        succ[b] = s
    return blocks, order, succ


def check_lines(src, want):
    """[(block, instruction, pending registers)] for the kernel whose symbol contains want."""
    start = next(i for i, ln in enumerate(src)
                 if not ln.startswith("\t") and re.match(r"^\S*" + re.escape(want) + r"\S*:", ln))
    end = next(i for i in range(start, len(src)) if "s_endpgm" in src[i])
    blocks, order, succ = _blocks(src[start + 1:end + 1])
    state_in = {b: None for b in order}
    state_in["__entry"] = []
    work, reports = ["__entry"], set()
    while work:
        b = work.pop()
        st = [set(x) for x in state_in[b]]
        for t in blocks[b]:
            op = t.split()[0]
            rest = t[len(op):]
            if op == "s_waitcnt":
                m = re.search(r"lgkmcnt\((\d+)\)", t)
                if m:
                    n = int(m.group(1))
                    st = [] if n == 0 else st[max(0, len(st) - n):]
                continue
            pend = set().union(*st) if st else set()
            if op.startswith("ds_read") or op.startswith("ds_load"):
                parts = rest.split(",")
                srcs = _regs(",".join(parts[1:]))
                if srcs & pend:
                    reports.add((b, t, tuple(sorted(srcs & pend))))
                st.append(_regs(parts[0]))
                continue
            used = _regs(rest)
            if used & pend:
                reports.add((b, t, tuple(sorted(used & pend))))
        for s2 in succ[b]:
            if s2 not in state_in:
                continue
            new = st if state_in[s2] is None else _merge(state_in[s2], st)
            if state_in[s2] is None or new != state_in[s2]:
                state_in[s2] = new
                work.append(s2)
    return sorted(reports)


def check(path, want):
    with open(path) as f:
        return check_lines(f.read().splitlines(), want)


if __name__ == "__main__":
    found = check(sys.argv[1], sys.argv[2])
    for b, t, r in found:
        print(f"{b}: {t}   pending {r[:8]}")
    print(f"{len(found)} uses of pending LDS destinations")
    sys.exit(1 if found else 0)
