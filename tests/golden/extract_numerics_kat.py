"""Transcribe the known-answer values of the reference's numerics test log into a fixture.

Source (read as text, in this container only):
  results/final_590258/logs/test_numerics_standalone.log  -- output of
  tests/test_numerics_standalone.cu on an H200.

Writes tests/golden/numerics_kat.json with
  * "log2P", "bound_k1024": per N = 8..20 (log lines 4-16),
  * "choose_1e15": oz2_choose_num_moduli(k, 1e-15) for six k (log line 17),
  * "sweep": per (m, n, k, phi) the naive-FP64 rel_cw of the generated data and, per N,
    the repaired-entry count "rep" and the printed error columns "cols" = [rel_cw, rel_abs,
    rel_nrm, bound, gate] (log lines 23-340),
  * "grouped_repaired" and "grouped": the 9-problem launch's repair total and, per problem,
    (m, n, k, N) with the same five columns (log lines 343-353),
  * "nonfinite_counter", "nonfinite_gate": section 4 (log line 355),
  * "repair_modes": section 5's counts, OFF == COUNT flag and the OFF / COUNT / ON gates (log line 357).
Run: python tests/golden/extract_numerics_kat.py [path/to/log]
"""
import json
import re
import sys
from pathlib import Path

LOG = Path("/root/reference/results/final_590258/logs/test_numerics_standalone.log")


def main():
    log = Path(sys.argv[1]) if len(sys.argv) > 1 else LOG
    lines = log.read_text().splitlines()
    out = {"source": "results/final_590258/logs/test_numerics_standalone.log",
           "log2P": {}, "bound_k1024": {}, "choose_1e15": {}, "sweep": []}
    cur = None
    for ln in lines:
        m = re.match(r"^\s*(\d+)\s+([\d.]+)\s+([\d.e+-]+)\s*$", ln)
        if m and cur is None:
            out["log2P"][m.group(1)] = float(m.group(2))
            out["bound_k1024"][m.group(1)] = float(m.group(3))
            continue
        m = re.match(r"^choose\(1e-15\): (.*)$", ln)
        if m:
            for kv in m.group(1).split():
                k, v = kv.split(":")
                out["choose_1e15"][k.replace("k=", "")] = int(v)
            continue
        m = re.match(r"^shape m=(\d+) n=(\d+) k=(\d+) phi=([\d.]+)\s+\(naive FP64 dot rel_cw=([\d.e+-]+)\)", ln)
        if m:
            cur = {"m": int(m.group(1)), "n": int(m.group(2)), "k": int(m.group(3)),
                   "phi": float(m.group(4)), "naive_rel_cw": float(m.group(5)), "rep": {}}
            out["sweep"].append(cur)
            continue
        m = re.match(r"^\s*(\d+)\s+([\d.e+-]+)\s+([\d.e+-]+)\s+([\d.e+-]+)\s+([\d.e+-]+)\s+([\d.e+-]+)\s+(\d+)\s+ok", ln)
        if m and cur is not None:
            cur["rep"][m.group(1)] = int(m.group(7))
            cur.setdefault("cols", {})[m.group(1)] = [float(m.group(q)) for q in range(2, 7)]
            continue
        m = re.match(r"^\s*(\d+)\s+(\d+)\s+(\d+)\s+(\d+)\s+([\d.e+-]+)\s+([\d.e+-]+)\s+([\d.e+-]+)\s+"
                     r"([\d.e+-]+)\s+([\d.e+-]+)\s+ok$", ln)
        if m and "grouped_repaired" in out:
            out.setdefault("grouped", []).append({"mnkN": [int(m.group(q)) for q in range(1, 5)],
                                                  "cols": [float(m.group(q)) for q in range(5, 10)]})
            continue
        m = re.match(r"^grouped launch .* total repaired entries=(\d+)", ln)
        if m:
            out["grouped_repaired"] = int(m.group(1))
        m = re.match(r"^non-finite: counter=(\d+) .* gate\(rest\)=([\d.e+-]+)", ln)
        if m:
            out["nonfinite_counter"] = int(m.group(1))
            out["nonfinite_gate"] = float(m.group(2))
        m = re.match(r"^repair modes .* OFF gate=([\d.e+-]+) \| COUNT gate=([\d.e+-]+) uncertified=(\d+) \| "
                     r"ON gate=([\d.e+-]+) repaired=(\d+) \| OFF==COUNT bitwise:(\d)", ln)
        if m:
            out["repair_modes"] = {"uncertified": int(m.group(3)), "repaired": int(m.group(5)),
                                   "off_eq_count": int(m.group(6)),
                                   "gates": [float(m.group(1)), float(m.group(2)), float(m.group(4))]}
    dst = Path(__file__).with_name("numerics_kat.json")
    dst.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {dst}: {len(out['sweep'])} sweep cases")


if __name__ == "__main__":
    main()
