"""Transcribe the outcomes the reference's planner unit test printed into a fixture.

Source (read as text, in this container only):
  results/planner_unit_590223/test_planner.log  -- output of tests/test_planner.cpp (the host-only
  planner test) with the device model of tests/testdata/planner/valid.json and 132 SMs.

Writes tests/golden/planner_unit_log.json with
  * "tiles":   4000 copies of (m, n, 4096), AUTO without fallback -> chosen tile edge (log :12-19,
               printed by tests/test_planner.cpp:294-296),
  * "shrink":  (m, n, k, G) -> N, tiles at 128, chosen tile edge (log :20-23, test :310-312),
  * "reeval":  (m, m, 8192) alone and in a group of 4000, AUTO with fallback -> tile edge, route and
               t_emu to the printed 3 significant digits (log :24-27, test :349-350),
  * "routes":  per path the route histogram of the 65535-problem group make_group(65535, 777) with
               fallback allowed (log :30-33, test :466-471).
Run: python tests/golden/extract_planner_log.py [path/to/log]
"""
import json
import re
import sys
from pathlib import Path

LOG = Path("/root/reference/results/planner_unit_590223/test_planner.log")


def main():
    log = Path(sys.argv[1]) if len(sys.argv) > 1 else LOG
    out = {"source": "results/planner_unit_590223/test_planner.log", "model": None,
           "tiles": [], "shrink": [], "reeval": [], "routes": {}, "passed": None}
    path = None
    for ln in log.read_text().splitlines():
        m = re.match(r"^model: num_sms=(\d+) fp64=([\d.e+]+) i8=([\d.e+]+) bw=([\d.e+]+) tiny_mnk=(\d+)", ln)
        if m:
            out["model"] = {"num_sms": int(m.group(1)), "fp64": float(m.group(2)), "i8": float(m.group(3)),
                            "bw": float(m.group(4)), "tiny_mnk": float(m.group(5))}
        m = re.match(r"^\s+(\d+)x(\d+)\s+x(\d+) -> tile (\d+) \(pad eff ([\d.]+), best ([\d.]+)\)", ln)
        if m:
            out["tiles"].append({"m": int(m.group(1)), "n": int(m.group(2)), "G": int(m.group(3)),
                                 "tile": int(m.group(4)), "pad_eff": m.group(5), "best": m.group(6)})
        m = re.match(r"^\s+shrink (\d+)x(\d+)x(\d+) G=(\d+) N=(\d+): 128-tiles=(\d+) \(2\*SM=(\d+)\) -> tile (\d+)", ln)
        if m:
            v = [int(m.group(q)) for q in range(1, 9)]
            out["shrink"].append(dict(zip(["m", "n", "k", "G", "N", "tiles128", "slots", "tile"], v)))
        m = re.match(r"^\s+re-eval (\d+)\^2x(\d+): alone tile (\d+) (\w+) t_emu ([\d.e+-]+) \| "
                     r"group tile (\d+) (\w+) t_emu ([\d.e+-]+)", ln)
        if m:
            out["reeval"].append({"m": int(m.group(1)), "k": int(m.group(2)),
                                  "alone": [int(m.group(3)), m.group(4), m.group(5)],
                                  "group": [int(m.group(6)), m.group(7), m.group(8)]})
        m = re.match(r"^\s+G=(\d+) path=(\d+): plan host time", ln)
        if m:
            path = m.group(2)
            out["routes"][path] = {"G": int(m.group(1))}
        m = re.match(r"^\s+routes:(.*)$", ln)
        if m and path is not None:
            for kv in m.group(1).split():
                k, v = kv.split("=")
                out["routes"][path][k] = int(v)
        m = re.match(r"^test_planner: (\d+) passed, (\d+) failed", ln)
        if m:
            out["passed"] = [int(m.group(1)), int(m.group(2))]
    dst = Path(__file__).with_name("planner_unit_log.json")
    dst.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {dst}: {len(out['tiles'])} tile, {len(out['shrink'])} shrink, {len(out['reeval'])} re-eval cases, "
          f"routes for paths {sorted(out['routes'])}")


if __name__ == "__main__":
    main()
