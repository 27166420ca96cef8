"""Calibration fit (coding-basic-hw-2_amd/calib/calib.py, the flow of bench/calib/fit.py) on the CPU.

Rows made from a known timing model t = t0 + work / peak must give back that peak, the launch
median and the copy bandwidth; the crossover table must follow the cost model it documents
(emulation wins from some size on for small N, never below it).  The shipped params file must
hold every key the planner reads, in the planner's accepted ranges."""
import importlib.util
import json
from pathlib import Path

import pytest

CALIB = Path(__file__).resolve().parents[1] / "coding-basic-hw-2_amd" / "calib"


def _calib():
    spec = importlib.util.spec_from_file_location("ggemm_calib", CALIB / "calib.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _rows(f64_peak, i8_peak, planes=16, t0=40e-6):
    rows = []

    def row(kind, param, d, nbytes, t_us, value):
        rows.append({"kind": kind, "param": param, "m": d, "n": d, "k": d, "bytes": nbytes, "iters": 1,
                     "time_us": t_us, "value": value, "unit": ""})
    for t in (4.1, 3.9, 4.0):
        row("launch_stream", "", 0, 0, t, 0.0)
        row("launch_sync", "", 0, 0, 15.0, 0.0)
    for sz in (1 << 12, 1 << 20, 1 << 26):
        row("h2d_pinned", "", 0, sz, (10e-6 + sz / 50e9) * 1e6, 0.0)
    row("bw_copy", "", 0, 16 << 27, 0.0, 5000.0)
    row("bw_read", "", 0, 8 << 27, 0.0, 6000.0)
    for d in (256, 512, 1024, 2048, 4096, 8192):
        w = 2.0 * d ** 3
        t = t0 + w / f64_peak
        row("dgemm", "", d, 0, t * 1e6, w / t / 1e9)
        w8 = planes * 2.0 * d * d * ((d + 31) // 32 * 32)
        t8 = t0 + w8 / i8_peak
        row("i8gemm", f"planes={planes}", d, 0, t8 * 1e6, w8 / t8 / 1e9)
    return rows


def test_fit_recovers_model():
    cal = _calib()
    meta = {"gpu": "gfx950", "sm_count": 256, "cc": "9.5", "name": "test"}
    out = cal.fit(meta, _rows(5.0e13, 2.0e15))
    assert out["f64_peak_flops"] == pytest.approx(5.0e13, rel=1e-9)
    assert out["i8_peak_ops"] == pytest.approx(2.0e15, rel=1e-9)
    assert out["extra"]["f64_t0_s"] == pytest.approx(40e-6, rel=1e-6)
    assert out["t_launch_s"] == pytest.approx(4.0e-6)
    assert out["bw_Bps"] == 5.0e12
    assert out["extra"]["h2d_pinned_latency_s"] == pytest.approx(10e-6, rel=1e-6)
    assert out["extra"]["h2d_pinned_Bps"] == pytest.approx(50e9, rel=1e-6)
    # the best measured rate sits below the asymptotic one (t0 > 0)
    assert out["extra"]["f64_peak_flops_max"] < out["f64_peak_flops"]
    cross = out["crossover_square_pow2_by_N"]
    ds = [cross[str(N)] for N in range(6, 21)]
    # more moduli never make the emulation win earlier
    assert all(a is None or b is None or a <= b for a, b in zip(ds, ds[1:]))
    # INT8 / FP64 = 40: emulation with N = 6 wins at large sizes, N = 20 x 2mnk can still win
    assert cross["6"] is not None


def test_linfit_exact_line():
    cal = _calib()
    a, b = cal.linfit([1.0, 2.0, 4.0], [3.0, 5.0, 9.0])
    assert (a, b) == pytest.approx((1.0, 2.0))
    assert cal.linfit([2.0, 2.0], [1.0, 3.0]) == (2.0, 0.0)


def test_shipped_params_are_in_planner_ranges():
    p = json.loads((CALIB / "params_gfx950.json").read_text())
    assert p["gpu"] == "gfx950" and p["schema"] == "ggemm-calib-v1"
    # accepted ranges of src/planner.cpp:23-25: fp64 [1e11, 1e16], i8 [1e12, 1e17], bw [1e10, 1e14]
    assert 1e11 <= p["f64_peak_flops"] <= 1e16
    assert 1e12 <= p["i8_peak_ops"] <= 1e17
    assert 1e10 <= p["bw_Bps"] <= 1e14
