"""rocprofv3 analysis (coding-basic-hw-2_amd/analysis/rocprof_report.py) on synthetic CSV files.

The call split, busy / gap arithmetic, stage shares, roofline figures and the copy-calibrated HBM
traffic are checked against values worked out by hand for the synthetic timelines below."""
import csv
import importlib.util
from pathlib import Path

import pytest

TOOL = Path(__file__).resolve().parents[1] / "coding-basic-hw-2_amd" / "analysis" / "rocprof_report.py"

PREP = "ggemm::(anonymous namespace)::prep_kernel(oz2_problem const*, int, ggemm::CrtTables const*, unsigned long long*, int)"
I8 = "ggemm::(anonymous namespace)::i8_large_kernel(i8_problem const*, ggemm::I8Epi const*, int const*)"
RECON = "void ggemm::(anonymous namespace)::recon_kernel<true>(oz2_problem const*, ggemm::YDesc const*, int)"
DOTS = "ggemm::(anonymous namespace)::dots_kernel(oz2_problem const*, ggemm::YDesc const*, int, int)"
F64 = "ggemm::(anonymous namespace)::f64_grouped_kernel(ggemm::F64Problem const*, int const*)"
TORCH = "void at::native::vectorized_elementwise_kernel<4, at::native::FillFunctor<double> >(int)"
COPY = "__amd_rocclr_copyBuffer"


def _tool():
    spec = importlib.util.spec_from_file_location("rocprof_report", TOOL)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _trace(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kind", "Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        for name, s, e in rows:
            w.writerow(["KERNEL_DISPATCH", name, s, e])


def _counters(path, counter, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Counter_Name", "Counter_Value"])
        for name, v in rows:
            w.writerow([name, counter, v])


# times in ns: two emulated calls separated by a foreign kernel, two native-only calls, then an
# AUTO-like call whose native kernel follows its reconstruct (one call)
TIMELINE = [(PREP, 0, 100_000), (I8, 110_000, 300_000), (RECON, 300_000, 350_000),
            (TORCH, 360_000, 370_000),
            (PREP, 400_000, 500_000), (COPY, 500_000, 501_000), (I8, 500_000, 700_000), (RECON, 705_000, 765_000),
            (TORCH, 780_000, 790_000), (F64, 800_000, 850_000), (F64, 860_000, 900_000),
            (PREP, 1_000_000, 1_010_000), (I8, 1_010_000, 1_020_000), (RECON, 1_020_000, 1_030_000),
            (F64, 1_030_000, 1_040_000)]


def test_calls_busy_gap_and_stages(tmp_path):
    rr = _tool()
    p = tmp_path / "run_kernel_trace.csv"
    _trace(p, TIMELINE)
    calls = [rr.call_metrics(c) for c in rr.split_calls(rr.read_trace(p))]
    assert [c["kernels"] for c in calls] == [3, 3, 1, 1, 4]
    c1, c2, n1, n2, mixed = calls
    assert (c1["span_us"], c1["busy_us"], c1["gap_us"]) == pytest.approx((350.0, 340.0, 10.0))
    assert (c1["prep_us"], c1["i8_gemm_us"], c1["reconstruct_us"]) == pytest.approx((100.0, 190.0, 50.0))
    assert (c2["span_us"], c2["busy_us"], c2["gap_us"]) == pytest.approx((365.0, 360.0, 5.0))
    assert (n1["native_us"], n2["native_us"]) == pytest.approx((50.0, 40.0))
    assert (mixed["span_us"], mixed["native_us"], mixed["gap_us"]) == pytest.approx((40.0, 10.0, 0.0))
    assert rr.union_length([(0, 10), (5, 20), (30, 40)]) == 30


def test_kernel_names_and_stages():
    rr = _tool()
    assert [rr.short_name(n) for n in (PREP, I8, RECON)] == ["prep_kernel", "i8_large_kernel", "recon_kernel<true>"]
    assert [rr.stage_of(n) for n in (PREP, I8, RECON, DOTS, F64, COPY, TORCH)] == \
        ["prep", "i8_gemm", "reconstruct", "reconstruct", "native", "memops", None]


def test_roofline_and_traffic(tmp_path):
    rr = _tool()
    tr = tmp_path / "t.csv"
    _trace(tr, TIMELINE)
    fe, wr, cf, cw = (tmp_path / f for f in ("fe.csv", "wr.csv", "cf.csv", "cw.csv"))
    _counters(fe, "FETCH_SIZE", [(I8, 100.0), (I8, 300.0), (PREP, 50.0), (COPY, 1.0)])
    _counters(wr, "WRITE_SIZE", [(I8, 64.0), (PREP, 32.0)])
    _counters(cf, "FETCH_SIZE", [(COPY, 524288.0), (COPY, 8.0)])    # 1 GiB copy reads as half
    _counters(cw, "WRITE_SIZE", [(COPY, 1048576.0)])
    args = rr.argparse.Namespace(trace=str(tr), workload="2,64,32,100,3,0.5", fetch=str(fe), write=str(wr),
                                 copy_fetch=str(cf), copy_write=str(cw), copy_bytes=float(1 << 30),
                                 out=str(tmp_path / "r.md"), csv=str(tmp_path / "r.csv"))
    _, rows = rr.report(args)
    by = {r["kernel"]: r for r in rows}
    # G=2, m=64, n=32, k=100 (Kp=128), N=3: I = 2 * 4 * 2 * 64 * 32 * 128 ops per launch
    ops = 2 * 4 * 2 * 64 * 32 * 128
    avg_i8 = (190.0 + 200.0 + 10.0) / 3
    assert by["i8_large_kernel"]["achieved"] == pytest.approx(ops / (avg_i8 * 1e-6) / 1e12)
    assert by["i8_large_kernel"]["frac"] == pytest.approx(ops / (avg_i8 * 1e-6) / 5.0e15)
    prep = 2 * (8.0 * (64 * 100 + 100 * 32) + 4 * (64 + 32) * 128 + 16.0 * (64 + 32))
    assert by["prep_kernel"]["achieved"] == pytest.approx(prep / 70e-6 / 1e12)
    recon = 2 * ((3 + 4.0) * 64 * 32 + 16.0 * 64 * 32 + 16.0 * (64 + 32))
    assert by["recon_kernel<true>"]["achieved"] == pytest.approx(recon / 40e-6 / 1e12)
    # FETCH reads half the bytes (factor 0.5), WRITE all of them: mean 200 KiB -> 400 KiB read
    assert by["i8_large_kernel"]["hbm_read_gb"] == pytest.approx(400 * 1024 / 1e9)
    assert by["i8_large_kernel"]["hbm_write_gb"] == pytest.approx(64 * 1024 / 1e9)
    assert by["prep_kernel"]["hbm_read_gb"] == pytest.approx(100 * 1024 / 1e9)
    text = (tmp_path / "r.md").read_text()
    assert "Calls (median over 5)" in text


def test_traffic_json_record(tmp_path):
    """--traffic-json writes the INT8 GEMM's calibrated bytes per launch (the figure bench.py
    reports as roofline.traffic) under its key and keeps the other keys of the file."""
    rr = _tool()
    tr = tmp_path / "t.csv"
    _trace(tr, TIMELINE)
    fe, wr, cf, cw = (tmp_path / f for f in ("fe.csv", "wr.csv", "cf.csv", "cw.csv"))
    _counters(fe, "FETCH_SIZE", [(I8, 100.0), (I8, 300.0), (PREP, 50.0)])
    _counters(wr, "WRITE_SIZE", [(I8, 64.0), (PREP, 32.0)])
    _counters(cf, "FETCH_SIZE", [(COPY, 524288.0)])
    _counters(cw, "WRITE_SIZE", [(COPY, 1048576.0)])
    js = tmp_path / "hbm.json"
    js.write_text('{"large": {"traffic_bytes": 7}}')
    rr.main([str(tr), "--fetch", str(fe), "--write", str(wr), "--copy-fetch", str(cf), "--copy-write", str(cw),
             "-o", str(tmp_path / "r.md"), "--traffic-json", str(js), "--traffic-key", "uniform"])
    data = rr.json.loads(js.read_text())
    assert data["large"] == {"traffic_bytes": 7}
    rec = data["uniform"]
    assert rec["kernel"] == "i8_large_kernel"
    assert rec["fetch_kib"] == pytest.approx(200.0) and rec["write_kib"] == pytest.approx(64.0)
    assert rec["fetch_factor"] == pytest.approx(0.5) and rec["write_factor"] == pytest.approx(1.0)
    assert rec["traffic_bytes"] == round((400 + 64) * 1024)


def test_traffic_json_record_prep(tmp_path):
    """--traffic-stage prep records prep's bytes per launch instead (the roofline kernel of a call
    whose prep outlasts its INT8 GEMM), under the profiler's kernel name."""
    rr = _tool()
    tr = tmp_path / "t.csv"
    _trace(tr, TIMELINE)
    fe, wr, cf, cw = (tmp_path / f for f in ("fe.csv", "wr.csv", "cf.csv", "cw.csv"))
    _counters(fe, "FETCH_SIZE", [(I8, 100.0), (PREP, 50.0), (PREP, 70.0)])
    _counters(wr, "WRITE_SIZE", [(I8, 64.0), (PREP, 32.0)])
    _counters(cf, "FETCH_SIZE", [(COPY, 524288.0)])
    _counters(cw, "WRITE_SIZE", [(COPY, 1048576.0)])
    js = tmp_path / "hbm.json"
    rr.main([str(tr), "--fetch", str(fe), "--write", str(wr), "--copy-fetch", str(cf), "--copy-write", str(cw),
             "-o", str(tmp_path / "r.md"), "--traffic-json", str(js), "--traffic-key", "hard",
             "--traffic-stage", "prep"])
    rec = rr.json.loads(js.read_text())["hard"]
    assert rec["kernel"] == rr.short_name(PREP)
    assert rec["fetch_kib"] == pytest.approx(60.0) and rec["write_kib"] == pytest.approx(32.0)
    assert rec["traffic_bytes"] == round((120 + 32) * 1024)


def test_dot_pass_counts_in_reconstruct_without_roofline(tmp_path):
    """The flagged entries' FP64 dot products (dots_kernel) run after recon_kernel: their time is
    reconstruct time, but the stage's algorithmic bytes are credited to recon_kernel alone."""
    rr = _tool()
    tr = tmp_path / "t.csv"
    _trace(tr, [(PREP, 0, 100_000), (I8, 100_000, 300_000), (RECON, 300_000, 340_000), (DOTS, 340_000, 400_000)])
    calls = [rr.call_metrics(c) for c in rr.split_calls(rr.read_trace(tr))]
    assert [c["kernels"] for c in calls] == [4]
    assert calls[0]["reconstruct_us"] == pytest.approx(100.0)
    args = rr.argparse.Namespace(trace=str(tr), workload="2,64,32,100,3", fetch=None, write=None, copy_fetch=None,
                                 copy_write=None, copy_bytes=float(1 << 30), out=str(tmp_path / "r.md"), csv=None)
    _, rows = rr.report(args)
    by = {r["kernel"]: r for r in rows}
    recon = 2 * ((3 + 4.0) * 64 * 32 + 8.0 * 64 * 32 + 16.0 * (64 + 32))
    assert by["recon_kernel<true>"]["achieved"] == pytest.approx(recon / 40e-6 / 1e12)
    assert by["dots_kernel"]["stage"] == "reconstruct" and by["dots_kernel"]["achieved"] is None
