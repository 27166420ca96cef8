"""Pins the CPU oracle before anything is checked against it (no GPU).

Each check is chosen so that a plausible mistake in the restatement (a dropped term, a wrong
index or reduction order, a transposed operand) fails it:
  * CRT tables: exact big-integer identities and the logged log2P / bound / choose KATs;
  * prep: the exact residue identity of the reference's residue check, the norm budget, the
    maximality of the shift, and the reference's logged per-case repair counts (which move
    with any change in a shift or a float-rounded norm bound);
  * int GEMM: numpy int64 product and the closed form at the int32 edge;
  * reconstruct: the logged repair / uncertified / non-finite KATs and the gamma_n gate;
  * planner: the reference planner unit test's route table.
"""
import ctypes as C
import json
import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle_lib import (REPAIR_COUNT, REPAIR_OFF, REPAIR_ON, SHIFT_NONFINITE, SHIFT_ZERO, DeviceModel,
                        HostProb, PlanEntry, Shape, katgen, kp_of, oracle, oracle_i8_gemm, oracle_prep,
                        tables)

GOLDEN = Path(__file__).resolve().parent / "golden"
KAT = json.loads((GOLDEN / "numerics_kat.json").read_text())
MODULI = [256, 255, 253, 251, 247, 239, 233, 229, 227, 223, 217, 211, 199, 197, 193, 191, 181, 179, 173, 167]


# ------------------------------------------------------------------------------ CRT tables
REFERENCE = Path("/root/reference")
REF_LIB = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "libref_moduli.so"


@pytest.mark.skipif(not (REFERENCE / "src" / "moduli.h").exists() and not REF_LIB.exists(),
                    reason="the reference checkout (and so its table builder) is not on this host")
def test_crt_tables_byte_identical_to_reference_build():
    """The reference's own table builder (src/moduli.h:124-181, compiled unmodified by
    `make -C oracle ref` into oracle/_ref/) and the oracle's restatement produce the same table,
    byte for byte: moduli, Barrett magics, 2^e mod p, s1 / s2 splits, CRT inverses, P1, P2, u1 / P,
    log2 u1, T_N and log2 P for every N (the ulp-level P2, inv_Pu and T_N included)."""
    import subprocess
    if (REFERENCE / "src" / "moduli.h").exists():
        subprocess.run(["make", "-s", "-C", str(REF_LIB.parents[1]), "ref"], check=True)
    ref = C.CDLL(str(REF_LIB))
    ref.ref_crt_tables_size.restype = C.c_size_t
    ref.ref_build_crt_tables.argtypes = [C.c_void_p, C.c_size_t]
    size = ref.ref_crt_tables_size()
    t = tables()
    assert size == C.sizeof(t) == 10368
    buf = C.create_string_buffer(size)
    assert ref.ref_build_crt_tables(buf, size) == 0
    ours = C.string_at(C.addressof(t), size)
    assert buf.raw == ours, [i for i in range(size) if buf.raw[i] != ours[i]][:16]


def test_crt_tables_exact_identities():
    t = tables()
    for a in range(20):
        for b in range(a + 1, 20):
            assert math.gcd(MODULI[a], MODULI[b]) == 1
    for l, p in enumerate(MODULI):
        assert t.p[l] == p
        assert t.magic[l] == (1 << 32) // p
        assert [t.pow2[l][e] for e in range(128)] == [pow(2, e, p) for e in range(128)]
    for N in range(1, 21):
        P = math.prod(MODULI[:N])
        sh = t.log2_u1[N]
        for l in range(N):
            M = P // MODULI[l]
            assert (M * t.qinv[N][l]) % MODULI[l] == 1 % MODULI[l]
            assert M.bit_length() - 49 <= sh
            # M_l / u1 = s1 + s2 2^-18 within 2^-19
            approx = Fraction(t.s1[N][l]) + Fraction(t.s2[N][l], 1 << 18)
            exact = Fraction(M, 1) / Fraction(2) ** sh
            assert abs(approx - exact) <= Fraction(1, 1 << 19)
            assert t.s1[N][l] < (1 << 49)
        assert max((P // p).bit_length() for p in MODULI[:N]) - 49 == sh
        assert t.P1[N] == (P >> sh if sh >= 0 else P << -sh)
        # P2 = frac(P / u1) to double accuracy
        frac = Fraction(P % (1 << sh), 1 << sh) if sh > 0 else Fraction(0)
        assert abs(Fraction(t.P2[N]) - frac) <= Fraction(1, 1 << 52)
        # T_N = sqrt(P/2 (1-2^-20)) (1-2^-40), and T_N^2 < P/2 strictly
        T = t.T[N]
        assert Fraction(T) ** 2 < Fraction(P, 2)
        assert abs(T / math.sqrt(P * 0.5 * (1 - 2 ** -20)) - 1) < 2 ** -38


def test_crt_logged_kats():
    t = tables()
    for N in range(8, 21):
        assert f"{t.log2P[N]:.2f}" == f"{KAT['log2P'][str(N)]:.2f}"
        assert f"{oracle().oz2o_error_bound(1024, N):.3e}" == f"{KAT['bound_k1024'][str(N)]:.3e}"
    for k, want in KAT["choose_1e15"].items():
        assert oracle().oz2o_choose_num_moduli(int(k), 1e-15) == want


def test_choose_num_moduli_boundaries():
    # exhaustive-scan boundaries of the a-priori rule: choose(k,1e-15) = 14 for k < 30,
    # 15 for 30 <= k < 5647, 16 for k >= 5647; choose_cw(k,16) = 16 / 15 / 14 at 15 | 2246
    ch = oracle().oz2o_choose_num_moduli
    cw = oracle().oz2o_choose_num_moduli_cw
    assert (ch(29, 1e-15), ch(30, 1e-15), ch(5646, 1e-15), ch(5647, 1e-15)) == (14, 15, 15, 16)
    assert ch(131040, 1e-15) == 16 and ch(131041, 1e-15) == -1
    assert (cw(15, 16.0), cw(16, 16.0), cw(2245, 16.0), cw(2246, 16.0)) == (16, 15, 15, 14)
    # monotone in k
    prev = 0
    for k in list(range(1, 200)) + [1000, 4096, 16384, 65536, 131040]:
        n = ch(k, 1e-15)
        assert n >= prev
        prev = n


# ------------------------------------------------------------------------------------ prep
def _sym(x, p):
    r = x % p
    return r - p if r > (p - 1) // 2 else r


def _exact_scaled(a, s):
    """trunc(a * 2^s) as an exact Python int (Fraction arithmetic, no float rounding)."""
    f = Fraction(a) * (Fraction(2) ** s)
    return int(f)  # int() truncates toward zero


@pytest.mark.parametrize("N", [1, 8, 13, 20])
def test_prep_residue_identity(N):
    """tests/test_numerics_standalone.cu:210-258: residues equal sym(trunc(a 2^s) mod p), abs plane
    trunc(|a| 2^sigma) in [0,127], ||A'_i|| <= T_N, and the shift is maximal."""
    rng = np.random.default_rng(100 + N)
    m, n, k = 13, 11, 70
    lda, ldb = m + 2, k + 1
    A = np.zeros(lda * k)
    B = np.zeros(ldb * n)
    for c in range(k):
        A[c * lda: c * lda + m] = (rng.random(m) - 0.5) * np.exp(2.0 * rng.standard_normal(m))
    for c in range(n):
        B[c * ldb: c * ldb + k] = (rng.random(k) - 0.5) * np.exp(2.0 * rng.standard_normal(k))
    A[3 + 5 * lda] = 0.0
    for c in range(k):            # one all-zero row and one tiny-magnitude row (rescale path)
        A[7 + c * lda] = 0.0
        A[9 + c * lda] *= 2.0 ** -600
    A8, B8, rws, cws, nf = oracle_prep(m, n, k, N, A, lda, B, ldb)
    assert nf == 0
    T = Fraction(tables().T[N])
    kp = kp_of(k)
    for which, (vecs, get, P8, ws) in enumerate([
            (m, lambda i, q: A[i + q * lda], A8, rws), (n, lambda j, q: B[q + j * ldb], B8, cws)]):
        for v in range(vecs):
            s, sg = int(ws[v]), int(ws[vecs + v])
            vals = [get(v, q) for q in range(k)]
            if all(x == 0.0 for x in vals):
                assert s == 0 and sg == SHIFT_ZERO
            else:
                assert sg == 6 - math.frexp(max(abs(x) for x in vals))[1] + 1
            n2 = Fraction(0)
            for q in range(kp):
                x = _exact_scaled(vals[q], s) if q < k else 0
                n2 += x * x
                for l in range(N):
                    assert int(P8[l * vecs * kp + v * kp + q]) == _sym(x, MODULI[l])
                av = 0 if (q >= k or sg == SHIFT_ZERO) else int(Fraction(abs(vals[q])) * Fraction(2) ** sg)
                assert 0 <= av <= 127
                assert int(P8[N * vecs * kp + v * kp + q]) == av
            assert n2 <= T * T
            if any(vals):
                # maximality: one more bit would exceed the budget (up to the 2^-30 margin)
                n2s = sum(Fraction(x) ** 2 for x in vals) * Fraction(4) ** (s + 1)
                assert n2s * (1 + Fraction(1, 1 << 30)) > T * T
            # norm upper bounds are float round-ups of the exact norms
            dnorm2 = sum((Fraction(x) * Fraction(2) ** s - _exact_scaled(x, s)) ** 2 for x in vals)
            da = np.array([ws[2 * vecs + v]], dtype=np.int32).view(np.float32)[0]
            na = np.array([ws[3 * vecs + v]], dtype=np.int32).view(np.float32)[0]
            assert Fraction(float(da)) ** 2 >= dnorm2
            assert Fraction(float(na)) ** 2 >= n2
            assert float(na) <= math.sqrt(float(n2)) * (1 + 2 ** -22) + 1e-30


def test_prep_nonfinite_marks_vector():
    m, n, k, N = 4, 3, 40, 15
    A = np.ones(m * k)
    B = np.ones(k * n)
    A[2 + 7 * m] = np.nan
    B[5 + 1 * k] = -np.inf
    A8, B8, rws, cws, nf = oracle_prep(m, n, k, N, A, m, B, k)
    assert nf == 2
    assert rws[2] == SHIFT_NONFINITE and cws[1] == SHIFT_NONFINITE
    kp = kp_of(k)
    assert not A8.reshape(N + 1, m, kp)[:, 2, :].any()


# -------------------------------------------------------------------------------- int GEMM
def test_i8_gemm_matches_int64_matmul():
    rng = np.random.default_rng(7)
    for (m, n, kp) in [(1, 1, 32), (17, 9, 96), (33, 40, 1024)]:
        A8 = rng.integers(-128, 128, size=m * kp, dtype=np.int8)
        B8 = rng.integers(-128, 128, size=n * kp, dtype=np.int8)
        C32 = oracle_i8_gemm(m, n, kp, A8, B8)
        ref = (A8.reshape(m, kp).astype(np.int64) @ B8.reshape(n, kp).astype(np.int64).T)
        assert np.array_equal(C32.reshape(n, m).T, ref)


def test_i8_gemm_int32_edge_closed_form():
    # tests/test_i8_grouped.cu:239-254: all -128 at kp = 131040 -> every entry 16384 * 131040
    kp = 131040
    A8 = np.full(2 * kp, -128, dtype=np.int8)
    B8 = np.full(3 * kp, -128, dtype=np.int8)
    C32 = oracle_i8_gemm(2, 3, kp, A8, B8)
    assert (C32 == 2146959360).all()


# --------------------------------------------------------------------- reconstruct + KATs
def _replay_prefix():
    """Advance the replayer through section 1 of the reference test (4 makes)."""
    katgen().katgen_seed(12345, 0)
    for _ in range(4):
        HostProb(37, 29, 100, 5, 2.0).make()


SWEEP_SHAPES = [(16, 16, 16), (64, 64, 64), (128, 96, 1000), (64, 64, 4096)]
PHIS = [0.0, 0.5, 1.0, 2.0, 4.0]


def test_sweep_repair_count_kats():
    """log lines 23-340: for every (shape, phi) the replayed data reproduces the logged naive FP64
    rel_cw, and the oracle's repaired-entry count and its four error columns (rel_cw, rel_abs,
    rel_nrm, gate) match the log for every N = 8..20 checked."""
    ora = oracle()
    _replay_prefix()
    ci = 0
    for sh in SWEEP_SHAPES:
        for phi in PHIS:
            exp = KAT["sweep"][ci]
            ci += 1
            h = HostProb(sh[0], sh[1], sh[2], 3, phi).make().reference()
            relcw = katgen().katgen_naive_relcw(h.m, h.n, h.k, h.A, h.lda, h.B, h.ldb, h.R)
            assert f"{relcw:.3e}" == f"{exp['naive_rel_cw']:.3e}", (sh, phi)
            Ns = range(8, 21) if sh[2] <= 64 else (8, 13, 14, 15, 16, 17, 20)
            for N in Ns:
                Cres, cnt = h.emulate(REPAIR_ON, N)
                assert int(cnt[2]) == exp["rep"][str(N)], (sh, phi, N)
                g, over = h.gate(Cres)
                assert g <= 1.0 and over == 0, (sh, phi, N, g)
                # every printed column to the log's 4 significant digits: the worst entry's error
                # (rel_cw, rel_abs, rel_nrm, gate) moves with any bit of any emulated entry
                cols, beta_ok = h.check(Cres)
                got = list(cols[:3]) + [ora.oz2o_error_bound(sh[2], N), cols[3]]
                assert beta_ok, (sh, phi, N)
                assert [f"{x:.3e}" for x in got] == [f"{x:.3e}" for x in exp["cols"][str(N)]], (sh, phi, N)


def _advance_to_section3():
    _replay_prefix()
    for sh in SWEEP_SHAPES:
        for phi in PHIS:
            HostProb(sh[0], sh[1], sh[2], 3, phi).make()


SECTION3 = [(200, 150, 777, 20, 1.0, 1.0, 0.0, 0), (1, 300, 64, 16, 0.5, -2.5, 1.0, 0),
            (300, 1, 129, 12, 2.0, 0.75, -0.5, 0), (77, 55, 1, 8, 1.0, 1.0, 2.0, 0),
            (64, 48, 512, 18, 1.0, 1.0, 0.0, 1), (40, 33, 300, 14, 1.0, 1.0, 0.0, 2),
            (33, 65, 2048, 10, 4.0, 1.0, 0.25, 0), (48, 48, 256, 15, 1.0, 1.0, 0.0, 3),
            (16, 16, 16, 15, 2.0, 1.0, 0.0, 0)]


def make_section3():
    """The 9 heterogeneous problems of tests/test_numerics_standalone.cu:317-351 (after replaying
    sections 1-2), with the same special modifications."""
    _advance_to_section3()
    hs = []
    for (m, n, k, N, phi, al, be, sp) in SECTION3:
        h = HostProb(m, n, k, 7, phi, al, be, N).make()
        if sp == 1:
            h.A[:] = np.ldexp(h.A, -700)
            h.B[:] = np.ldexp(h.B, 650)
        elif sp == 2:
            h.A[3 + np.arange(k) * h.lda] = 0.0
            h.B[np.arange(k) + 5 * h.ldb] = 0.0
        elif sp == 3:
            for j in range(n):
                for q in range(0, k - 1, 2):
                    h.B[q + j * h.ldb] = h.A[(q + 1) * h.lda]
                    h.B[q + 1 + j * h.ldb] = -h.A[q * h.lda] * (1.0 + np.ldexp(float(j), -40))
        hs.append(h.reference())
    return hs


def make_section4():
    hs = make_section3()
    h = HostProb(50, 40, 200, 2, 1.0, 1.0, 0.0, 16).make().reference()
    h.A[2 + 17 * h.lda] = np.nan
    h.B[33 + 4 * h.ldb] = np.inf
    return hs, h


def make_section5():
    _, _ = make_section4()
    return [HostProb(16, 16, 16, 0, 2.0, 1.0, 0.0, 15).make().reference() for _ in range(64)]


def test_grouped_and_nonfinite_kats():
    """log lines 343-355: the 9-problem launch's repair total and, per problem, the four error
    columns and the a-priori bound to the printed digits; the non-finite problem's counter, its
    poisoned row / column, and the gate over the other entries."""
    hs, h4 = make_section4()
    total = 0
    for h, exp in zip(hs, KAT["grouped"]):
        assert [h.m, h.n, h.k, h.N] == exp["mnkN"]
        Cres, cnt = h.emulate(REPAIR_ON)
        total += int(cnt[2])
        g, over = h.gate(Cres)
        assert g <= 1.0
        cols, beta_ok = h.check(Cres)
        got = list(cols[:3]) + [oracle().oz2o_error_bound(h.k, h.N), cols[3]]
        assert beta_ok
        assert [f"{x:.3e}" for x in got] == [f"{x:.3e}" for x in exp["cols"]], exp["mnkN"]
    assert total == KAT["grouped_repaired"]
    Cres, cnt = h4.emulate(REPAIR_ON)
    assert int(cnt[0]) == KAT["nonfinite_counter"]
    Cm = Cres.reshape(h4.n, h4.ldc)[:, :h4.m].T
    assert not np.isfinite(Cm[2, :]).any() and not np.isfinite(Cm[:, 4]).any()
    # gate(rest): err / (gamma_n |A||B|) over the entries outside row 2 and column 4, with R and
    # |A||B| of the data before the NaN / Inf were planted (tests/test_numerics_standalone.cu:368-398)
    u = 2.0 ** -53
    gam = h4.k * u / (1 - h4.k * u)
    R = h4.R.reshape(h4.n, h4.m).T
    ab = h4.absAB.reshape(h4.n, h4.m).T
    keep = np.ones((h4.m, h4.n), dtype=bool)
    keep[2, :] = False
    keep[:, 4] = False
    gate = float(np.max(np.abs(Cm[keep].astype(np.longdouble) - R[keep]) / (gam * ab[keep])))
    assert f"{gate:.3e}" == f"{KAT['nonfinite_gate']:.3e}"


def test_repair_mode_kats():
    hs = make_section5()
    outs, cnts, gates = {}, {}, []
    for mode in (REPAIR_OFF, REPAIR_COUNT, REPAIR_ON):
        res = [h.emulate(mode) for h in hs]
        outs[mode] = np.concatenate([r[0] for r in res])
        cnts[mode] = sum(r[1] for r in res)
        gmax = max(h.gate(r[0])[0] for h, r in zip(hs, res))
        gates.append(max(h.check(r[0])[0][3] for h, r in zip(hs, res)))
        if mode == REPAIR_ON:
            assert gmax <= 1.0
    assert [f"{x:.3e}" for x in gates] == [f"{x:.3e}" for x in KAT["repair_modes"]["gates"]]
    assert int(cnts[REPAIR_COUNT][1]) == KAT["repair_modes"]["uncertified"]
    assert int(cnts[REPAIR_ON][2]) == KAT["repair_modes"]["repaired"]
    assert np.array_equal(outs[REPAIR_OFF].view(np.int64), outs[REPAIR_COUNT].view(np.int64))


def test_blas_edge_semantics():
    """tests/test_numerics_standalone.cu:435-466: alpha=0 never reads A/B; NaN alpha with a zero row
    gives NaN; Inf C0 with beta != 0 propagates without repair or safety."""
    h0 = HostProb(20, 10, 50, 0, 1.0, 0.0, 0.5, 15).make()
    h0.A[3] = np.nan
    C0, c0 = h0.emulate(REPAIR_ON)
    M0 = h0.C0.reshape(h0.n, h0.ldc)[:, :h0.m]
    assert np.array_equal(C0.reshape(h0.n, h0.ldc)[:, :h0.m], 0.5 * M0)
    h1 = HostProb(20, 10, 50, 0, 1.0, np.nan, 0.0, 15).make()
    h1.A[4 + np.arange(50) * h1.lda] = 0.0
    C1, c1 = h1.emulate(REPAIR_ON)
    assert np.isnan(C1.reshape(h1.n, h1.ldc)[:, :h1.m]).all()
    h2 = HostProb(20, 10, 50, 0, 1.0, 1.0, 1.0, 15).make()
    h2.C0[7] = np.inf
    C2, c2 = h2.emulate(REPAIR_ON)
    assert not np.isfinite(C2[7])
    assert int(c0[3] + c1[3] + c2[3]) == 0


# --------------------------------------------------------------------------------- planner
def _valid_model(num_sms=132):
    v = json.loads((GOLDEN / "planner_valid.json").read_text())
    return DeviceModel(num_sms, v["f64_peak_flops"], v["i8_peak_ops"], v["bw_Bps"], 32.0 ** 3)


def test_planner_route_table():
    dm = _valid_model()
    cases = json.loads((GOLDEN / "planner_routes.json").read_text())["cases"]
    for c in cases:
        s = Shape(c["m"], c["n"], c["k"], c.get("alpha", 1.0), c.get("beta", 0.0))
        e = PlanEntry()
        rc = oracle().oz2o_plan(C.byref(s), 1, c["nm"], 1e-15, c["fb"], c["path"], C.byref(dm), 16.0,
                                C.byref(e))
        assert rc == c["rc"], c["name"]
        if rc == 0:
            if c["route"] < 0:
                assert e.route != 7, c["name"]
            else:
                assert e.route == c["route"], c["name"]


def test_planner_auto_num_moduli_and_costs():
    dm = _valid_model()
    for k in [17, 32, 100, 512, 1024, 4096, 16384, 65536, 131040]:
        s = Shape(4096, 4096, k, 1.0, 0.0)
        e = PlanEntry()
        assert oracle().oz2o_plan(C.byref(s), 1, 0, 1e-15, 0, 4, C.byref(dm), 16.0, C.byref(e)) == 0
        want = min(max(oracle().oz2o_choose_num_moduli_cw(k, 16.0), 2), 20)
        assert e.route == 0 and e.num_moduli == want
    # routes agree with the reported costs after tile re-evaluation (tests/test_planner.cpp:330-345)
    sz = [24, 48, 96, 160, 224, 256, 384, 512, 768, 1024, 2048]
    kk = [17, 64, 256, 1024, 4096, 16384]
    mix = [Shape(m, n, k, 1.0, 0.0 if (m + n) % 3 else 1.0) for m in sz for n in sz for k in kk]
    arr = (Shape * len(mix))(*mix)
    out = (PlanEntry * len(mix))()
    assert oracle().oz2o_plan(arr, len(mix), 0, 1e-15, 1, 4, C.byref(dm), 16.0, out) == 0
    for e in out:
        if e.route == 0:
            assert e.t_emu_s <= e.t_native_s
        if e.route == 5:
            assert e.t_emu_s > e.t_native_s


# ------------------------------------------------------------------------- CPU baseline GEMM
@pytest.mark.parametrize("m,n,k,lda_pad,alpha,beta", [(1, 1, 1, 0, 1.0, 0.0), (70, 33, 300, 5, -1.5, 0.5),
                                                       (129, 65, 257, 0, 2.0, 1.0), (64, 32, 256, 3, 0.0, -0.75),
                                                       (200, 97, 5, 0, 1.0, 0.0)])
def test_cpu_baseline_dgemm_matches_numpy(m, n, k, lda_pad, alpha, beta):
    """oracle/oz2_dgemm.c (the bench's timed CPU baseline): C = alpha A B + beta C, column-major with
    leading dimensions above the row counts, block edges (m, n, k not multiples of the 64 / 32 / 256
    blocks), alpha = 0, and beta = 0 never reading C (NaN there must not propagate).  Against numpy's
    float64 product within the componentwise FP64 bound gamma_{k+2} (|alpha| |A| |B| + |beta C|)."""
    rng = np.random.default_rng(m * 1000 + n * 10 + k)
    lda, ldb, ldc = m + lda_pad, k + lda_pad, m + lda_pad
    A = rng.standard_normal((k, lda))          # column-major m x k with leading dimension lda
    B = rng.standard_normal((n, ldb))          # column-major k x n
    C0 = rng.standard_normal((n, ldc))         # column-major m x n
    if beta == 0.0:
        C0[:, :m] = np.nan
    Cw = C0.copy()
    oracle().oz2o_dgemm(m, n, k, alpha, A.reshape(-1), lda, B.reshape(-1), ldb, beta, Cw.reshape(-1), ldc)
    a, b = A[:, :m].T, B[:, :k].T               # m x k, k x n
    c0 = np.zeros((m, n)) if beta == 0.0 else C0[:, :m].T
    ref = alpha * (a @ b) + beta * c0
    bound = abs(alpha) * (np.abs(a) @ np.abs(b)) + abs(beta) * np.abs(c0)
    u = 2.0 ** -53
    gam = (k + 2) * u / (1 - (k + 2) * u)
    got = Cw[:, :m].T
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - ref) <= 2 * gam * bound + 1e-300)
    assert np.array_equal(Cw[:, m:], C0[:, m:], equal_nan=True)   # padding rows untouched
