"""ctypes access to the CPU oracle (oracle/liboz2oracle.so) and the KAT data replayer
(tests/golden/libkatgen.so).  Test infrastructure: the checker, never the thing under test."""
import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parents[1]
ORACLE_DIR = REPO / "oracle"
GOLDEN = REPO / "tests" / "golden"

_dp = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_ldp = np.ctypeslib.ndpointer(dtype=np.longdouble, flags="C_CONTIGUOUS")

MAXN = 20
SHIFT_NONFINITE = -2147483648
SHIFT_ZERO = -2147483647
REPAIR_OFF, REPAIR_COUNT, REPAIR_ON = 0, 1, 2


class Tables(C.Structure):
    _fields_ = [("p", C.c_int32 * MAXN), ("magic", C.c_uint32 * MAXN),
                ("pow2", (C.c_uint8 * 128) * MAXN),
                ("s1", (C.c_uint64 * MAXN) * (MAXN + 1)), ("s2", (C.c_uint32 * MAXN) * (MAXN + 1)),
                ("qinv", (C.c_int32 * MAXN) * (MAXN + 1)), ("P1", C.c_int64 * (MAXN + 1)),
                ("P2", C.c_double * (MAXN + 1)), ("inv_Pu", C.c_double * (MAXN + 1)),
                ("log2_u1", C.c_int32 * (MAXN + 1)), ("T", C.c_double * (MAXN + 1)),
                ("log2P", C.c_double * (MAXN + 1))]


class DeviceModel(C.Structure):
    _fields_ = [("num_sms", C.c_int), ("fp64_flops", C.c_double), ("int8_ops", C.c_double),
                ("mem_bw", C.c_double), ("tiny_mnk", C.c_double)]


class PlanEntry(C.Structure):
    _fields_ = [("route", C.c_int), ("num_moduli", C.c_int), ("tile_cfg", C.c_int),
                ("t_emu_s", C.c_double), ("t_native_s", C.c_double)]


class Shape(C.Structure):
    _fields_ = [("m", C.c_int), ("n", C.c_int), ("k", C.c_int), ("alpha", C.c_double), ("beta", C.c_double)]


def _build_if_missing(path, builder):
    if not path.exists():
        builder()
    return path


def build_oracle():
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)


def build_katgen():
    subprocess.run(["python3", str(GOLDEN / "build_katgen.py")], check=True)


_ora = None
_kat = None


def oracle():
    global _ora
    if _ora is None:
        lib = C.CDLL(str(_build_if_missing(ORACLE_DIR / "liboz2oracle.so", build_oracle)))
        lib.oz2o_tables_get.restype = C.POINTER(Tables)
        lib.oz2o_build_tables.argtypes = [C.POINTER(Tables)]
        lib.oz2o_error_bound.restype = C.c_double
        lib.oz2o_error_bound.argtypes = [C.c_int, C.c_int]
        lib.oz2o_choose_num_moduli.argtypes = [C.c_int, C.c_double]
        lib.oz2o_choose_num_moduli_cw.argtypes = [C.c_int, C.c_double]
        lib.oz2o_prep_rows.argtypes = [C.c_int, C.c_int, C.c_int, _dp, C.c_int, _i8p, _i32p, _i64p]
        lib.oz2o_prep_cols.argtypes = [C.c_int, C.c_int, C.c_int, _dp, C.c_int, _i8p, _i32p, _i64p]
        lib.oz2o_i8_gemm.argtypes = [C.c_int, C.c_int, C.c_int, _i8p, _i8p, _i32p]
        lib.oz2o_reconstruct.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, _dp, C.c_int, _dp, C.c_int,
                                         _dp, C.c_int, C.c_double, C.c_double, _i32p, _i32p, _i32p,
                                         C.c_int, _i64p]
        lib.oz2o_emulate.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, _dp, C.c_int, _dp, C.c_int,
                                     _dp, C.c_int, C.c_double, C.c_double, C.c_int, _i64p]
        lib.oz2o_fp64_dot.restype = C.c_double
        lib.oz2o_dgemm.argtypes = [C.c_int, C.c_int, C.c_int, C.c_double, _dp, C.c_int, _dp, C.c_int,
                                   C.c_double, _dp, C.c_int]
        lib.oz2o_plan.argtypes = [C.POINTER(Shape), C.c_int, C.c_int, C.c_double, C.c_int, C.c_int,
                                  C.POINTER(DeviceModel), C.c_double, C.POINTER(PlanEntry)]
        lib.oz2o_route_is_fallback.argtypes = [C.c_int]
        _ora = lib
    return _ora


def katgen():
    global _kat
    if _kat is None:
        lib = C.CDLL(str(_build_if_missing(GOLDEN / "libkatgen.so", build_katgen)))
        lib.katgen_seed.argtypes = [C.c_ulonglong, C.c_int]
        lib.katgen_make.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_double, _dp, _dp, _dp]
        lib.katgen_reference.argtypes = [C.c_int, C.c_int, C.c_int, _dp, C.c_int, _dp, C.c_int, _dp,
                                         C.c_int, C.c_double, C.c_double, _ldp, _dp, _dp]
        lib.katgen_reference_dd.argtypes = [C.c_int, C.c_int, C.c_int, _dp, C.c_int, _dp, C.c_int, _dp,
                                            C.c_int, C.c_double, C.c_double, _dp, _dp, _dp, _dp]
        lib.katgen_naive_relcw.restype = C.c_double
        lib.katgen_naive_relcw.argtypes = [C.c_int, C.c_int, C.c_int, _dp, C.c_int, _dp, C.c_int, _ldp]
        lib.katgen_check.argtypes = [C.c_int, C.c_int, C.c_int, C.c_double, C.c_double, _dp, _dp, C.c_int,
                                     _ldp, _dp, _dp, _dp]
        lib.katgen_gate.restype = C.c_double
        lib.katgen_gate.argtypes = [C.c_int, C.c_int, C.c_int, C.c_double, C.c_double, _dp, C.c_int,
                                    _dp, C.c_int, _ldp, _dp, C.POINTER(C.c_longlong)]
        _kat = lib
    return _kat


def tables():
    return oracle().oz2o_tables_get().contents


def kp_of(k):
    return (k + 31) // 32 * 32


class HostProb:
    """One problem in the reference test's host layout (column-major with padded leading dims)."""

    def __init__(self, m, n, k, lda_pad, phi, alpha=1.0, beta=0.0, N=15):
        self.m, self.n, self.k, self.phi = m, n, k, phi
        self.lda, self.ldb, self.ldc = m + lda_pad, k + 3, m + 1
        self.alpha, self.beta, self.N = alpha, beta, N
        self.A = np.zeros(self.lda * max(k, 1))
        self.B = np.zeros(self.ldb * max(n, 1))
        self.C0 = np.zeros(self.ldc * max(n, 1))

    def make(self):
        katgen().katgen_make(self.m, self.n, self.k, self.lda - self.m, self.phi, self.A, self.B, self.C0)
        return self

    def reference(self):
        m, n = self.m, self.n
        self.R = np.zeros(m * n, dtype=np.longdouble)
        self.absAB = np.zeros(m * n)
        self.nrm = np.zeros(m * n)
        katgen().katgen_reference(m, n, self.k, self.A, self.lda, self.B, self.ldb, self.C0, self.ldc,
                                  self.alpha, self.beta, self.R, self.absAB, self.nrm)
        return self

    def gate(self, Cres):
        """(max err / (gamma_n den), #entries over the bound) of Cres (ldc layout) vs R."""
        cnt = C.c_longlong(0)
        g = katgen().katgen_gate(self.m, self.n, self.k, self.alpha, self.beta, Cres, self.ldc, self.C0,
                                 self.ldc, self.R, self.absAB, C.byref(cnt))
        return g, cnt.value

    def check(self, Cres):
        """The reference test's error columns of Cres (ldc layout) against R (after reference()):
        (rel_cw, rel_abs, rel_nrm, gate), and whether C's padding rows equal C0's."""
        out = np.zeros(4)
        ok = katgen().katgen_check(self.m, self.n, self.k, self.alpha, self.beta, np.ascontiguousarray(Cres),
                                   self.C0, self.ldc, self.R, self.absAB, self.nrm, out)
        return tuple(float(x) for x in out), bool(ok)

    def emulate(self, mode=REPAIR_ON, N=None):
        """Oracle result C (ldc layout) and counters [nonfinite, uncertified, repaired, safety]."""
        N = self.N if N is None else N
        Cout = self.C0.copy()
        cnt = np.zeros(4, dtype=np.int64)
        rc = oracle().oz2o_emulate(self.m, self.n, self.k, N, self.A, self.lda, self.B, self.ldb, Cout,
                                   self.ldc, self.alpha, self.beta, mode, cnt)
        assert rc == 0, rc
        return Cout, cnt


def oracle_prep(m, n, k, N, A, lda, B, ldb):
    """Oracle residues and workspaces for one problem: (A8, B8, rws, cws, nonfinite)."""
    kp = kp_of(k)
    A8 = np.zeros((N + 1) * m * kp + 1, dtype=np.int8)
    B8 = np.zeros((N + 1) * n * kp + 1, dtype=np.int8)
    rws = np.zeros(4 * m + 1, dtype=np.int32)
    cws = np.zeros(4 * n + 1, dtype=np.int32)
    nf = np.zeros(1, dtype=np.int64)
    oracle().oz2o_prep_rows(m, k, N, A, lda, A8, rws, nf)
    oracle().oz2o_prep_cols(n, k, N, B, ldb, B8, cws, nf)
    return A8[:-1], B8[:-1], rws[:-1], cws[:-1], int(nf[0])


def oracle_i8_gemm(m, n, kp, A8, B8):
    C32 = np.zeros(m * n + 1, dtype=np.int32)
    bad = oracle().oz2o_i8_gemm(m, n, kp, np.ascontiguousarray(A8), np.ascontiguousarray(B8), C32)
    assert bad == 0
    return C32[:-1]
