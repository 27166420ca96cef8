"""ctypes binding of the MI355X grouped Ozaki-II DGEMM library (libggemm_mi355x.so).

Mirrors the C ABI of include/ggemm.h, include/ggemm_graph.h and include/ggemm_oz2.h: same names,
struct layouts and return codes as the reference's interface.  Device memory is passed as plain
integer addresses (e.g. torch_tensor.data_ptr()); streams as integer handles (0 = default).
The library must be built (coding-basic-hw-2_amd/build_lib.py); there is no fallback path.
"""
import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libggemm_mi355x.so"

GGEMM_OK, GGEMM_ERR_INVALID, GGEMM_ERR_WORKSPACE, GGEMM_ERR_UNSAFE = 0, 1, 2, 3
GGEMM_ERR_CUDA, GGEMM_ERR_CUBLAS, GGEMM_ERR_NUMERICS, GGEMM_ERR_I8GEMM, GGEMM_ERR_ALLOC = 4, 5, 6, 7, 8
PATH_NATIVE_LOOP, PATH_NATIVE_GROUPED, PATH_EMU_LOOP, PATH_EMU_GROUPED = 0, 1, 2, 3
PATH_AUTO, PATH_EMU_GROUPED_REUSE, PATH_EMU_LOOP_BATCHED = 4, 5, 6
REPAIR_DEFAULT, REPAIR_OFF, REPAIR_COUNT, REPAIR_ON = 0, 1, 2, 3
OZ2_REPAIR_OFF, OZ2_REPAIR_COUNT, OZ2_REPAIR_ON = 0, 1, 2
MAX_MODULI = 20
MAX_K_EXACT = 131040
NOALLOC_SCRATCH_BYTES = 64 << 20
NOALLOC_MAX_PROBLEMS = 64
NOALLOC_MAX_ELEMS = 262144
SHIFT_NONFINITE = -2147483648
SHIFT_ZERO = -2147483647
ROUTES = ["EMU", "EMPTY", "K_ZERO", "K_TOO_LARGE", "TINY", "UNPROFITABLE", "PRECISION", "SMALL_K", "ALPHA_ZERO"]


class Problem(C.Structure):
    _fields_ = [("m", C.c_int), ("n", C.c_int), ("k", C.c_int),
                ("A", C.c_void_p), ("lda", C.c_int),
                ("B", C.c_void_p), ("ldb", C.c_int),
                ("C", C.c_void_p), ("ldc", C.c_int),
                ("alpha", C.c_double), ("beta", C.c_double)]


class Config(C.Structure):
    _fields_ = [("num_moduli", C.c_int), ("target_rel_err", C.c_double),
                ("allow_fallback", C.c_int), ("repair_mode", C.c_int)]


class Stats(C.Structure):
    _fields_ = [("num_problems", C.c_int), ("num_fallback", C.c_int), ("kernel_launches", C.c_int),
                ("moduli_min", C.c_int), ("moduli_max", C.c_int), ("reuse_enabled", C.c_int),
                ("num_unique_A", C.c_int), ("num_unique_B", C.c_int), ("num_promoted", C.c_int),
                ("num_repaired", C.c_longlong), ("num_uncertified", C.c_longlong),
                ("num_safety_fallback", C.c_longlong)]

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_}


class Oz2Problem(C.Structure):
    _fields_ = [("m", C.c_int), ("n", C.c_int), ("k", C.c_int), ("kp", C.c_int), ("num_moduli", C.c_int),
                ("lda", C.c_int), ("ldb", C.c_int), ("ldc", C.c_int),
                ("A", C.c_void_p), ("B", C.c_void_p), ("C", C.c_void_p),
                ("alpha", C.c_double), ("beta", C.c_double),
                ("A8", C.c_void_p), ("B8", C.c_void_p),
                ("a8_mod_stride", C.c_size_t), ("b8_mod_stride", C.c_size_t),
                ("C32", C.c_void_p), ("c32_mod_stride", C.c_size_t),
                ("row_shift", C.c_void_p), ("col_shift", C.c_void_p)]


class Oz2Counters(C.Structure):
    _fields_ = [("nonfinite_vectors", C.c_ulonglong), ("uncertified", C.c_ulonglong),
                ("repaired", C.c_ulonglong), ("safety_fallback", C.c_ulonglong)]


class I8Problem(C.Structure):
    _fields_ = [("m", C.c_int), ("n", C.c_int), ("kp", C.c_int), ("A", C.c_void_p), ("B", C.c_void_p),
                ("C", C.c_void_p), ("tile_cfg", C.c_int)]


class I8SchedInfo(C.Structure):
    _fields_ = [("tiles_main", C.c_int), ("tiles_splitk", C.c_int), ("num_launches", C.c_int),
                ("ws2_offset_ints", C.c_int), ("bytes_used", C.c_size_t)]


class PlanEntry(C.Structure):
    _fields_ = [("route", C.c_int), ("num_moduli", C.c_int), ("tile_cfg", C.c_int),
                ("t_emu_s", C.c_double), ("t_native_s", C.c_double)]


class DeviceModel(C.Structure):
    _fields_ = [("num_sms", C.c_int), ("fp64_flops", C.c_double), ("int8_ops", C.c_double),
                ("mem_bw", C.c_double), ("tiny_mnk", C.c_double)]


class ReusePlan(C.Structure):
    """include/ggemm_reuse.h reuse_plan (a view into the arena)."""
    _fields_ = [("status", C.c_int), ("num_problems", C.c_int), ("num_ua", C.c_int), ("num_ub", C.c_int),
                ("num_emu", C.c_int), ("num_promoted", C.c_int),
                ("ua_rep", C.POINTER(C.c_int)), ("ua_nmod", C.POINTER(C.c_int)),
                ("ub_rep", C.POINTER(C.c_int)), ("ub_nmod", C.POINTER(C.c_int)),
                ("prob_a", C.POINTER(C.c_int)), ("prob_b", C.POINTER(C.c_int)), ("eff_nmod", C.POINTER(C.c_int))]


class ReuseBytes(C.Structure):
    _fields_ = [("prep_read", C.c_double), ("prep_write", C.c_double), ("ws_A8", C.c_double),
                ("ws_B8", C.c_double)]


REUSE_EXACT_N, REUSE_PROMOTE = 0, 1
REUSE_OK, REUSE_ERR_CAPACITY, REUSE_ERR_INVALID = 0, 1, 2

_P = C.c_void_p
# (name, restype, argtypes) of every exported C entry point
SIGNATURES = [
    ("ggemm_create", C.c_int, [C.POINTER(_P), C.c_int, C.c_size_t, C.c_size_t, C.c_size_t, _P]),
    ("ggemm_create_ex", C.c_int, [C.POINTER(_P), C.c_int, C.c_size_t, C.c_size_t, C.c_size_t, _P, C.c_int]),
    ("ggemm_destroy", None, [_P]),
    ("ggemm_grouped_dgemm", C.c_int, [_P, C.c_int, C.POINTER(Config), C.POINTER(Problem), C.c_int,
                                      C.POINTER(Stats)]),
    ("ggemm_grouped_dgemm_noalloc", C.c_int, [C.c_int, C.POINTER(Config), C.POINTER(Problem), C.c_int, _P,
                                              C.POINTER(Stats)]),
    ("ggemm_make_plan", _P, [_P, C.c_int, C.POINTER(Config), C.POINTER(Problem), C.c_int]),
    ("ggemm_make_plan_ex", _P, [_P, C.c_int, C.POINTER(Config), C.POINTER(Problem), C.c_int, C.POINTER(C.c_int)]),
    ("ggemm_execute_plan", C.c_int, [_P, _P]),
    ("ggemm_plan_update_pointers", C.c_int, [_P, C.POINTER(_P), C.POINTER(_P), C.POINTER(_P)]),
    ("ggemm_plan_get_stats", C.c_int, [_P, C.POINTER(Stats)]),
    ("ggemm_destroy_plan", None, [_P]),
    ("oz2_init_constants", C.c_int, []),
    ("oz2_prep_grouped", C.c_int, [_P, C.c_int, C.c_int, C.c_int, _P]),
    ("oz2_reconstruct_grouped", C.c_int, [_P, C.c_int, C.c_int, C.c_int, _P, C.c_int]),
    ("oz2_choose_num_moduli", C.c_int, [C.c_int, C.c_double]),
    ("oz2_error_bound", C.c_double, [C.c_int, C.c_int]),
    ("oz2_choose_num_moduli_cw", C.c_int, [C.c_int, C.c_double]),
    ("oz2_read_counters", C.c_int, [C.POINTER(Oz2Counters), C.c_int, _P]),
    ("oz2_debug_force_prep_split", None, [C.c_int]),
    ("oz2_mfma_f64_chains", C.c_int, [_P, _P, _P, C.c_int, C.c_int, _P]),
    ("i8_grouped_gemm_sched_ws_bytes", C.c_size_t, [C.c_int, C.c_size_t]),
    ("i8_grouped_gemm_reserve", None, [C.c_int, C.c_size_t]),
    ("i8_grouped_gemm_host_allocs", C.c_longlong, []),
    ("i8_grouped_gemm_build_schedule", C.c_int, [C.POINTER(I8Problem), C.c_int, _P, C.c_size_t,
                                                 C.POINTER(I8SchedInfo)]),
    ("i8_grouped_gemm_launch", C.c_int, [_P, C.c_int, _P, C.POINTER(I8SchedInfo), _P]),
    ("i8_grouped_gemm_ex", C.c_int, [_P, C.c_int, C.POINTER(I8Problem), _P, C.c_size_t, _P, C.POINTER(C.c_int)]),
    ("ggemm_device_model_init", None, [C.POINTER(DeviceModel), C.c_char_p, C.c_int, C.c_int, C.c_int]),
    ("ggemm_plan_num_moduli", C.c_int, [C.POINTER(Config), C.c_int]),
    ("ggemm_plan", C.c_int, [C.POINTER(Problem), C.c_int, C.POINTER(Config), C.c_int, C.POINTER(DeviceModel),
                             C.POINTER(PlanEntry)]),
    ("ggemm_plan_ex", C.c_int, [C.POINTER(Problem), C.c_int, C.POINTER(Config), C.c_int, C.POINTER(DeviceModel),
                                C.POINTER(PlanEntry), C.POINTER(C.c_int), C.c_size_t]),
    ("ggemm_plan_memo_cap", C.c_size_t, [C.c_int]),
    ("ggemm_profile_enable", C.c_int, [C.c_int]),
    ("ggemm_profile_read", C.c_int, [C.POINTER(C.c_double), C.POINTER(C.c_longlong), C.c_int]),
    ("ggemm_profile_i8_kernel", C.c_char_p, []),
    ("reuse_arena_create", C.c_int, [C.c_int, C.POINTER(_P)]),
    ("reuse_arena_destroy", None, [_P]),
    ("reuse_arena_capacity", C.c_int, [_P]),
    ("build_operand_reuse", ReusePlan, [_P, C.POINTER(Problem), C.c_int, C.POINTER(C.c_int), C.c_int]),
    ("operand_reuse_bytes", None, [C.POINTER(ReusePlan), C.POINTER(Problem), C.POINTER(C.c_int),
                                   C.POINTER(ReuseBytes), C.POINTER(ReuseBytes)]),
]

_lib = None


def lib():
    """The loaded library; raises if it has not been built (no CPU fallback exists)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with coding-basic-hw-2_amd/build_lib.py")
        L = C.CDLL(str(LIB_PATH))
        for name, res, args in SIGNATURES:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def problems_array(probs):
    arr = (Problem * max(len(probs), 1))()
    for i, p in enumerate(probs):
        arr[i] = p
    return arr


def check(rc, what=""):
    if rc != GGEMM_OK:
        raise RuntimeError(f"{what} failed with GGEMM error {rc}")
    return rc


class Handle:
    """RAII wrapper of ggemm_handle_t."""

    def __init__(self, max_problems, max_a, max_b, max_c, stream=0, min_k=None):
        self.h = C.c_void_p()
        if min_k is None:
            rc = lib().ggemm_create(C.byref(self.h), max_problems, max_a, max_b, max_c, stream)
        else:
            rc = lib().ggemm_create_ex(C.byref(self.h), max_problems, max_a, max_b, max_c, stream, min_k)
        check(rc, "ggemm_create")

    def dgemm(self, path, cfg, probs, stats=None):
        arr = problems_array(probs)
        st = stats if stats is not None else Stats()
        rc = lib().ggemm_grouped_dgemm(self.h, path, C.byref(cfg) if cfg is not None else None, arr, len(probs),
                                       C.byref(st))
        return rc, st

    def close(self):
        if self.h:
            lib().ggemm_destroy(self.h)
            self.h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def stats_repair_enabled():
    return os.environ.get("GGEMM_STATS_REPAIR") == "1"
