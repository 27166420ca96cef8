"""End-to-end ggemm_grouped_dgemm on the GPU through the C ABI (tests/test_grouped.cu semantics).

Emulated problems must equal the oracle bit for bit (same shifts, exact integer products, same
CRT / certificate arithmetic, same sequential repair dots); native-route problems (own FP64 MFMA
GEMM) must meet the componentwise gamma_n gate against a long-double reference.  Stats
(num_fallback, moduli range, repair / uncertified / safety counts, launches) must equal what the
oracle's planner and pipeline give."""
import ctypes as C
import os

import numpy as np
import pytest
import torch

os.environ["GGEMM_STATS_REPAIR"] = "1"   # read at handle creation

import ggemm as G
import oracle_lib as O
from gpu_util import dev, host, same_bits, say

pytestmark = pytest.mark.gpu


def gen(rng, shape_elems, phi):
    v = rng.random(shape_elems) - 0.5
    if phi:
        v *= np.exp(phi * rng.standard_normal(shape_elems))
    return v


class Case:
    """A group of problems with host data (column-major, lda = m + pad) and device copies."""

    def __init__(self, shapes, seed, phi=1.0, alpha=1.0, beta=0.0, pad=0):
        rng = np.random.default_rng(seed)
        self.hp = []
        for s in shapes:
            m, n, k = s[:3]
            a = s[3] if len(s) > 3 else alpha
            b = s[4] if len(s) > 4 else beta
            h = O.HostProb(m, n, k, pad, phi, a, b)
            h.ldb = max(1, k + pad)
            h.ldc = max(1, m + pad)
            h.lda = max(1, m + pad)
            h.A = np.zeros(h.lda * max(k, 1))
            h.B = np.zeros(h.ldb * max(n, 1))
            h.C0 = np.zeros(h.ldc * max(n, 1))
            for c in range(k):
                h.A[c * h.lda: c * h.lda + m] = gen(rng, m, phi)
            for c in range(n):
                h.B[c * h.ldb: c * h.ldb + k] = gen(rng, k, phi)
            for c in range(n):
                h.C0[c * h.ldc: c * h.ldc + m] = gen(rng, m, 0.0)
            self.hp.append(h)
        self.alloc()

    def alloc(self):
        self.dA = [dev(h.A) for h in self.hp]
        self.dB = [dev(h.B) for h in self.hp]
        self.dC = [dev(h.C0) for h in self.hp]

    def reset_C(self):
        for d, h in zip(self.dC, self.hp):
            d.copy_(torch.from_numpy(h.C0))
        torch.cuda.synchronize()

    def problems(self):
        return [G.Problem(h.m, h.n, h.k, a.data_ptr(), h.lda, b.data_ptr(), h.ldb, c.data_ptr(), h.ldc, h.alpha,
                          h.beta) for h, a, b, c in zip(self.hp, self.dA, self.dB, self.dC)]

    def sizes(self):
        return (sum(h.m * h.k for h in self.hp) + 1, sum(h.k * h.n for h in self.hp) + 1,
                sum(h.m * h.n for h in self.hp) + 1)

    def C(self, g):
        return host(self.dC[g])


def run(case, path, cfg, handle=None, min_k=None):
    own = handle is None
    if own:
        handle = G.Handle(max(len(case.hp), 1), *case.sizes(), min_k=min_k)
    case.reset_C()
    rc, st = handle.dgemm(path, cfg, case.problems())
    torch.cuda.synchronize()
    if own:
        handle.close()
    return rc, st


def oracle_plan(case, cfg, path, dm=None):
    if dm is None:
        dm = G.DeviceModel()
        G.lib().ggemm_device_model_init(C.byref(dm), b"gfx950", 9, 5, 256)
    probs = [O.Shape(h.m, h.n, h.k, h.alpha, h.beta) for h in case.hp]
    arr = (O.Shape * max(len(probs), 1))(*probs)
    odm = O.DeviceModel(dm.num_sms, dm.fp64_flops, dm.int8_ops, dm.mem_bw, dm.tiny_mnk)
    out = (O.PlanEntry * max(len(probs), 1))()
    rc = O.oracle().oz2o_plan(arr, len(probs), cfg.num_moduli, cfg.target_rel_err, cfg.allow_fallback, path,
                              C.byref(odm), 16.0, out)
    return rc, list(out)[:len(probs)]


def device_model():
    props = torch.cuda.get_device_properties(0)
    dm = G.DeviceModel()
    G.lib().ggemm_device_model_init(C.byref(dm), props.gcnArchName.encode(), 9, 5, props.multi_processor_count)
    return dm


# kernels of one emulated group call besides prep and the INT8 GEMM: the reconstruct, plus the
# dot-product pass with the blocked digit layout (the default; GGEMM_DIGITS_COLMAJOR=1 turns it off)
def recon_launches(blocked=True):
    """Kernels of the reconstruct stage: the reconstruct, and with blocked digits the dot-product
    pass, the gather of the crossings rows and the crossings pass."""
    return 4 if blocked else 1


def check_case(case, path, cfg, st, mode, blocked=True):
    """Each problem vs the oracle: bitwise for emulated routes, gamma_n gate for native routes.
    Returns the oracle's counters {uncertified, repaired, safety}."""
    plan_path = G.PATH_EMU_LOOP if path == G.PATH_EMU_LOOP_BATCHED else path
    rc, plan = oracle_plan(case, cfg, plan_path, device_model())
    assert rc == 0
    tot = np.zeros(4, dtype=np.int64)
    nfb, nmin, nmax = 0, 99, 0
    for g, (h, e) in enumerate(zip(case.hp, plan)):
        Cg = case.C(g)
        if e.route == 1:   # EMPTY: C untouched
            assert same_bits(Cg, h.C0), g
            continue
        if e.route == 0:
            nmin, nmax = min(nmin, e.num_moduli), max(nmax, e.num_moduli)
            Co, cnt = h.emulate(mode, e.num_moduli)
            tot += cnt
            assert same_bits(Cg, Co), f"problem {g} ({h.m}x{h.n}x{h.k}) differs"
        else:
            nfb += O.oracle().oz2o_route_is_fallback(e.route)
            h.reference()
            gate, over = h.gate(Cg)
            if np.isfinite(h.A).all() and np.isfinite(h.B).all() and np.isfinite(h.C0).all():
                assert gate <= 1.0, f"native problem {g} gate {gate}"
    assert st.num_fallback == nfb
    n_emu = sum(1 for e in plan if e.route == 0)
    n_nat = sum(1 for e in plan if e.route not in (0, 1))
    rl = recon_launches(blocked)
    if path in (G.PATH_EMU_GROUPED, G.PATH_AUTO):
        want = (2 + rl if n_emu else 0) + (1 if n_nat else 0)
    elif path == G.PATH_EMU_LOOP:
        want = sum(e.num_moduli + 2 + rl for e in plan if e.route == 0) + (1 if n_nat else 0)
    else:
        want = (2 + rl) * n_emu + (1 if n_nat else 0)
    assert st.kernel_launches == want, (st.kernel_launches, want)
    if nmax:
        assert (st.moduli_min, st.moduli_max) == (nmin, nmax)
    assert (st.num_uncertified, st.num_repaired, st.num_safety_fallback) == (tot[1], tot[2], tot[3])
    return tot


CFG_EMU = G.Config(0, 1e-15, 0, 0)
CFG_AUTO = G.Config(0, 1e-15, 1, 0)


def test_config1_plumbing_fixed_n14():
    """G=1, 256^3, U(-0.5,0.5), alpha=1 beta=0, fixed N=14 (EMU_GROUPED, COUNT mode)."""
    case = Case([(256, 256, 256)], 20261201, phi=0.0)
    say("config1 256^3 N=14")
    cfg = G.Config(14, 1e-15, 1, 0)
    rc, st = run(case, G.PATH_EMU_GROUPED, cfg)
    assert rc == 0
    assert st.kernel_launches == 2 + recon_launches() and st.moduli_min == st.moduli_max == 14 and st.num_fallback == 0
    check_case(case, G.PATH_EMU_GROUPED, cfg, st, O.REPAIR_COUNT)


@pytest.mark.parametrize("N", [16, 17, 20])
@pytest.mark.parametrize("path", [G.PATH_EMU_GROUPED, G.PATH_EMU_LOOP])
def test_fixed_moduli_digit_widths(path, N):
    """Fixed N on both sides of the residue kernel's digit-width switch (two 32-bit digit words
    of the scaled integers for N <= 16, three above), wide exponent range (phi = 2) so that
    every row and column uses the whole norm budget; ragged k (kp = 32 mod 64)."""
    case = Case([(96, 80, 160), (64, 72, 100), (130, 66, 33)], 20261208 + N, phi=2.0, beta=0.5)
    cfg = G.Config(N, 1e-15, 0, 0)
    say(f"fixed N={N} path={path}")
    rc, st = run(case, path, cfg)
    assert rc == 0
    assert st.moduli_min == st.moduli_max == N
    check_case(case, path, cfg, st, O.REPAIR_COUNT)


@pytest.mark.parametrize("N", [12, 16])
def test_single_read_columns_special_values(N):
    """With two-word digits (N <= 16) the production prep reads a B column with k <= 1024 once and
    keeps it in registers: k at and around the chunk (128) and register (1024) limits (1025 takes
    the two-pass path), the rescale path (2^650 and 2^-700 magnitudes, one 1e300 entry), a zero
    column and NaN / Inf columns, all in one call; bitwise against the oracle with equal counters."""
    shapes = [(40, 24, 1), (40, 24, 33), (36, 20, 127), (33, 17, 129), (48, 40, 1000), (40, 24, 1024),
              (40, 24, 1025)]
    case = Case(shapes, 20261220 + N, phi=1.0, beta=0.5)
    case.hp[2].B[:] = np.ldexp(case.hp[2].B, 650)
    case.hp[3].B[:] = np.ldexp(case.hp[3].B, -700)
    h = case.hp[4]
    h.B[3 * h.ldb: 3 * h.ldb + h.k] = 0.0
    h.B[5 + 7 * h.ldb] = np.nan
    h.B[999 + 11 * h.ldb] = np.inf
    h = case.hp[5]
    h.B[1023 + 2 * h.ldb] = 1e300
    case.alloc()
    cfg = G.Config(N, 1e-15, 0, 0)
    say(f"single-read columns N={N}")
    rc, st = run(case, G.PATH_EMU_GROUPED, cfg)
    assert rc == 0
    assert st.moduli_min == st.moduli_max == N
    check_case(case, G.PATH_EMU_GROUPED, cfg, st, O.REPAIR_COUNT)


@pytest.mark.parametrize("path", [G.PATH_EMU_GROUPED, G.PATH_AUTO, G.PATH_EMU_LOOP, G.PATH_EMU_LOOP_BATCHED])
def test_uniform_group_beta(path):
    """Config-2 shape family, reduced: G=8 x 192^3, (U-0.5)exp(0.5 Z), alpha=1, beta=0.5."""
    case = Case([(192, 192, 192)] * 8, 20261202, phi=0.5, beta=0.5)
    cfg = CFG_AUTO if path == G.PATH_AUTO else CFG_EMU
    say(f"uniform group path={path}")
    rc, st = run(case, path, cfg)
    assert rc == 0
    check_case(case, path, cfg, st, O.REPAIR_ON if path == G.PATH_AUTO else O.REPAIR_COUNT)


def ran_kernel(name, env=None):
    """The INT8 kernel the last call ran is `name`, or its persistent form when the persistent
    schedule is selected for the handle (env) or for the whole process."""
    sched = (env or {}).get("GGEMM_I8_SCHED", os.environ.get("GGEMM_I8_SCHED"))
    want = name.replace("_kernel", "_persistent_kernel") if sched == "persistent" else name
    return G.lib().ggemm_profile_i8_kernel().decode() == want


def kernel_handle(case, kernel=None, **env):
    """A handle created with GGEMM_I8_KERNEL (and further variables) set: read at creation."""
    saved = dict(os.environ)
    if kernel:
        os.environ["GGEMM_I8_KERNEL"] = kernel
    os.environ.update(env)
    try:
        return G.Handle(len(case.hp), *case.sizes())
    finally:
        os.environ.clear()
        os.environ.update(saved)


def run_kernel(case, kernel, cfg=CFG_EMU, **env):
    """EMU_GROUPED through a handle forced onto one INT8 kernel; checks that kernel ran."""
    with kernel_handle(case, kernel, **env) as h:
        rc, st = run(case, G.PATH_EMU_GROUPED, cfg, handle=h)
        assert rc == 0
        assert ran_kernel({"large": "i8_large_kernel", "general": "i8_grouped_kernel"}[kernel], env)
        check_case(case, G.PATH_EMU_GROUPED, cfg, st, O.REPAIR_COUNT, blocked=env.get("GGEMM_DIGITS_COLMAJOR") != "1")
        return [case.C(g).copy() for g in range(len(case.hp))]


SCHED_ENV = {"dispatch": {}, "persistent": {"GGEMM_I8_SCHED": "persistent"}, "rowmajor": {"GGEMM_PACKED_MAX_KP": "0"}}


@pytest.mark.parametrize("sched", ["dispatch", "persistent", "rowmajor"])
@pytest.mark.parametrize("kernel", ["large", "general"])
def test_large_tile_kernel_ragged_edges(kernel, sched):
    """The large-tile INT8 kernel (forced with GGEMM_I8_KERNEL; by default it serves long-k
    calls) and the general kernel on the same products, each with one workgroup per tile, as
    persistent work-stealing kernels (GGEMM_I8_SCHED=persistent), and on row-major residues
    (GGEMM_PACKED_MAX_KP=0: the large kernel's 128-byte stages): m, n are not multiples of 256
    (clamped edge rows) and kp = 480 is 32 mod 64 and 96 mod 128 (the zeroed partial stages)."""
    case = Case([(520, 600, 470)] * 3, 20261206, phi=0.5, beta=0.5)
    say(f"{kernel} kernel, ragged edges, {sched}")
    run_kernel(case, kernel, **SCHED_ENV[sched])


@pytest.mark.parametrize("kernel", ["large", "general"])
def test_persistent_kernels_ragged_group(kernel):
    """The persistent work-stealing INT8 kernels on a ragged group: tile configurations change
    between consecutive tiles of a workgroup (general kernel), queues run dry at different times and
    workgroups steal; k from 32 to 1055, half stages included.  Oracle bits and counters in COUNT
    mode, twice on one handle (the queue counters reset themselves)."""
    rng = np.random.default_rng(20261215)
    shapes = [(int(rng.integers(1, 700)), int(rng.integers(1, 700)), int(rng.integers(32, 1056))) for _ in range(40)]
    case = Case(shapes, 20261215, phi=1.0, beta=0.5)
    say(f"persistent {kernel} kernel, ragged group of {len(shapes)}")
    env = {"GGEMM_I8_SCHED": "persistent"}
    with kernel_handle(case, kernel, **env) as h:
        for rep in range(2):
            case.reset_C()
            rc, st = run(case, G.PATH_EMU_GROUPED, CFG_EMU, handle=h)
            assert rc == 0, rep
            want = {"large": "i8_large_persistent_kernel", "general": "i8_grouped_persistent_kernel"}[kernel]
            assert G.lib().ggemm_profile_i8_kernel().decode() == want
            check_case(case, G.PATH_EMU_GROUPED, CFG_EMU, st, O.REPAIR_COUNT)


@pytest.mark.parametrize("colmajor", [False, True])
def test_large_tile_kernel_mixed_k_stream(colmajor):
    """The large-tile kernel on products with 1 to 9 k-stages (kp = 64 .. 576; kp mod 128 = 0, 32,
    64 and 96, the final partial stages of the 128-byte stages that row-major residues take), full
    tiles and a ragged n (edge stores), with the packed residues and blocked digits (64-byte
    stages) and with the row-major / column-major layouts (GGEMM_DIGITS_COLMAJOR=1)."""
    shapes = [(512, 512, 40), (512, 512, 64), (512, 512, 100), (512, 512, 160), (512, 512, 224),
              (512, 520, 300), (512, 512, 350), (512, 512, 520), (512, 512, 576)]
    case = Case(shapes, 20261207, phi=0.5, beta=0.5)
    say(f"large-tile kernel, mixed k stream, colmajor={colmajor}")
    run_kernel(case, "large", **({"GGEMM_DIGITS_COLMAJOR": "1"} if colmajor else {}))


def test_default_kernel_choice():
    """Automatic choice: the general kernel for calls with packed residues (every Kp <= 4096),
    the large-tile kernel for long-k calls whose 256 x 256 tiles fill the GPU."""
    say("default kernel choice")
    short = Case([(256, 256, 300)] * 2, 20261209, phi=0.5)
    with kernel_handle(short) as h:
        rc, st = run(short, G.PATH_EMU_GROUPED, CFG_EMU, handle=h)
        assert rc == 0 and ran_kernel("i8_grouped_kernel")
    props = torch.cuda.get_device_properties(0)
    g = (props.multi_processor_count + 3) // 4      # 4 tiles of 256 x 256 per problem
    long_k = Case([(512, 512, 4128)] * g, 20261210, phi=0.5)   # kp = 4128 > 4096: row-major
    outs = []
    for kernel, name in ((None, "i8_large_kernel"), ("general", "i8_grouped_kernel")):
        with kernel_handle(long_k, kernel) as h:
            rc, st = run(long_k, G.PATH_EMU_GROUPED, CFG_EMU, handle=h)
            assert rc == 0 and ran_kernel(name)
            outs.append([long_k.C(q).copy() for q in range(g)])
    for a, b in zip(*outs):   # the oracle checks both kernels on smaller shapes above
        assert same_bits(a, b)


def test_default_layout_long_k_matches_oracle():
    """The production layout of a call whose largest Kp exceeds 4096 -- row-major residue planes
    for the problems with Kp > 4096, packed planes for the others (Kp = 1024, and 4096 exactly and
    by rounding k = 4065 up), 16 x 16 blocked digits -- bitwise against the oracle in COUNT mode
    (uncertified entries keep their emulated values), on the default handle (general INT8 kernel
    for this small group) and with the 256 x 256 kernel forced; mixed N (15 at k <= 5000, 16 at
    k = 16384); odd row counts, a single-row problem, ragged tile edges and final half k-stages
    (Kp % 64 = 32)."""
    case = Case([(256, 256, 4160)] * 3 + [(128, 96, 16384), (257, 129, 4097), (3, 1, 4200), (255, 63, 5000),
                                          (200, 150, 1000), (64, 300, 4096), (33, 17, 4065)],
                20261230, phi=1.0, beta=0.5)
    cfg = G.Config(0, 1e-15, 0, G.REPAIR_COUNT)
    rc, plan = oracle_plan(case, cfg, G.PATH_EMU_GROUPED)
    assert rc == 0 and [e.num_moduli for e in plan] == [15, 15, 15, 16, 15, 15, 15, 15, 15, 15]
    want = [h.emulate(O.REPAIR_COUNT, e.num_moduli) for h, e in zip(case.hp, plan)]
    for kernel, name in ((None, "i8_grouped_kernel"), ("large", "i8_large_kernel")):
        say(f"long-k default layout, kernel {name}")
        with kernel_handle(case, kernel) as h:
            rc, st = run(case, G.PATH_EMU_GROUPED, cfg, handle=h)
            assert rc == 0 and ran_kernel(name)
        assert (st.moduli_min, st.moduli_max, st.kernel_launches) == (15, 16, 2 + recon_launches())
        for g, (Co, cnt) in enumerate(want):
            assert same_bits(case.C(g), Co), f"{name}: problem {g} differs"
        assert st.num_uncertified == sum(int(c[1]) for _, c in want)


@pytest.mark.parametrize("shapes", [[(300, 270, 200)] * 2 + [(17, 33, 90), (64, 48, 40)],   # general kernel
                                    [(520, 600, 470)] * 3],                                   # large-tile kernel
                         ids=["general", "large"])
def test_blocked_and_columnmajor_digits_same_bits(shapes):
    """The production layouts -- residue planes packed in 64-byte k-blocks, CRT digits and
    abs-plane products in 16 x 16 blocks -- against the kernel-level ones (row-major residues,
    column-major digits; GGEMM_DIGITS_COLMAJOR=1 forces them).  Both give the oracle's bits; m, n
    are not multiples of 16 (padded blocks) and kp = 96, 224, 480 end in a 32-byte half block."""
    case = Case(shapes, 20261208, phi=0.5, beta=0.5)
    kernel = "large" if len(shapes) == 3 else "general"
    say(f"blocked vs column-major digits, {kernel} kernel")
    outs = [run_kernel(case, kernel), run_kernel(case, kernel, GGEMM_DIGITS_COLMAJOR="1")]
    for a, b in zip(*outs):
        assert same_bits(a, b)


def test_ragged_group_auto():
    """Config-3 family, reduced: m, n log-uniform in [16, 300], k log-uniform in [1, 700] (k <= 16
    takes SMALL_K, k in (16, 32) exercises Kp padding), alpha ~ U(-2, 2) with 3 zeros,
    beta ~ U(-1, 1), phi = 1, AUTO with create_ex(min_k = 1)."""
    rng = np.random.default_rng(20261203)
    shapes = []
    for g in range(24):
        m, n = (int(np.exp(rng.uniform(np.log(16), np.log(300)))) for _ in range(2))
        k = int(np.exp(rng.uniform(0, np.log(700))))
        a = 0.0 if g in (3, 11, 19) else float(rng.uniform(-2, 2))
        shapes.append((m, n, k, a, float(rng.uniform(-1, 1))))
    shapes[5] = (40, 33, 20, 1.0, 0.0)   # k in (16, 32)
    case = Case(shapes, 7, phi=1.0)
    say("ragged auto")
    rc, st = run(case, G.PATH_AUTO, CFG_AUTO, min_k=1)
    assert rc == 0
    check_case(case, G.PATH_AUTO, CFG_AUTO, st, O.REPAIR_ON)


def test_hard_numerics_nan_inf_and_repair():
    """Config-5 family, reduced: (U-0.5)exp(4Z), 0.1% NaN/Inf entries, repair ON (AUTO)."""
    case = Case([(96, 80, 256)] * 4 + [(64, 64, 3000)], 20261205, phi=4.0)
    rng = np.random.default_rng(5)
    for h in case.hp:
        for arr, rows, cols, ld in ((h.A, h.m, h.k, h.lda), (h.B, h.k, h.n, h.ldb)):
            nbad = max(1, rows * cols // 1000)
            r = rng.integers(0, rows, nbad)
            c = rng.integers(0, cols, nbad)
            arr[r + c * ld] = rng.choice([np.nan, np.inf, -np.inf], nbad)
    case.alloc()
    say("hard numerics EMU_GROUPED repair ON")
    cfg = G.Config(0, 1e-15, 1, G.REPAIR_ON)
    rc, st = run(case, G.PATH_EMU_GROUPED, cfg)
    assert rc == 0
    tot = check_case(case, G.PATH_EMU_GROUPED, cfg, st, O.REPAIR_ON)
    assert tot[3] > 0 and tot[2] > 0
    say("hard numerics AUTO")
    rc, st = run(case, G.PATH_AUTO, CFG_AUTO)
    assert rc == 0
    check_case(case, G.PATH_AUTO, CFG_AUTO, st, O.REPAIR_ON)


@pytest.mark.parametrize("sched", ["dispatch", "persistent", "rowmajor"])
@pytest.mark.parametrize("kernel", ["large", "general"])
def test_nonfinite_tiles_skipped(kernel, sched):
    """INT8 GEMM tiles whose rows (or columns) are all non-finite are not computed by the
    dispatched kernels (every entry takes the safety fallback; on packed and, with
    GGEMM_PACKED_MAX_KP=0, on row-major residues); the persistent kernels compute
    them.  Either way the bits and counters are the oracle's: a problem with a non-finite value
    in every A row, one whose first 256 B columns are non-finite (later columns finite), one whose
    first 256 A rows are non-finite, a short-k problem with every row non-finite (below the
    check's stage count), and a finite problem."""
    case = Case([(300, 200, 400), (260, 300, 300), (512, 96, 500), (100, 90, 100), (128, 128, 256)],
                20261206, phi=2.0)
    rng = np.random.default_rng(6)
    bad = [np.nan, np.inf, -np.inf]

    def spoil_rows(h, rows):   # one non-finite value in each given row of A
        for i in rows:
            h.A[i + rng.integers(0, h.k) * h.lda] = bad[i % 3]

    spoil_rows(case.hp[0], range(300))
    for j in range(256):   # one non-finite value in each of the first 256 columns of B
        h = case.hp[1]
        h.B[rng.integers(0, h.k) + j * h.ldb] = bad[j % 3]
    spoil_rows(case.hp[2], range(256))
    spoil_rows(case.hp[3], range(100))
    case.alloc()
    say(f"non-finite tiles, {kernel} kernel, {sched}")
    run_kernel(case, kernel, **SCHED_ENV[sched])
    say("non-finite tiles, default kernel, repair ON")
    cfg = G.Config(0, 1e-15, 1, G.REPAIR_ON)
    rc, st = run(case, G.PATH_EMU_GROUPED, cfg)
    assert rc == 0
    tot = check_case(case, G.PATH_EMU_GROUPED, cfg, st, O.REPAIR_ON)
    assert tot[3] == 300 * 200 + 256 * 260 + 256 * 96 + 100 * 90


def test_compacted_tiles():
    """Products with NaN / Inf rows and columns in the large-tile kernel on packed residues compute
    only their finite rows x finite columns, in tiles over prep's finite-row and finite-column lists
    dealt to every s-th unit: the bits and counters equal the oracle's and those of a handle that
    computes every tile (GGEMM_COMPACT=0).  Lists of 2 x 2 tiles over a 3 x 3 grid with m, n not
    multiples of 4 (the lists' padding bytes), exactly 257 finite rows (a one-row second tile
    row), 4 x 4 tiles filling a 5 x 5 grid, no finite row, a finite product, and kp = 4000 (a
    half last k-block) with alpha != 1, beta != 0."""
    shapes = [(601, 523, 300, 1.0, 0.0), (300, 700, 130, -1.5, 0.5), (1030, 1100, 200, 1.0, 0.0),
              (512, 512, 64, 1.0, 0.0), (256, 256, 96, 1.0, 0.0), (700, 300, 4000, 2.0, 0.25)]
    rates = [(0.55, 0.5), (43, 0.3), (0.1, 0.1), (1.0, 0.0), (0.0, 0.0), (0.5, 0.5)]
    case = Case(shapes, 20261290, phi=2.0)
    rng = np.random.default_rng(90)
    bad = [np.nan, np.inf, -np.inf]

    def spoiled(count, rate):
        if isinstance(rate, float):
            return [x for x in range(count) if rng.random() < rate]
        return sorted(rng.choice(count, rate, replace=False).tolist())

    for h, (rr, cr) in zip(case.hp, rates):
        for i in spoiled(h.m, rr):
            h.A[i + int(rng.integers(0, h.k)) * h.lda] = bad[i % 3]
        for j in spoiled(h.n, cr):
            h.B[int(rng.integers(0, h.k)) + j * h.ldb] = bad[j % 3]
    case.alloc()
    outs = []
    for env in ({}, {"GGEMM_COMPACT": "0"}):
        say(f"compacted tiles, large kernel, {env}")
        outs.append(run_kernel(case, "large", **env))
    for a, b in zip(*outs):
        assert same_bits(a, b)


def test_tail_workgroups_mixed_units():
    """The 256 x 256 kernel's tail workgroups over more units than compute units (four finite
    768 x 768 x 512 products, 9 tiles x 16 planes each, so every workgroup runs a chain of units,
    the next unit's stages issued before the epilogue), with a product with NaN / Inf rows and
    columns among them (compacted tiles and units without one between finite tiles) and a short
    finite product: bits and counters equal the oracle's and those of one workgroup per tile
    (GGEMM_COMPACT=0)."""
    shapes = [(768, 768, 512, 1.0, 0.0)] * 4 + [(600, 520, 300, -1.0, 0.5), (512, 512, 64, 1.0, 0.0)]
    case = Case(shapes, 20261291, phi=1.0)
    rng = np.random.default_rng(91)
    bad = [np.nan, np.inf, -np.inf]
    h = case.hp[4]
    for i in range(h.m):
        if rng.random() < 0.6:
            h.A[i + int(rng.integers(0, h.k)) * h.lda] = bad[i % 3]
    for j in range(h.n):
        if rng.random() < 0.5:
            h.B[int(rng.integers(0, h.k)) + j * h.ldb] = bad[j % 3]
    case.alloc()
    outs = []
    for env in ({}, {"GGEMM_COMPACT": "0"}):
        say(f"tail workgroups, mixed units, {env}")
        outs.append(run_kernel(case, "large", **env))
    for a, b in zip(*outs):
        assert same_bits(a, b)


def env_handle(case, min_k=None, **env):
    """A handle created with environment variables set (read at creation)."""
    saved = dict(os.environ)
    os.environ.update(env)
    try:
        return G.Handle(max(len(case.hp), 1), *case.sizes(), min_k=min_k)
    finally:
        os.environ.clear()
        os.environ.update(saved)


@pytest.mark.parametrize("form", ["auto", "dense", "blocks", "list"])
@pytest.mark.parametrize("chains", [True, False])
@pytest.mark.parametrize("k", [5, 16, 17, 40, 333])
def test_dense_and_sparse_dot_forms(k, chains, form):
    """The dot-product pass's forms against the oracle's chains, bit for bit, COUNT and ON: tiles
    whose NaN / Inf rows and columns put more than a quarter of their entries on the safety fallback
    (dense form: k-chunks with a partial last chunk for k % 8 != 0 and a single partial chunk for
    k < 8), tiles with a few such rows (compact form, or per block), and repairs scattered over clean
    tiles (compact form, or the per-workgroup list); ragged m, n, alpha != 1, beta != 0.  chains: the
    safety entries run their fma chains (GGEMM_SAFETY_CHAINS=1), else they are decided from prep's
    non-finite summaries.  form (GGEMM_DOT_FORM): the automatic choice, or every flagged tile dense,
    per-block and listed entries only, listed entries only (more than the list holds: per-lane
    chains)."""
    shapes = [(70, 130, k, -1.5, 0.75), (130, 70, k, 2.0, -0.5), (64, 64, k, 1.0, 0.0), (200, 17, k, 0.5, 1.0)]
    case = Case(shapes, 20261216 + k, phi=3.0)
    rng = np.random.default_rng(k)
    h = case.hp[0]          # dense: every fifth row of A and every seventh column of B
    for r in range(0, h.m, 5):
        h.A[r + (k // 2) * h.lda] = np.nan
    for c in range(0, h.n, 7):
        h.B[(k - 1) + c * h.ldb] = np.inf
    h = case.hp[1]          # per block: two rows
    h.A[3 + 0 * h.lda] = -np.inf
    h.A[100 + (k - 1) * h.lda] = np.nan
    h = case.hp[3]          # dense by columns only
    for c in range(0, h.n, 2):
        h.B[int(rng.integers(0, k)) + c * h.ldb] = np.nan
    case.alloc()
    for mode in (G.REPAIR_COUNT, G.REPAIR_ON):
        say(f"dot forms k={k} mode={mode} chains={chains} form={form}")
        cfg = G.Config(0, 1e-15, 1, mode)
        env = {"GGEMM_SAFETY_CHAINS": "1" if chains else "0"}
        if form != "auto":
            env["GGEMM_DOT_FORM"] = form
        with env_handle(case, min_k=1, **env) as hd:
            rc, st = run(case, G.PATH_EMU_GROUPED, cfg, handle=hd)
        assert rc == 0
        tot = check_case(case, G.PATH_EMU_GROUPED, cfg, st, O.REPAIR_ON if mode == G.REPAIR_ON else O.REPAIR_COUNT)
        assert tot[3] > 0


@pytest.mark.parametrize("kernel", ["auto", "large"])
@pytest.mark.parametrize("k", [3, 150, 1030])
def test_repair_subgrid_dot_pass(k, kernel):
    """Repairs concentrated in a sparse finite sub-grid (the hard config's pattern at reduced size):
    most rows of A and columns of B hold a NaN / Inf and phi = 4 leaves most finite-row x
    finite-column entries uncertified, so the dot pass decides the safety entries from the
    summaries and runs the repairs' chains in the compact form over a tile's few rows and columns.
    Tiles whose crossings are dense defer them to the crossings pass (regions of 2 x 16 tiles, the
    chains in 16 x 16 blocks on the FP64 matrix cores).  ON and COUNT bitwise against the oracle
    with the oracle's counts, and the same bits from a handle whose tiles never defer
    (GGEMM_DOT_FORM=tile).  Shapes: several tiles and regions with short last ones (m = 300, 130),
    a single tile row over 520 and 4200 columns (5 regions), repair rows in half the rows of one tile
    row (m = 64, 1200 columns), and exactly 9 finite rows and 28 finite columns in every tile
    (m = 128, n = 1100: 18 rows x 448 columns of crossings in the first region, 2 x 28 blocks in two
    passes); k below a k-chunk, k % 4 != 0, alpha != 1, beta != 0.  kernel large: the 256 x 256
    INT8 kernel (GGEMM_I8_KERNEL), whose compacted tiles give the finite sub-grid's digits."""
    shapes = [(300, 280, k, -1.5, 0.5), (130, 300, k, 1.0, 0.0), (64, 520, k, 2.0, 1.0), (70, 4200, 40, 1.0, 0.0),
              (64, 1200, 60, 1.0, 0.25), (128, 1100, k, 0.5, 0.0)]
    # rows, columns with NaN / Inf: a rate, or exactly all but (9, 28) per 64-row / 64-column tile
    rates = [(0.85, 0.85), (0.85, 0.85), (0.85, 0.85), (0.85, 0.85), (0.5, 0.875), (9, 28)]
    case = Case(shapes, 20261251 + k, phi=4.0)
    rng = np.random.default_rng(k + 7)
    bad = [np.nan, np.inf, -np.inf]

    def nonfinite(count, rate):
        if isinstance(rate, float):
            return [x for x in range(count) if rng.random() < rate]
        keep = set()
        for t0 in range(0, count, 64):
            w = min(64, count - t0)
            keep.update((t0 + rng.choice(w, min(rate, w), replace=False)).tolist())
        return [x for x in range(count) if x not in keep]

    for h, (rr, cr) in zip(case.hp, rates):
        for i in nonfinite(h.m, rr):
            h.A[i + int(rng.integers(0, h.k)) * h.lda] = bad[i % 3]
        for j in nonfinite(h.n, cr):
            h.B[int(rng.integers(0, h.k)) + j * h.ldb] = bad[j % 3]
    case.alloc()
    for mode in (G.REPAIR_ON, G.REPAIR_COUNT):
        cfg = G.Config(0, 1e-15, 1, mode)
        outs = []
        for form in ("auto", "tile"):
            say(f"repair sub-grid k={k} mode={mode} form={form} kernel={kernel}")
            env = {} if form == "auto" else {"GGEMM_DOT_FORM": "tile"}
            if kernel == "large":
                env["GGEMM_I8_KERNEL"] = "large"
            with env_handle(case, min_k=1, **env) as hd:
                rc, st = run(case, G.PATH_EMU_GROUPED, cfg, handle=hd)
            assert rc == 0
            tot = check_case(case, G.PATH_EMU_GROUPED, cfg, st, O.REPAIR_ON if mode == G.REPAIR_ON else O.REPAIR_COUNT)
            if mode == G.REPAIR_ON:
                assert tot[2] > 1000, tot
            outs.append([case.C(g).copy() for g in range(len(case.hp))])
        for other in outs[1:]:
            for a, b in zip(outs[0], other):
                assert same_bits(a, b)


def _inf_patterns(seed):
    """Problems whose NaN / Inf rows and columns cover each case of the summary evaluation, with
    the full fma chain as the expected value (oracle)."""
    rng = np.random.default_rng(seed)
    shapes = [(40, 36, 50, 1.0, 0.0),        # single-read B columns (k <= 1024), ragged tiles
              (8, 8, 64, 1.0, 0.0),          # overflow bound
              (70, 66, 90, -1.5, 0.5),       # beta != 0, C0 with NaN / Inf
              (20, 24, 1500, 2.0, 0.0)]      # B columns read in chunks (k > 1024)
    case = Case(shapes, seed, phi=1.0)
    inf, nan = np.inf, np.nan
    h = case.hp[0]
    A = lambda i, k: i + k * h.lda
    B = lambda k, j: k + j * h.ldb
    h.A[A(0, 3)] = inf                       # +Inf against b = 0 (NaN) and b < 0 (-Inf)
    h.B[B(3, 0)] = 0.0
    h.B[B(3, 1)] = -2.0
    h.A[A(1, 5)] = inf                       # +Inf and -Inf: NaN where the products' signs differ
    h.A[A(1, 9)] = -inf
    h.A[A(2, 7)] = nan                       # NaN row
    for k in range(10, 30):                  # more infinities than the summary lists: chains
        h.A[A(3, k)] = inf
    h.B[B(np.arange(10, 30), 2)] = np.abs(h.B[B(np.arange(10, 30), 2)]) + 0.5   # +Inf through the chain
    h.A[A(4, np.arange(h.k))] = 0.0          # no finite nonzero entry besides the infinity
    h.A[A(4, 0)] = -inf
    h.B[B(11, 3)] = inf                      # column infinity against a = 0 (NaN) and a = -Inf
    h.A[A(5, 11)] = 0.0
    h.A[A(6, 11)] = -inf
    h.B[B(20, 4)] = nan                      # NaN column
    h.A[A(7, 13)] = inf                      # row and column infinity at the same k
    h.B[B(13, 5)] = -inf
    h.B[B(33, 6)] = -inf                     # column with two infinities of either sign
    h.B[B(40, 6)] = inf
    h = case.hp[1]
    A = lambda i, k: i + k * h.lda
    B = lambda k, j: k + j * h.ldb
    h.A[A(0, np.arange(63))] = 1e300         # finite sum overflows to +Inf before the -Inf: NaN
    h.A[A(0, 63)] = -inf
    h.B[B(np.arange(64), 0)] = 1e10
    h.A[A(1, 0)] = 1e300                     # first product overflows
    h.A[A(1, 63)] = -inf
    h.B[B(0, 1)] = 1e300
    h.B[B(63, 1)] = 1.0
    h.A[A(2, np.arange(63))] = 1e150         # inside the bound: -Inf
    h.A[A(2, 63)] = -inf
    h.B[B(np.arange(64), 2)] = 1e150
    h = case.hp[2]
    for _ in range(40):
        arr, ld, rows, cols = (h.A, h.lda, h.m, h.k) if rng.random() < 0.5 else (h.B, h.ldb, h.k, h.n)
        arr[int(rng.integers(0, rows)) + int(rng.integers(0, cols)) * ld] = rng.choice([inf, -inf, inf, -inf, nan])
    h.C0[int(rng.integers(0, h.m)) + np.arange(h.n) * h.ldc] = rng.choice([nan, inf, -inf, 1.0], h.n)
    h = case.hp[3]
    for c in range(0, h.n, 3):               # infinities past the first 1024 k
        h.B[int(rng.integers(1024, h.k)) + c * h.ldb] = rng.choice([inf, -inf])
    for r in range(0, h.m, 4):
        h.A[r + int(rng.integers(0, h.k)) * h.lda] = rng.choice([inf, -inf])
    case.alloc()
    return case


@pytest.mark.parametrize("N", [0, 18])
def test_safety_entries_from_summaries(N):
    """Safety-fallback entries decided from prep's non-finite summaries equal the oracle's fma
    chains bit for bit (NaN payloads aside) in every repair mode -- zero and NaN factors, infinite
    products of both signs, rows and columns with infinities at the same k, more infinities than a
    summary lists, finite sums that overflow before the infinity and ones inside the bound, beta
    C0 non-finite -- and equal a handle that runs every chain.  N = 18: three-word digits."""
    case = _inf_patterns(20261202 + N)
    outs = {}
    for chains in ("0", "1"):
        for mode, omode in ((G.REPAIR_OFF, O.REPAIR_OFF), (G.REPAIR_COUNT, O.REPAIR_COUNT),
                            (G.REPAIR_ON, O.REPAIR_ON)):
            say(f"summaries N={N} chains={chains} mode={mode}")
            cfg = G.Config(N, 1e-15, 0, mode)
            with env_handle(case, min_k=1, GGEMM_SAFETY_CHAINS=chains) as hd:
                rc, st = run(case, G.PATH_EMU_GROUPED, cfg, handle=hd)
            assert rc == 0
            tot = check_case(case, G.PATH_EMU_GROUPED, cfg, st, omode)
            assert tot[3] > 0
            outs[(chains, mode)] = [case.C(g).copy() for g in range(len(case.hp))]
    for mode in (G.REPAIR_OFF, G.REPAIR_COUNT, G.REPAIR_ON):
        for a, b in zip(outs[("0", mode)], outs[("1", mode)]):
            assert same_bits(a, b)
    h = case.hp[1]   # the overflow cases are NaN, the bounded one -Inf
    C1 = outs[("0", G.REPAIR_ON)][1]
    assert np.isnan(C1[0]) and np.isnan(C1[1 + h.ldc]) and C1[2 + 2 * h.ldc] == -np.inf


def test_edge_cases():
    say("edge: num_problems = 0")
    with G.Handle(4, 64, 64, 64) as h:
        for path in range(7):
            st = G.Stats()
            rc = G.lib().ggemm_grouped_dgemm(h.h, path, C.byref(CFG_EMU), None, 0, C.byref(st))
            assert rc == 0, path
            assert st.num_problems == 0 and st.num_fallback == 0 and st.kernel_launches == 0
    cases = [([(100, 70, 50)], 1.0, 0.0), ([(1, 1, 1)], 1.0, 0.0),
             ([(0, 32, 32), (32, 0, 32), (32, 32, 0), (48, 40, 36), (0, 0, 0)], 1.5, -0.5),
             ([(0, 16, 16), (16, 0, 16)], 1.0, 0.0), ([(33, 31, 1), (65, 3, 31), (5, 129, 97)], -2.0, 1.0)]
    for shapes, a, b in cases:
        case = Case(shapes, 12345 + len(shapes), phi=1.0, alpha=a, beta=b)
        for path, cfg, mode in [(G.PATH_EMU_GROUPED, CFG_EMU, O.REPAIR_COUNT), (G.PATH_AUTO, CFG_AUTO, O.REPAIR_ON)]:
            say(f"edge {shapes} path={path}")
            rc, st = run(case, path, cfg, min_k=1)
            assert rc == 0
            check_case(case, path, cfg, st, mode)
    # beta = 0 must not read C: NaN-filled C0
    case = Case([(40, 24, 72), (17, 33, 5)], 99, phi=1.0)
    for h in case.hp:
        h.C0[:] = np.nan
    case.alloc()
    say("edge beta0 NaN C")
    rc, st = run(case, G.PATH_EMU_GROUPED, CFG_EMU, min_k=1)
    assert rc == 0
    for g in range(2):
        assert np.isfinite(case.C(g).reshape(case.hp[g].n, case.hp[g].ldc)[:, :case.hp[g].m]).all()


@pytest.mark.parametrize("path", [G.PATH_NATIVE_LOOP, G.PATH_NATIVE_GROUPED])
def test_native_paths_gate(path):
    case = Case([(100, 70, 50), (64, 64, 300), (1, 1, 1), (33, 17, 0), (0, 5, 5)], 31, phi=1.0, alpha=1.5, beta=-0.5)
    say(f"native path {path}")
    rc, st = run(case, path, CFG_EMU)
    assert rc == 0
    for g, h in enumerate(case.hp):
        if h.m == 0 or h.n == 0:
            continue
        h.reference()
        gate, _ = h.gate(case.C(g))
        assert gate <= 1.0, (g, gate)
    assert st.kernel_launches == (1 if path == G.PATH_NATIVE_GROUPED else 4)


@pytest.mark.parametrize("path", [G.PATH_NATIVE_LOOP, G.PATH_NATIVE_GROUPED])
@pytest.mark.parametrize("beta", [-0.5, 0.0])
def test_native_tile_sizes_bitwise(path, beta):
    """The native GEMM's 64 x 64 and 128 x 128 tile kernels (forced with GGEMM_F64_TILE) on the
    same ragged group -- partial tiles on both edges, k not a multiple of the 16-deep stage, k = 0
    and empty problems: every output bit equal (each entry takes the same k-ordered MFMA chain at
    either size), each problem within the gamma_n gate of the host reference."""
    shapes = [(300, 200, 77), (128, 128, 16), (129, 257, 300), (1, 1, 1), (33, 17, 0), (0, 5, 5), (260, 140, 1),
              # full tiles of both sizes over several 16-deep stages (the bounds-test-free path), next
              # to partial tiles of the same problem
              (256, 256, 64), (384, 256, 1024), (260, 128, 48)]
    outs = {}
    for tile in ("64", "128"):
        case = Case(shapes, 33, phi=1.0, alpha=1.5, beta=beta)
        say(f"native path {path}, tile {tile}, beta {beta}")
        with kernel_handle(case, None, GGEMM_F64_TILE=tile) as hd:
            rc, st = run(case, path, CFG_EMU, handle=hd)
        assert rc == 0
        outs[tile] = [case.C(g).copy() for g in range(len(shapes))]
        for g, h in enumerate(case.hp):
            if h.m == 0 or h.n == 0:
                continue
            h.reference()
            gate, _ = h.gate(case.C(g))
            assert gate <= 1.0, (tile, g, gate)
    for g in range(len(shapes)):
        assert same_bits(outs["64"][g], outs["128"][g]), f"problem {g} {shapes[g]} differs between tile sizes"


def test_bigk_fallback_and_unsafe():
    """k = 140000 > 131040: AUTO with fallback -> native route counted; allow_fallback = 0 ->
    GGEMM_ERR_UNSAFE (tests/test_grouped.cu:185-231)."""
    case = Case([(4, 4, 140000), (64, 64, 64), (8, 8, 8)], 5, phi=0.5)
    say("bigk fallback")
    rc, st = run(case, G.PATH_AUTO, CFG_AUTO)
    assert rc == 0 and st.num_fallback >= 1
    check_case(case, G.PATH_AUTO, CFG_AUTO, st, O.REPAIR_ON)
    for path in (G.PATH_EMU_GROUPED, G.PATH_AUTO):
        rc, st = run(case, path, G.Config(0, 1e-15, 0, 0))
        assert rc == G.GGEMM_ERR_UNSAFE


def test_capacity_and_argument_errors():
    case = Case([(16, 16, 16)] * 3, 3, phi=0.0)
    say("capacity errors")
    for path in (G.PATH_NATIVE_LOOP, G.PATH_NATIVE_GROUPED, G.PATH_EMU_LOOP, G.PATH_EMU_GROUPED, G.PATH_AUTO):
        with G.Handle(2, 4096, 4096, 4096) as h:
            rc, _ = h.dgemm(path, CFG_AUTO, case.problems())
            assert rc == G.GGEMM_ERR_INVALID
        with G.Handle(8, 100, 100, 100) as h:
            rc, _ = h.dgemm(path, CFG_AUTO, case.problems())
            assert rc == G.GGEMM_ERR_WORKSPACE
    with G.Handle(8, 4096, 4096, 4096) as h:
        for path in (G.PATH_EMU_GROUPED, G.PATH_AUTO):
            for bad in (1, G.MAX_MODULI + 1, -1):
                rc, _ = h.dgemm(path, G.Config(bad, 1e-15, 1, 0), case.problems())
                assert rc == G.GGEMM_ERR_INVALID
            rc, _ = h.dgemm(path, G.Config(0, 1e-15, 1, 7), case.problems())   # repair mode out of range
            assert rc == G.GGEMM_ERR_INVALID
    # k < min_k residue inflation -> WORKSPACE with one diagnostic line
    small = Case([(64, 64, 1)] * 2, 4, phi=0.0)
    with G.Handle(2, 64 * 2, 64 * 2, 64 * 64 * 2) as h:
        rc, _ = h.dgemm(G.PATH_EMU_GROUPED, CFG_EMU, small.problems())
        assert rc == G.GGEMM_ERR_WORKSPACE
    torch.cuda.synchronize()


def test_launch_count_independent_of_group_size():
    launches = []
    for n_probs in (16, 1024):
        case = Case([(32, 32, 32)] * n_probs, 8, phi=0.5)
        say(f"launch count G={n_probs}")
        rc, st = run(case, G.PATH_EMU_GROUPED, CFG_EMU)
        assert rc == 0
        launches.append(st.kernel_launches)
    assert launches[0] == launches[1] == 2 + recon_launches()


@pytest.mark.parametrize("path", [G.PATH_EMU_GROUPED, G.PATH_AUTO, G.PATH_NATIVE_GROUPED])
def test_bitwise_reproducible(path):
    case = Case([(int(m), 256, 512) for m in np.random.default_rng(2).integers(16, 513, 12)], 9, phi=1.0)
    say(f"reproducibility path={path}")
    with G.Handle(len(case.hp), *case.sizes()) as h:
        outs = []
        for _ in range(2):
            case.reset_C()
            rc, _ = h.dgemm(path, CFG_AUTO if path == G.PATH_AUTO else CFG_EMU, case.problems())
            assert rc == 0
            outs.append(np.concatenate([case.C(g) for g in range(len(case.hp))]))
        assert same_bits(outs[0], outs[1])


@pytest.mark.parametrize("pad", [1, 3])
def test_padded_leading_dimensions(pad):
    """Leading dimensions past m / k (lda = ldc = m + pad, ldb = k + pad): columns of C then start at
    any 8-byte offset, so the reconstruct's 128-bit accesses of C (and of the shift arrays, whatever
    m mod 4) read and write unaligned rows; beta != 0, a NaN row and an Inf column, repair ON;
    bitwise against the oracle with equal counters."""
    shapes = [(33, 17, 40), (64, 40, 100), (70, 66, 129), (130, 33, 64), (257, 48, 300)]
    case = Case(shapes, 20261240 + pad, phi=1.0, beta=0.5, pad=pad)
    h = case.hp[1]
    h.A[5 + 7 * h.lda] = np.nan
    h = case.hp[3]
    h.B[10 + 20 * h.ldb] = np.inf
    case.alloc()
    cfg = G.Config(0, 1e-15, 0, G.REPAIR_ON)
    say(f"padded leading dimensions, pad {pad}")
    rc, st = run(case, G.PATH_EMU_GROUPED, cfg)
    assert rc == 0
    check_case(case, G.PATH_EMU_GROUPED, cfg, st, O.REPAIR_ON)
