"""Kernel-level parity of the HIP pipeline (prep -> INT8 GEMM -> reconstruct) against the oracle
and the reference's logged known answers (tests/test_numerics_standalone.cu sections 1-7).

Bar: residue planes, shifts and norm bounds bit-exact; INT8 products bit-exact; reconstructed C
bit-identical to the oracle; repaired / uncertified / safety / non-finite counts equal to the
oracle's and to the reference log."""
import ctypes as C
import json
from pathlib import Path

import numpy as np
import pytest
import torch  # noqa: F401  (imported at collection: the first import on a fresh box is slow)

import ggemm as G
import oracle_lib as O
from gpu_util import WhiteboxRun, read_counters, same_bits, say
from test_oracle import PHIS, SWEEP_SHAPES, _replay_prefix, make_section3, make_section4, make_section5

pytestmark = pytest.mark.gpu
KAT = json.loads((Path(__file__).resolve().parent / "golden" / "numerics_kat.json").read_text())


def _assert_prep_matches_oracle(run, g):
    h = run.hs[g]
    A8, B8, C32, rs, cs = run.planes(g)
    oA8, oB8, ors, ocs, _ = O.oracle_prep(h.m, h.n, h.k, h.N, h.A, h.lda, h.B, h.ldb)
    assert np.array_equal(rs, ors), f"row workspace differs (problem {g})"
    assert np.array_equal(cs, ocs), f"col workspace differs (problem {g})"
    assert np.array_equal(A8, oA8), f"A residues differ (problem {g})"
    assert np.array_equal(B8, oB8), f"B residues differ (problem {g})"
    return A8, B8, C32


def test_prep_residues_bit_exact_section1():
    """Section 1 data (37 x 29 x 100, phi = 2) for N = 1, 8, 13, 20 (log lines 18-21)."""
    O.katgen().katgen_seed(12345, 0)
    for N in (1, 8, 13, 20):
        h = O.HostProb(37, 29, 100, 5, 2.0, N=N).make()
        say(f"prep section1 N={N}")
        run = WhiteboxRun([h])
        run.prep()
        _assert_prep_matches_oracle(run, 0)
        read_counters()


def test_prep_special_rows_and_int8_products():
    """Rescale path (2^-700 / 2^650 magnitudes), zero rows/columns, NaN/Inf vectors, k not a
    multiple of 32; then the INT8 products of every plane against the oracle's int64 products."""
    rng = np.random.default_rng(3)
    hs = []
    for (m, n, k, N, mode) in [(33, 17, 45, 15, 0), (64, 48, 300, 18, 1), (40, 33, 129, 14, 2), (20, 30, 1, 8, 3),
                               (5, 64, 2048, 16, 4)]:
        h = O.HostProb(m, n, k, 3, 1.0, N=N)
        for c in range(k):
            h.A[c * h.lda: c * h.lda + m] = (rng.random(m) - 0.5) * np.exp(rng.standard_normal(m))
        for c in range(n):
            h.B[c * h.ldb: c * h.ldb + k] = (rng.random(k) - 0.5) * np.exp(rng.standard_normal(k))
        if mode == 1:
            h.A[:] = np.ldexp(h.A, -700)
            h.B[:] = np.ldexp(h.B, 650)
        elif mode == 2:
            h.A[3 + np.arange(k) * h.lda] = 0.0
            h.B[np.arange(k) + 5 * h.ldb] = 0.0
        elif mode == 4:
            h.A[2 + 100 * h.lda] = np.nan
            h.B[7 + 9 * h.ldb] = -np.inf
        hs.append(h)
    say("prep special rows")
    read_counters()
    run = WhiteboxRun(hs)
    run.prep()
    for g, h in enumerate(hs):
        A8, B8, _ = _assert_prep_matches_oracle(run, g)
    assert read_counters().nonfinite_vectors == 2
    say("int8 products of the prepped planes")
    run.gemm()
    for g, h in enumerate(hs):
        A8, B8, C32, _, _ = run.planes(g)
        kp = O.kp_of(h.k)
        for l in range(h.N + 1):
            ref = O.oracle_i8_gemm(h.m, h.n, kp, A8[l * h.m * kp:(l + 1) * h.m * kp],
                                   B8[l * h.n * kp:(l + 1) * h.n * kp])
            assert np.array_equal(C32[l * h.m * h.n:(l + 1) * h.m * h.n], ref), (g, l)


def _gpu_vs_oracle(h, mode):
    run = WhiteboxRun([h])
    read_counters()
    run.run(mode)
    c = read_counters()
    Cg = run.C(0)
    Co, cnt = h.emulate(mode)
    return run, c, Cg, Co, cnt


def test_kat_sweep_through_gpu():
    """Log lines 23-340: every (shape, phi, N) repaired count from the GPU pipeline equals the
    logged count, and C is bit-identical to the oracle."""
    _replay_prefix()
    ci = 0
    for sh in SWEEP_SHAPES:
        for phi in PHIS:
            exp = KAT["sweep"][ci]
            ci += 1
            base = O.HostProb(sh[0], sh[1], sh[2], 3, phi).make()
            for N in range(8, 21):
                h = O.HostProb(sh[0], sh[1], sh[2], 3, phi, N=N)
                h.A, h.B, h.C0 = base.A, base.B, base.C0
                say(f"kat sweep {sh} phi={phi} N={N}")
                run, c, Cg, Co, cnt = _gpu_vs_oracle(h, G.OZ2_REPAIR_ON)
                assert c.repaired == exp["rep"][str(N)], (sh, phi, N, c.repaired)
                assert c.repaired == cnt[2] and c.safety_fallback == cnt[3] and c.uncertified == 0
                assert same_bits(Cg, Co), (sh, phi, N)


def test_kat_grouped_nonfinite_and_modes():
    """Log lines 343-357: 9-problem grouped launch -> 6688 repairs; NaN row + Inf column ->
    non-finite counter 2; 64 x 16^3 phi=2 N=15 -> 899 uncertified (COUNT) == 899 repaired (ON),
    OFF bitwise equal to COUNT."""
    hs, h4 = make_section4()
    say("kat grouped 9 problems")
    run = WhiteboxRun(hs)
    read_counters()
    run.run(G.OZ2_REPAIR_ON)
    c = read_counters()
    assert c.repaired == KAT["grouped_repaired"]
    for g, h in enumerate(hs):
        Co, _ = h.emulate(G.OZ2_REPAIR_ON)
        assert same_bits(run.C(g), Co), g
    say("kat non-finite")
    run, c, Cg, Co, cnt = _gpu_vs_oracle(h4, G.OZ2_REPAIR_ON)
    assert c.nonfinite_vectors == KAT["nonfinite_counter"]
    assert c.safety_fallback == cnt[3] > 0
    assert same_bits(Cg, Co)
    hs5 = make_section5()
    outs, cnts = {}, {}
    for mode in (G.OZ2_REPAIR_OFF, G.OZ2_REPAIR_COUNT, G.OZ2_REPAIR_ON):
        say(f"kat repair mode {mode}")
        run = WhiteboxRun(hs5)
        read_counters()
        run.run(mode)
        cnts[mode] = read_counters()
        outs[mode] = np.concatenate([run.C(g) for g in range(len(hs5))])
        ref = np.concatenate([h.emulate(mode)[0] for h in hs5])
        assert same_bits(outs[mode], ref), mode
    assert cnts[G.OZ2_REPAIR_COUNT].uncertified == KAT["repair_modes"]["uncertified"]
    assert cnts[G.OZ2_REPAIR_ON].repaired == KAT["repair_modes"]["repaired"]
    assert same_bits(outs[G.OZ2_REPAIR_OFF], outs[G.OZ2_REPAIR_COUNT])


def test_blas_edge_semantics():
    """Section 6: alpha = 0 with NaN in A -> beta C0 exactly; NaN alpha with a zero row -> NaN;
    Inf C0 with beta != 0 -> non-finite without repair; no safety fallback counted."""
    O.katgen().katgen_seed(777, 0)
    h0 = O.HostProb(20, 10, 50, 0, 1.0, 0.0, 0.5, 15).make()
    h0.A[3] = np.nan
    h1 = O.HostProb(20, 10, 50, 0, 1.0, np.nan, 0.0, 15).make()
    h1.A[4 + np.arange(50) * h1.lda] = 0.0
    h2 = O.HostProb(20, 10, 50, 0, 1.0, 1.0, 1.0, 15).make()
    h2.C0[7] = np.inf
    say("blas edge cases")
    run = WhiteboxRun([h0, h1, h2])
    read_counters()
    run.run(G.OZ2_REPAIR_ON)
    c = read_counters()
    C0 = run.C(0).reshape(h0.n, h0.ldc)[:, :h0.m]
    assert np.array_equal(C0, 0.5 * h0.C0.reshape(h0.n, h0.ldc)[:, :h0.m])
    assert np.isnan(run.C(1).reshape(h1.n, h1.ldc)[:, :h1.m]).all()
    assert not np.isfinite(run.C(2)[7])
    assert c.safety_fallback == 0
    for g, h in enumerate([h0, h1, h2]):
        Co, _ = h.emulate(G.OZ2_REPAIR_ON)
        assert same_bits(run.C(g), Co), g


def test_prep_split_invariance():
    """Section 7: forced prep K-split factors give bit-identical planes, workspace and C."""
    O.katgen().katgen_seed(4242, 0)
    hs = [O.HostProb(16, 40, 3000, 1, 2.0, N=15).make(), O.HostProb(37, 9, 1000, 3, 1.0, -1.5, 0.5, 20).make(),
          O.HostProb(70, 33, 129, 2, 4.0, N=9).make(), O.HostProb(5, 64, 2048, 0, 0.5, 1.0, 1.0, 16).make()]
    hs[3].A[2 + 100 * hs[3].lda] = np.nan
    ref = None
    try:
        for S in (1, 2, 3, 7, 16, 64):
            say(f"prep split S={S}")
            G.lib().oz2_debug_force_prep_split(S)
            run = WhiteboxRun(hs)
            run.run(G.OZ2_REPAIR_ON)
            cur = []
            for g in range(len(hs)):
                cur.extend(run.planes(g))
                cur.append(run.C(g))
            if ref is None:
                ref = cur
            else:
                for a, b in zip(ref, cur):
                    assert np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8)), S
    finally:
        G.lib().oz2_debug_force_prep_split(0)
        read_counters()


def _chain_operands(rng, kind, waves, K):
    """Per wave a 16 x K block of A and a K x 16 block of B (column-major) of one input class."""
    def wide(shape, lo, hi):
        v = np.ldexp(rng.uniform(1.0, 2.0, shape), rng.integers(lo, hi + 1, shape))
        return np.where(rng.random(shape) < 0.5, -v, v)

    A = wide((waves, K, 16), -60, 60)   # [w][k][i]
    B = wide((waves, 16, K), -60, 60)   # [w][j][k]
    if kind == "cancellation":          # each chain's later products undo its first one's rounding
        A = wide((waves, K, 16), -2, 2)
        B = wide((waves, 16, K), -2, 2)
        A[:, 1::2, :] = -A[:, 0::2, :] * (1.0 + np.ldexp(rng.integers(-3, 4, A[:, 1::2, :].shape), -52))
        A[:, 2::4, :] = np.ldexp(A[:, 2::4, :], -rng.integers(20, 60, A[:, 2::4, :].shape))
    elif kind == "subnormal":
        A = wide((waves, K, 16), -540, -500)
        B = wide((waves, 16, K), -540, -500)
    elif kind == "zeros":               # signed zeros and products that underflow to -0 / +0
        A = wide((waves, K, 16), -560, -520)
        B = wide((waves, 16, K), -540, -500)
        A = np.where(rng.random(A.shape) < 0.25, np.where(rng.random(A.shape) < 0.5, -0.0, 0.0), A)
        B = np.where(rng.random(B.shape) < 0.25, np.where(rng.random(B.shape) < 0.5, -0.0, 0.0), B)
    elif kind == "overflow":            # +-Inf and NaN factors, sums past the largest double
        A = wide((waves, K, 16), 500, 512)
        B = wide((waves, 16, K), 500, 512)
        r = rng.integers(0, 16, A.shape)
        A = np.where(r == 0, np.inf, np.where(r == 1, -np.inf, np.where(r == 2, np.nan, A)))
    return A, B


@pytest.mark.parametrize("kind", ["wide", "cancellation", "subnormal", "zeros", "overflow"])
@pytest.mark.parametrize("steps", [1, 3, 64])
def test_fp64_mfma_chains_are_sequential_fmas(kind, steps):
    """The dot pass's crossings pass computes repair chains with v_mfma_f64_16x16x4f64: its four
    k-steps must be four sequential IEEE fmas in k order, so that a block's chains equal the
    oracle's fp64_dot (one fma chain in ascending k from +0) bit for bit.  Inputs that tell the
    orders apart (one rounding of the exact sum, or k descending, differ from the chain in a
    large share of these cases): wide exponents, cancellation, subnormal products, signed zeros
    and underflow to zero, infinities and NaN with overflowing sums; k = 4, 12, 256."""
    rng = np.random.default_rng(20261202 + steps + 100 * len(kind))
    waves, K = 64, 4 * steps
    A, B = _chain_operands(rng, kind, waves, K)
    # lane l of step t holds A[i = l % 16][k = 4 t + l / 16] and B[k][j = l % 16]
    l = np.arange(64)
    kk = 4 * np.arange(steps)[:, None] + (l // 16)[None, :]               # [t][l]
    Al = A[:, kk, (l % 16)[None, :]]                                      # [w][t][l]
    Bl = B[:, (l % 16)[None, :], kk]
    dA = torch.from_numpy(np.ascontiguousarray(Al)).cuda()
    dB = torch.from_numpy(np.ascontiguousarray(Bl)).cuda()
    dD = torch.full((waves * 256,), 7.0, dtype=torch.float64, device="cuda")
    say(f"mfma chains {kind} steps={steps}")
    assert G.lib().oz2_mfma_f64_chains(dA.data_ptr(), dB.data_ptr(), dD.data_ptr(), waves, steps, None) == 0
    D = dD.cpu().numpy().reshape(waves, 64, 4)
    lib = O.oracle()
    want = np.empty_like(D)
    alt = 0
    for w in range(waves):
        Aw = np.ascontiguousarray(A[w])          # [k][i]: row i at Aw + i with stride 16
        Bw = np.ascontiguousarray(B[w])          # [j][k]: column j contiguous
        for ln in range(64):
            for e in range(4):
                i, j = ln // 16 + 4 * e, ln % 16
                want[w, ln, e] = lib.oz2o_fp64_dot(K, C.c_void_p(Aw[:, i:].ctypes.data), 16,
                                                   C.c_void_p(Bw[j].ctypes.data))
                with np.errstate(all="ignore"):   # another order: must differ sometimes
                    exact = float(np.sum(Aw[:, i] * Bw[j]))
                alt += not same_bits(exact, want[w, ln, e])
    assert same_bits(D, want), f"{kind}: {np.sum(~((D == want) | (np.isnan(D) & np.isnan(want))))} chains differ"
    if steps > 1 and kind in ("wide", "cancellation", "subnormal"):
        assert alt > 0, "the inputs do not tell the summation orders apart"
