"""The residue arithmetic of the MI355X prep kernel (coding-basic-hw-2_amd/csrc/prep.hip), checked
on the CPU against exact integer arithmetic (no GPU).

The kernel forms sym(x mod p) of an integer-valued double x with |x| <= T_N from 32-bit digit words
(exact floor splits), byte dot products against per-modulus weights and one float32 fma that
floors (u + h) / p.  These tests emulate each step bit for bit:
  * the float floor is checked exhaustively over every u the dot products can produce and every
    modulus (a float32 fma is a float64 sum of exact terms, rounded once to float32 here);
  * the whole chain is checked against Python integers on edge values (0, +-1, word boundaries,
    powers of two, +-T_N) and random integers of every size up to T_20, for both word layouts;
  * the two-word layout's precondition T_N < 1.5 2^62 holds exactly for N <= 16.
The GPU tests then compare the kernel's bytes with the oracle's.
"""
import math

import numpy as np
import pytest

MODULI = [256, 255, 253, 251, 247, 239, 233, 229, 227, 223, 217, 211, 199, 197, 193, 191, 181, 179, 173, 167]
SHIFT = 2048   # the float constant's integer offset; 2048 p = 0 (mod 256)


def _consts(p):
    ipf = np.float32(1.0 / p)
    cf = np.float32((p // 2 + 0.5) / p + SHIFT)
    return ipf, cf


def _sym(r, p):
    h = p // 2
    r %= p
    return r - p if r > p - 1 - h else r


def _T(N):
    P = math.prod(MODULI[:N])
    return math.sqrt(P * 0.5 * (1.0 - 2.0 ** -20)) * (1.0 - 2.0 ** -40)


def _floor_q(u, p):
    """trunc(fmaf(u, ipf, cf)) on int64 arrays u: exact float64 sum, one rounding to float32."""
    ipf, cf = _consts(p)
    v = (u.astype(np.float64) * np.float64(ipf) + np.float64(cf)).astype(np.float32)
    return np.trunc(v).astype(np.int64)


@pytest.mark.parametrize("p", MODULI)
def test_float_floor_exhaustive(p):
    # unsigned words give [0, 8 * 255^2], the signed word [-4 * 128 * 127, 4 * 128^2]: every u of
    # both layouts lies in [-2^16, 2^19 + 2^16)
    u = np.arange(-(1 << 16), (1 << 19) + (1 << 16), dtype=np.int64)
    q = _floor_q(u, p)
    h = p // 2
    assert np.array_equal(q - SHIFT, np.floor_divide(u + h, p))
    r = u - q * p
    # r = sym(u mod p) - 2048 p, whose low byte is sym(u mod p)'s
    assert np.array_equal((r & 0xFF), ((np.floor_divide(u + h, p) * -p + u) & 0xFF))
    assert np.all((r + SHIFT * p >= -h) & (r + SHIFT * p <= p - 1 - h))


def _weights(p, q=1):
    e = [(q * pow(2, 8 * i, p)) % p for i in range(12)]
    return e   # unsigned weights; signed ones are _sym(e, p)


def _digits(x, wide):
    """The kernel's digit words of an integer-valued double x: exact float64 floor splits."""
    h = math.floor(x * 2.0 ** -32)
    lo = int(x - h * 2.0 ** 32)   # exact: the difference is an integer in [0, 2^32)
    words = [lo]
    if wide:
        t = math.floor(h * 2.0 ** -32)
        words.append(int(h - t * 2.0 ** 32))
        h = t
    H = (int(h) + 0x80808080) & 0xFFFFFFFF
    words.append(H ^ 0x80808080)
    for w in words:
        assert 0 <= w < 1 << 32
    return words


def _residue_byte(x, p, q, wide):
    w = _digits(x, wide)
    e = _weights(p, q)
    ub = lambda word, i: (word >> (8 * i)) & 0xFF
    sb = lambda word, i: ((word >> (8 * i)) & 0xFF) - 256 * (((word >> (8 * i)) & 0xFF) >= 128)
    u = sum(ub(w[0], i) * e[i] for i in range(4))
    if wide:
        u += sum(ub(w[1], i) * e[4 + i] for i in range(4))
        u += sum(sb(w[2], i) * _sym(e[8 + i], p) for i in range(4))
    else:
        u += sum(sb(w[1], i) * _sym(e[4 + i], p) for i in range(4))
    assert -(1 << 16) <= u < (1 << 19) + (1 << 16)
    qq = int(_floor_q(np.array([u]), p)[0])
    return (u - qq * p) & 0xFF


def _edge_values(T):
    vals = [0.0, -0.0, 1.0, -1.0, 255.0, -255.0, 256.0, -256.0]
    for b in (31, 32, 33, 52, 53, 54, 62, 63, 64, 65, 76):
        for v in (2.0 ** b, 2.0 ** b - 1, 2.0 ** b + 2 ** max(0, b - 52)):
            if v <= T:
                vals += [v, -v]
    Tf = math.floor(T)
    vals += [float(Tf), -float(Tf)]
    return vals


@pytest.mark.parametrize("N", [2, 8, 14, 15, 16, 17, 20])
def test_residue_chain_matches_integers(N):
    T = _T(N)
    wide = not (T < 1.5 * 2.0 ** 62)
    rng = np.random.default_rng(N)
    xs = _edge_values(T)
    top = int(math.floor(math.log2(T)))
    for b in range(0, top + 1, 3):   # random integers of every size, exactly representable
        for _ in range(6):
            m = int(rng.integers(1 << 52, 1 << 53))
            v = math.ldexp(m, b - 52) if b >= 52 else float(m >> (52 - b))
            v = math.floor(v)
            if v <= T:
                xs += [v, -v]
    for x in xs:
        xi = int(x)
        for l in range(N):
            p = MODULI[l]
            for q in (1, 1 + (l * 7) % (p - 1)):   # plain and a folded multiplier
                want = _sym(q * xi, p) & 0xFF
                assert _residue_byte(x, p, q, wide) == want, (N, x, p, q, wide)
                if not wide:   # the three-word layout is valid for every N
                    assert _residue_byte(x, p, q, True) == want, (N, x, p, q)


def test_two_word_layout_range():
    # two words: |x| <= T_N and x + 2^32 H-bias must not wrap: T_N < 1.5 2^62 exactly for N <= 16
    assert [N for N in range(1, 21) if _T(N) < 1.5 * 2.0 ** 62] == list(range(1, 17))
    assert _T(20) < 2.0 ** 77


# ------------------------------------------------------------------- INT8 GEMM epilogue (i8gemm.hip)
def _epi_params(p, kp):
    mc = -(-(1 << 32) // p)
    if kp <= 32768:
        return mc, p * -(-(1 << 29) // p), True
    return mc, p * -(-(1 << 31) // p), False


def _epi_byte(c, p, kp):
    """The epilogue's C mod p from the int32 product c (uint32 / int32 wrap emulated)."""
    mc, bias, acc = _epi_params(p, kp)
    u = (c + bias) & 0xFFFFFFFF
    q = (u * mc) >> 32
    if acc:
        assert q < 1 << 23 and u < (1 << 31)   # 24-bit multiply-add operand, non-negative int32 accumulator
        r = u - q * p
    else:
        r = (u - q * p) & 0xFFFFFFFF
        r = r - (1 << 32) if r >= 1 << 31 else r
    assert -p <= r < p
    return min(r & 0xFFFFFFFF, (r + p) & 0xFFFFFFFF)


@pytest.mark.parametrize("kp", [32, 1024, 32768, 32800, 131040])
def test_gemm_epilogue_residue(kp):
    cmax = 128 * 128 * kp   # |C| <= 128^2 kp for residues in [-128, 127]
    rng = np.random.default_rng(kp)
    for p in MODULI:
        cs = set(int(v) for v in rng.integers(-cmax, cmax + 1, 2000))
        for base in (0, cmax, -cmax, 1 << 20, -(1 << 20)):
            for d in range(-2 * p, 2 * p + 1):
                if -cmax <= base + d <= cmax:
                    cs.add(base + d)
        for c in cs:
            assert _epi_byte(c, p, kp) == c % p, (c, p, kp)
