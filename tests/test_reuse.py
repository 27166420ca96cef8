"""Operand reuse host pass through the C ABI (include/ggemm_reuse.h), on the CPU.

The cases of tests/test_operand_reuse.cu:25-121: operand keys (pointer, ld, rows, k), first-
appearance numbering and representatives, EXACT_N vs PROMOTE (component maximum of N), ignored
problems, capacity errors, repeated builds on one arena, and the modelled prep bytes.  Pointers
are fake addresses (never dereferenced)."""
import ctypes as C

import pytest

import ggemm as G


def P(x):
    return x * 4096


def mk(A, lda, B, ldb, m, n, k):
    return G.Problem(m, n, k, A, lda, B, ldb, 0, m, 1.0, 0.0)


class Arena:
    def __init__(self, cap):
        self.a = C.c_void_p()
        self.rc = G.lib().reuse_arena_create(cap, C.byref(self.a))

    def build(self, probs, nmod, policy=G.REUSE_PROMOTE):
        self.probs = G.problems_array(probs)
        self.nm = (C.c_int * max(len(nmod), 1))(*nmod)
        self.plan = G.lib().build_operand_reuse(self.a, self.probs, len(probs), self.nm, policy)
        return self.plan

    def bytes(self):
        b, a = G.ReuseBytes(), G.ReuseBytes()
        G.lib().operand_reuse_bytes(C.byref(self.plan), self.probs, self.nm, C.byref(b), C.byref(a))
        return b, a

    def close(self):
        G.lib().reuse_arena_destroy(self.a)


@pytest.fixture
def arena():
    a = Arena(64)
    assert a.rc == G.REUSE_OK and G.lib().reuse_arena_capacity(a.a) == 64
    yield a
    a.close()


def test_no_sharing(arena):
    pr = [mk(P(1000 + g), 64, P(2000 + g), 64, 64, 32, 64) for g in range(50)]
    r = arena.build(pr, [6] * 50)
    assert r.status == G.REUSE_OK
    assert (r.num_ua, r.num_ub, r.num_promoted, r.num_emu) == (50, 50, 0, 50)
    for g in range(50):
        assert (r.prob_a[g], r.prob_b[g], r.eff_nmod[g]) == (g, g, 6)
    b, a = arena.bytes()
    assert (b.prep_read, b.prep_write, b.ws_A8) == (a.prep_read, a.prep_write, a.ws_A8)


def test_all_share_A(arena):
    # tensor parallel: one A, B split into column blocks
    pr = [mk(P(1), 512, P(100 + g), 256, 512, 128 + g, 256) for g in range(8)]
    r = arena.build(pr, [7] * 8)
    assert (r.num_ua, r.num_ub) == (1, 8)
    assert (r.ua_rep[0], r.ua_nmod[0]) == (0, 7)
    for g in range(8):
        assert (r.prob_a[g], r.prob_b[g], r.eff_nmod[g]) == (0, g, 7)
    b, a = arena.bytes()
    m, k, kp = 512.0, 256.0, 256.0
    assert b.prep_read - a.prep_read == 7 * 16 * m * k
    assert b.prep_write - a.prep_write == 7 * (7 * m * kp + 4 * m)
    assert b.ws_A8 == 8 * a.ws_A8


def test_lora(arena):
    # two token batches x three adapters; adapters shared too
    pr = [mk(P(10 + x), 128, P(50 + a), 4096, 128, 16, 4096) for x in range(2) for a in range(3)]
    r = arena.build(pr, [8] * 6)
    assert (r.num_ua, r.num_ub) == (2, 3)
    for g in range(6):
        assert (r.prob_a[g], r.prob_b[g]) == (g // 3, g % 3)
    assert (r.ua_rep[1], r.ub_rep[2]) == (3, 2)


def test_same_pointer_different_key(arena):
    pr = [mk(P(7), 256, P(8), 64, 128, 32, 64),
          mk(P(7), 512, P(8), 128, 128, 32, 64),   # same pointers, other lda / ldb
          mk(P(7), 256, P(8), 64, 64, 32, 64),     # other m: A not shared, B shared
          mk(P(7), 256, P(8), 64, 128, 32, 32),    # other k: nothing shared
          mk(P(7), 256, P(8), 64, 128, 16, 64)]    # A key of #0, other n: A shared, B not
    r = arena.build(pr, [5] * 5)
    assert (r.num_ua, r.num_ub) == (4, 4)
    assert r.prob_a[0] != r.prob_a[1] and r.prob_b[0] != r.prob_b[1]
    assert r.prob_a[0] != r.prob_a[2] and r.prob_b[0] == r.prob_b[2]
    assert r.prob_a[0] != r.prob_a[3] and r.prob_b[0] != r.prob_b[3]
    assert r.prob_a[0] == r.prob_a[4] and r.prob_b[0] != r.prob_b[4]


def test_different_N_promote_and_exact(arena):
    # P0 (A0, B0, N=3), P1 (A0, B1, 5), P2 (A1, B1, 2), P3 (A2, B2, 4), P4 not emulated
    pr = [mk(P(1), 64, P(11), 64, 64, 64, 64), mk(P(1), 64, P(12), 64, 64, 64, 64),
          mk(P(2), 64, P(12), 64, 64, 64, 64), mk(P(3), 64, P(13), 64, 64, 64, 64),
          mk(P(1), 64, P(11), 64, 64, 64, 64)]
    nm = [3, 5, 2, 4, 0]
    r = arena.build(pr, nm, G.REUSE_PROMOTE)
    assert (r.num_ua, r.num_ub, r.num_emu) == (3, 3, 4)
    assert [r.ua_nmod[r.prob_a[g]] for g in (0, 2, 3)] == [5, 5, 4]
    assert [r.ub_nmod[r.prob_b[g]] for g in (0, 1, 3)] == [5, 5, 4]
    assert [r.eff_nmod[g] for g in range(4)] == [5, 5, 5, 4]
    assert r.num_promoted == 2
    assert (r.prob_a[4], r.prob_b[4], r.eff_nmod[4]) == (-1, -1, 0)
    e = arena.build(pr, nm, G.REUSE_EXACT_N)   # different N never share
    assert (e.num_ua, e.num_ub, e.num_promoted) == (4, 4, 0)
    assert e.prob_a[0] != e.prob_a[1]
    assert [e.eff_nmod[g] for g in range(4)] == nm[:4]
    e = arena.build(pr, [5, 5, 2, 4, 0], G.REUSE_EXACT_N)   # equal N does share
    assert e.prob_a[0] == e.prob_a[1] and e.ua_nmod[e.prob_a[0]] == 5


def test_capacity_invalid_and_repeated_builds(arena):
    pr = [mk(P(1), 8, P(2), 8, 8, 8, 8)] * 65
    assert arena.build(pr, [2] * 65).status == G.REUSE_ERR_CAPACITY
    for _ in range(3):   # no stale table entries from the previous build
        r = arena.build(pr[:64], [2] * 64)
        assert (r.status, r.num_ua, r.num_ub) == (G.REUSE_OK, 1, 1)
    assert arena.build(pr[:4], [2] * 4, policy=7).status == G.REUSE_ERR_INVALID
    r = arena.build([], [])
    assert (r.status, r.num_ua, r.num_ub, r.num_emu) == (G.REUSE_OK, 0, 0, 0)


def test_oversized_arena_reports_capacity():
    a = Arena((1 << 30) + 1)
    try:
        assert a.rc == G.REUSE_ERR_CAPACITY
        assert G.lib().reuse_arena_capacity(a.a) == 0
    finally:
        a.close()
