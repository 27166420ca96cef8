"""The INT8 GEMM's persistent tile scheduler, checked on the CPU: the host-built schedule image
(i8_grouped_gemm_build_schedule, through the C ABI) is executed by a model of the kernel's queue
protocol -- per-XCD queue counters, a fetch per tile, stealing from the other queues in turn --
under random interleavings of the workgroups' atomic operations.  Every tile must be run exactly
once, every workgroup must stop, and the tiles of each product must cover its output grid
(src/int8_grouped_gemm.cu:360-407 is the reference's persistent loop)."""
import ctypes as C
import random

import numpy as np
import pytest

import gpu_util  # noqa: F401  (puts the package on sys.path)
import ggemm as G

XCDS, HDR, HDR_XCD = 8, 64, 8
TILE = {0: (256, 128), 1: (128, 128), 2: (64, 64)}
GROUP_M = 8


def build(shapes):
    """Schedule image of products (m, n, kp, tile_cfg) for the general kernel."""
    n = len(shapes)
    arr = (G.I8Problem * max(n, 1))()
    for i, (m, nn, kp, cfg) in enumerate(shapes):
        arr[i] = G.I8Problem(m, nn, kp, 0x1000, 0x2000, 0x3000, cfg)   # never dereferenced on the host
    nbytes = G.lib().i8_grouped_gemm_sched_ws_bytes(n, 0)
    img = (C.c_int * (nbytes // 4 + 1))()
    info = G.I8SchedInfo()
    rc = G.lib().i8_grouped_gemm_build_schedule(arr, n, img, nbytes, C.byref(info))
    assert rc == 0
    return np.ctypeslib.as_array(img)[: info.bytes_used // 4].copy(), info


def raster(local, m, n, bm, bn, gm):
    """The kernel's grouped raster: blocks of gm tile-rows, m fastest inside a block."""
    tiles_m, tiles_n = -(-m // bm), -(-n // bn)
    per_group = gm * tiles_n
    g = local // per_group
    first_m = g * gm
    gsz = min(gm, tiles_m - first_m)
    r = local - g * per_group
    return first_m + r % gsz, r // gsz


def decode(img, u, shapes):
    ne, per = int(img[1]), int(img[2])
    prefix = img[HDR:HDR + ne + 1]
    entry = img[HDR + ne + 1:HDR + 2 * ne + 1]
    if per > 0:
        e, local = u // per, u % per
    else:
        e = int(np.searchsorted(prefix, u, side="right")) - 1
        local = u - int(prefix[e])
    pi, cfg = int(entry[e]) >> 2, int(entry[e]) & 3
    m, n = shapes[pi][0], shapes[pi][1]
    bm, bn = TILE[cfg]
    return pi, cfg, raster(local, m, n, bm, bn, GROUP_M)


def run_protocol(img, grid, rng):
    """Model of the kernel's queue protocol.  Each workgroup: a first tile without a fetch (its index
    on its XCD), then per tile one fetch, resolved (stealing on exhaustion) before the tile ends.  Returns the units run by each
    workgroup and the number of counter operations."""
    xs = [int(v) for v in img[HDR_XCD:HDR_XCD + XCDS + 1]]
    total, ch = int(img[0]), int(img[3])
    ctr = [0] * XCDS
    ops = [0]

    def fetch(q):
        ops[0] += 1
        v = ctr[q]
        ctr[q] += 1
        return v + (grid - q + XCDS - 1) // XCDS   # past the queue's workgroups' first tiles

    def resolve(own, st, v):
        while True:
            q = (own + st["qi"]) % XCDS
            if ch > 0:
                u = ((v // ch) * XCDS + q) * ch + v % ch
                if u < total:
                    return u
            else:
                u = xs[q] + v
                if u < xs[q + 1]:
                    return u
            st["qi"] += 1
            if st["qi"] == XCDS:
                return -1
            v = fetch((own + st["qi"]) % XCDS)

    # each workgroup is a generator that yields before every counter operation
    def wg(b, out):
        own = b % XCDS
        st = {"qi": 0}
        yield
        u = resolve(own, st, b // XCDS)       # first tile: the workgroup's index on its XCD
        while u >= 0:
            out.append(u)             # the tile runs; when its last stage has landed the next is claimed
            yield
            u = resolve(own, st, fetch((own + st["qi"]) % XCDS))

    runs = [[] for _ in range(grid)]
    live = {b: wg(b, runs[b]) for b in range(grid)}
    while live:
        b = rng.choice(list(live))
        try:
            next(live[b])
        except StopIteration:
            del live[b]
    return runs, ops[0]


CASES = {
    "uniform": [(1024, 1024, 1024, -1)] * 64 * 16,
    "large": [(8192, 8192, 16384, -1)] * 17,
    "ragged": None,
    "few": [(256, 256, 256, -1)] * 15,
    "one": [(4096, 4096, 2048, -1)],
}


def ragged_shapes(seed=5):
    rng = np.random.default_rng(seed)
    lu = lambda lo, hi: int(np.exp(rng.uniform(np.log(lo), np.log(hi))))
    out = []
    for _ in range(96):
        m, n, k = lu(16, 4096), lu(16, 4096), lu(16, 8192)
        out += [(m, n, (k + 31) // 32 * 32, -1)] * 3
    return out


@pytest.mark.parametrize("case", sorted(CASES))
@pytest.mark.parametrize("seed", [0, 1])
@pytest.mark.parametrize("chunk", [0, 32])
def test_every_tile_once_and_workgroups_stop(case, seed, chunk):
    """chunk 0: the image's queue ranges (the kernel-level default image holds every tile in queue 0,
    so seven XCDs' workgroups steal throughout); chunk 32: the persistent kernels' chunked queues."""
    shapes = CASES[case] or ragged_shapes()
    img, info = build(shapes)
    img[3] = chunk
    total = int(img[0])
    assert total == info.tiles_main > 0
    xs = [int(v) for v in img[HDR_XCD:HDR_XCD + XCDS + 1]]
    assert xs[0] == 0 and xs[-1] == total and all(a <= b for a, b in zip(xs, xs[1:]))
    assert not img[32:41].any()          # queue counters and finished count start at zero
    grid = min(total, 512)
    runs, ops = run_protocol(img, grid, random.Random(seed))
    done = sorted(u for r in runs for u in r)
    assert done == list(range(total))
    # bounded work: one fetch per tile, plus at most eight exhausted fetches per workgroup
    assert ops <= total + XCDS * grid + grid
    # the first round of each XCD is the contiguous start of its queue
    if chunk == 0:
        for b in range(min(grid, XCDS)):
            firsts = sorted(r[0] for bb, r in enumerate(runs) if bb % XCDS == b and r and xs[b] <= r[0] < xs[b + 1])
            assert firsts == list(range(xs[b], xs[b] + len(firsts)))
    # each product's tiles cover its grid exactly once
    seen = {}
    for u in range(total):
        pi, cfg, (tm, tn) = decode(img, u, shapes)
        seen.setdefault(pi, []).append((cfg, tm, tn))
    for pi, tiles in seen.items():
        m, n = shapes[pi][0], shapes[pi][1]
        cfg = tiles[0][0]
        bm, bn = TILE[cfg]
        want = {(i, j) for i in range(-(-m // bm)) for j in range(-(-n // bn))}
        got = [(tm, tn) for c, tm, tn in tiles]
        assert all(c == cfg for c, _, _ in tiles) and len(got) == len(want) and set(got) == want


DEAL_SCRIPT = r"""
import sys, json
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[2])
import test_i8_schedule as T
img, _ = T.build(T.CASES["large"][:16])
print(json.dumps([int(v) for v in img]))
"""


def test_products_dealt_whole_to_queues():
    """GGEMM_I8_SCHED=persistent GGEMM_I8_CHUNK=0 (read once per process, hence a child process):
    each (problem, plane) product sits in one XCD queue, and equal products give equal queues."""
    import json
    import os
    import subprocess
    import sys
    from pathlib import Path
    here = Path(__file__).resolve().parent
    env = dict(os.environ, GGEMM_I8_SCHED="persistent", GGEMM_I8_CHUNK="0")
    out = subprocess.run([sys.executable, "-c", DEAL_SCRIPT, str(here), str(here.parent / "coding-basic-hw-2_amd")],
                         env=env, capture_output=True, text=True,
                         timeout=120, check=True)
    img = np.array(json.loads(out.stdout.strip().splitlines()[-1]))
    assert int(img[3]) == 0
    ne = int(img[1])
    prefix = set(int(p) for p in img[HDR:HDR + ne + 1])
    xs = [int(v) for v in img[HDR_XCD:HDR_XCD + XCDS + 1]]
    assert all(x in prefix for x in xs)     # queue boundaries fall on entry boundaries
    sizes = [xs[x + 1] - xs[x] for x in range(XCDS)]
    assert len(set(sizes)) == 1 and sizes[0] > 0


@pytest.mark.parametrize("chunk", [16, 32])
def test_chunked_queues_cover_every_tile(chunk):
    """The chunked queue mode (image word 3: queue x = chunks x, x + 8, ... of the LPT table)."""
    img, _ = build(ragged_shapes(7))
    img[3] = chunk
    total = int(img[0])
    runs, _ = run_protocol(img, min(total, 512), random.Random(3))
    assert sorted(u for r in runs for u in r) == list(range(total))


def run_tail(hw, total, grid, rng, chunk=32):
    """Model of the 256 x 256 kernel's tail workgroups (i8_large_kernel<true>, blockIdx >= hw): the
    queue q = chunks q, q + 8, ... of `chunk` units of [hw, total); a tail workgroup on XCD b mod 8
    starts at its rank among that XCD's tail workgroups, then fetches from the queue's counter and
    moves on to the next queues in turn.  The atomics are interleaved at random; returns the units
    each workgroup ran and the counters left."""
    ctr = [0] * XCDS

    def tail_wgs(q):
        f = hw + ((q - hw) % XCDS + XCDS) % XCDS
        return (grid - f + XCDS - 1) // XCDS if f < grid else 0

    def unit_of(q, l):
        v = hw + ((l // chunk) * XCDS + q) * chunk + l % chunk
        return v if v < total else -1

    def workgroup(b):
        own, sq = b % XCDS, 0
        runs = []

        def resolve(l):
            nonlocal sq
            while True:
                v = unit_of((own + sq) % XCDS, l)
                if v >= 0:
                    return v
                sq += 1
                if sq == XCDS:
                    return -1
                q2 = (own + sq) % XCDS
                l = tail_wgs(q2) + ctr[q2]
                ctr[q2] += 1

        first = hw + ((own - hw) % XCDS + XCDS) % XCDS
        u = resolve((b - first) // XCDS)
        while u >= 0:
            runs.append(u)
            yield None                      # a tile's work: other workgroups' atomics may interleave
            if sq == XCDS:
                break
            q = (own + sq) % XCDS
            l = tail_wgs(q) + ctr[q]
            ctr[q] += 1
            u = resolve(l)
        yield runs

    gens = {b: workgroup(b) for b in range(hw, grid)}
    done = {}
    while gens:
        b = rng.choice(sorted(gens))
        r = next(gens[b])
        if r is not None:
            done[b] = r
            del gens[b]
    return done, ctr


@pytest.mark.parametrize("hw,total,grid", [(0, 40, 40), (0, 700, 256), (4096, 34816, 4096 + 256), (5, 1000, 5 + 256),
                                           (0, 300, 7), (3, 3 + 65, 3 + 64), (100, 100 + 513, 100 + 256)])
def test_tail_workgroups_run_every_unit_once(hw, total, grid):
    """Every unit of the tail runs exactly once and every tail workgroup stops, under random
    interleavings of the queue counters' atomics, with tails smaller and larger than the grid,
    XCDs without tail workgroups (whose queues are stolen) and a first tail workgroup off XCD 0."""
    for seed in range(3):
        done, _ = run_tail(hw, total, grid, random.Random(seed))
        units = sorted(u for r in done.values() for u in r)
        assert units == list(range(hw, total))
        assert sorted(done) == list(range(hw, grid))


@pytest.mark.parametrize("m,n", [(2048, 2048), (300, 700), (1030, 1100), (256, 256), (2500, 300)])
def test_compacted_tiles_dealt_once(m, n):
    """The compacted tiles of a 256 x 256-tile product: for every list size, tile i goes to the unit at
    raster index off + i s (s = units / tiles, off = 16 pi mod s), and the inverse of the raster
    (the unit's local index from its tile position) finds each exactly once."""
    bm = bn = 256
    tiles_m, tiles_n = -(-m // bm), -(-n // bn)
    units = tiles_m * tiles_n
    pos = {raster(local, m, n, bm, bn, 4): local for local in range(units)}

    def raster_local(tm, tn):   # the kernel's inverse raster (groups of 4 tile-rows)
        g = tm // 4
        first = g * 4
        gsz = min(4, tiles_m - first)
        return g * 4 * tiles_n + tn * gsz + (tm - first)

    assert all(raster_local(*t) == local for t, local in pos.items())
    for nrt in range(1, m + 1, max(1, m // 7)):
        for nct in range(1, n + 1, max(1, n // 5)):
            tcm, tcn = -(-nrt // bm), -(-nct // bn)
            nt = tcm * tcn
            for pi in (0, 1, 5, 37):
                s = units // nt
                off = (pi * 16) % s
                got = []
                for (tm, tn), _ in pos.items():
                    local = raster_local(tm, tn) - off
                    if local >= 0 and local % s == 0 and local // s < nt:
                        got.append(local // s)
                assert sorted(got) == list(range(nt))
