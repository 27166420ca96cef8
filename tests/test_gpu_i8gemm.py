"""Bit-exactness of the grouped INT8 MFMA GEMM (tests/test_i8_grouped.cu:193-254 cases).

The reference product of int8 matrices with kp <= 131040 has |C| < 2^31, so the float64 BLAS
product on the host is exact and serves as the checker at every size (cross-checked against
the oracle's int64 brute force on the small shapes)."""
import ctypes as C

import numpy as np
import pytest
import torch

import ggemm as G
import oracle_lib as O
from gpu_util import dev, dev_struct_array, dev_zeros, host, say

pytestmark = pytest.mark.gpu

HETERO = [(1, 1, 32), (1, 257, 4096), (257, 1, 96), (33, 17, 64), (129, 131, 1024), (127, 255, 32),
          (64, 64, 65536), (3, 5, 131040), (500, 300, 2048), (1000, 1, 512), (1, 1000, 512), (77, 1000, 320),
          (1024, 768, 1024), (31, 33, 160), (0, 7, 64), (65, 63, 8192), (129, 1, 131040), (2, 2, 224), (9, 7, 0)]


class Group:
    def __init__(self, shapes, seed, fill=None):
        rng = np.random.default_rng(seed)
        self.shapes = shapes
        offA, offB, offC = [], [], []
        ta = tb = tc = 0
        for (m, n, kp) in shapes:
            offA.append(ta); ta += -(-m * kp // 256) * 256
            offB.append(tb); tb += -(-n * kp // 256) * 256
            offC.append(tc); tc += -(-m * n // 64) * 64
        if fill is None:
            self.hA = rng.integers(-128, 128, size=max(ta, 1), dtype=np.int8)
            self.hB = rng.integers(-128, 128, size=max(tb, 1), dtype=np.int8)
        else:
            self.hA = np.full(max(ta, 1), fill, dtype=np.int8)
            self.hB = np.full(max(tb, 1), fill, dtype=np.int8)
        self.dA, self.dB = dev(self.hA.view(np.uint8)), dev(self.hB.view(np.uint8))
        self.dC = torch.zeros(max(tc, 1), dtype=torch.int32, device="cuda")
        self.offA, self.offB, self.offC = offA, offB, offC

    def problems(self, cfg):
        return [G.I8Problem(m, n, kp, self.dA.data_ptr() + self.offA[i], self.dB.data_ptr() + self.offB[i],
                            self.dC.data_ptr() + 4 * self.offC[i], cfg(i) if callable(cfg) else cfg)
                for i, (m, n, kp) in enumerate(self.shapes)]

    def run(self, cfg):
        self.dC.fill_(0x7F7F7F7F)
        probs = self.problems(cfg)
        d_probs = dev_struct_array(probs, G.I8Problem)
        nb = G.lib().i8_grouped_gemm_sched_ws_bytes(len(probs), 0)
        ws = dev_zeros(nb)
        arr = (G.I8Problem * len(probs))(*probs)
        nl = C.c_int(-1)
        rc = G.lib().i8_grouped_gemm_ex(d_probs.data_ptr(), len(probs), arr, ws.data_ptr(), nb, None, C.byref(nl))
        assert rc == 0
        return nl.value, host(self.dC)

    def check(self, Cres):
        for i, (m, n, kp) in enumerate(self.shapes):
            if m == 0 or n == 0 or kp == 0:
                continue
            a = self.hA[self.offA[i]:self.offA[i] + m * kp].reshape(m, kp).astype(np.float64)
            b = self.hB[self.offB[i]:self.offB[i] + n * kp].reshape(n, kp).astype(np.float64)
            ref = (a @ b.T)   # exact: |entries| < 2^31 < 2^53
            got = Cres[self.offC[i]:self.offC[i] + m * n].reshape(n, m).T
            assert np.array_equal(got.astype(np.float64), ref), (i, m, n, kp)


def test_float64_checker_is_exact():
    rng = np.random.default_rng(11)
    for (m, n, kp) in [(17, 9, 96), (33, 40, 1024)]:
        a = rng.integers(-128, 128, size=m * kp, dtype=np.int8)
        b = rng.integers(-128, 128, size=n * kp, dtype=np.int8)
        ref = O.oracle_i8_gemm(m, n, kp, a, b).reshape(n, m).T
        f = a.reshape(m, kp).astype(np.float64) @ b.reshape(n, kp).astype(np.float64).T
        assert np.array_equal(ref.astype(np.float64), f)


@pytest.fixture(params=["dispatch", "persistent"])
def sched(request, monkeypatch):
    """The kernel-level API runs one workgroup per tile, or (GGEMM_I8_SCHED=persistent) the persistent
    work-stealing kernels."""
    if request.param == "persistent":
        monkeypatch.setenv("GGEMM_I8_SCHED", "persistent")
    else:
        monkeypatch.delenv("GGEMM_I8_SCHED", raising=False)
    return request.param


@pytest.mark.parametrize("cfg", [0, 1, 2, -1, "mixed"])
def test_hetero_bit_exact(cfg, sched):
    g = Group(HETERO, 1234)
    say(f"i8 hetero cfg={cfg} {sched}")
    nl, Cres = g.run((lambda i: i % 3) if cfg == "mixed" else cfg)
    assert nl == 1
    g.check(Cres)


def test_int32_edge_all_minus128(sched):
    g = Group([(3, 5, 131040), (17, 9, 131040), (1, 1, 32)], 1, fill=-128)
    for cfg in (-1, 0, 2):
        say(f"i8 -128 edge cfg={cfg} {sched}")
        nl, Cres = g.run(cfg)
        for i, (m, n, kp) in enumerate(g.shapes):
            got = Cres[g.offC[i]:g.offC[i] + m * n]
            assert (got == 16384 * kp).all(), (cfg, i)
    assert 16384 * 131040 == 2146959360


def test_relaunch_split_schedule(sched):
    """build_schedule + launch three times without re-uploading the schedule (the persistent kernels'
    queue counters reset themselves at the end of each launch)."""
    say(f"i8 relaunch {sched}")
    g = Group([(200, 100, 640), (64, 300, 96), (5, 5, 32)] + [(512, 384, 256)] * 40, 99)
    probs = g.problems(-1)
    d_probs = dev_struct_array(probs, G.I8Problem)
    nb = G.lib().i8_grouped_gemm_sched_ws_bytes(len(probs), 0)
    himg = (C.c_uint8 * nb)()
    info = G.I8SchedInfo()
    arr = (G.I8Problem * len(probs))(*probs)
    assert G.lib().i8_grouped_gemm_build_schedule(arr, len(probs), himg, nb, C.byref(info)) == 0
    assert info.num_launches == 1 and info.bytes_used <= nb
    ws = dev(np.frombuffer(bytes(himg), dtype=np.uint8))
    for _ in range(3):
        g.dC.zero_()
        assert G.lib().i8_grouped_gemm_launch(d_probs.data_ptr(), len(probs), ws.data_ptr(), C.byref(info), None) == 0
        g.check(host(g.dC))
    # counters and finished count back at zero after every launch
    assert not host(ws).view(np.int32)[32:41].any()


def test_invalid_problem_rejected():
    g = Group([(4, 4, 48)], 5)   # kp % 32 != 0 must be refused on the host
    probs = g.problems(-1)
    arr = (G.I8Problem * 1)(*probs)
    nb = G.lib().i8_grouped_gemm_sched_ws_bytes(1, 0)
    himg = (C.c_uint8 * nb)()
    info = G.I8SchedInfo()
    assert G.lib().i8_grouped_gemm_build_schedule(arr, 1, himg, nb, C.byref(info)) != 0
