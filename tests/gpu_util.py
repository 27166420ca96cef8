"""Helpers for the GPU parity tests: device buffers through torch (plumbing only) and the
kernel-level pipeline of the library run on the reference test's host problems."""
import ctypes as C
import sys

import numpy as np

import ggemm as G
import oracle_lib as O


def torch():
    import torch as t
    return t


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(arr, dtype=None):
    """numpy -> device tensor (contiguous copy)."""
    t = torch()
    a = np.ascontiguousarray(arr)
    return t.from_numpy(a.copy()).to("cuda")


def host(t_):
    torch().cuda.synchronize()
    return t_.detach().cpu().numpy()


def dev_zeros(nbytes, dtype="uint8"):
    t = torch()
    dt = {"uint8": t.uint8, "int8": t.int8, "int32": t.int32, "float64": t.float64}[dtype]
    itemsize = {"uint8": 1, "int8": 1, "int32": 4, "float64": 8}[dtype]
    return t.zeros(max(1, (nbytes + itemsize - 1) // itemsize), dtype=dt, device="cuda")


def dev_struct_array(structs, ctype):
    """Copy a list of ctypes structures into device memory; returns the uint8 tensor."""
    n = max(len(structs), 1)
    arr = (ctype * n)(*structs)
    raw = np.frombuffer(bytes(arr), dtype=np.uint8).copy()
    return dev(raw)


def same_bits(a, b):
    """float64 arrays equal bit for bit, except that any NaN equals any NaN (NaN payloads are
    not specified by IEEE arithmetic and differ between the host and the GPU)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    if a.shape != b.shape:
        return False
    both_nan = np.isnan(a) & np.isnan(b)
    return bool(np.all((a.view(np.int64) == b.view(np.int64)) | both_nan))


def read_counters(reset=True):
    c = G.Oz2Counters()
    torch().cuda.synchronize()
    assert G.lib().oz2_read_counters(C.byref(c), 1 if reset else 0, None) == 0
    return c


class WhiteboxRun:
    """prep -> grouped INT8 GEMM -> reconstruct through the kernel-level ABI for a list of
    oracle_lib.HostProb, laid out like the reference numerics test (tight planes per problem)."""

    def __init__(self, hs, poison=0x5A):
        t = torch()
        self.hs = hs
        self.dA, self.dB, self.dC = [], [], []
        self.descs = []
        a8 = b8 = c32 = rsz = csz = 0
        for h in hs:
            kp = O.kp_of(h.k)
            NP = h.N + 1
            a8 += NP * h.m * kp
            b8 += NP * h.n * kp
            c32 += NP * h.m * h.n
            rsz += 4 * h.m
            csz += 4 * h.n
        self.A8 = t.full((a8 + 16,), poison, dtype=t.uint8, device="cuda")
        self.B8 = t.full((b8 + 16,), poison, dtype=t.uint8, device="cuda")
        self.C32 = t.zeros((c32 + 16,), dtype=t.int32, device="cuda")
        self.rs = t.zeros((rsz + 16,), dtype=t.int32, device="cuda")
        self.cs = t.zeros((csz + 16,), dtype=t.int32, device="cuda")
        oa = ob = oc = orr = occ = 0
        self.offs = []
        for h in hs:
            kp = O.kp_of(h.k)
            NP = h.N + 1
            A = dev(h.A)
            B = dev(h.B)
            Cm = dev(h.C0)
            self.dA.append(A)
            self.dB.append(B)
            self.dC.append(Cm)
            p = G.Oz2Problem()
            p.m, p.n, p.k, p.kp, p.num_moduli = h.m, h.n, h.k, kp, h.N
            p.lda, p.ldb, p.ldc = h.lda, h.ldb, h.ldc
            p.A, p.B, p.C = A.data_ptr(), B.data_ptr(), Cm.data_ptr()
            p.alpha, p.beta = h.alpha, h.beta
            p.A8 = self.A8.data_ptr() + oa
            p.a8_mod_stride = h.m * kp
            p.B8 = self.B8.data_ptr() + ob
            p.b8_mod_stride = h.n * kp
            p.C32 = self.C32.data_ptr() + 4 * oc
            p.c32_mod_stride = h.m * h.n
            p.row_shift = self.rs.data_ptr() + 4 * orr
            p.col_shift = self.cs.data_ptr() + 4 * occ
            self.descs.append(p)
            self.offs.append((oa, ob, oc, orr, occ))
            oa += NP * h.m * kp
            ob += NP * h.n * kp
            oc += NP * h.m * h.n
            orr += 4 * h.m
            occ += 4 * h.n
        self.d_desc = dev_struct_array(self.descs, G.Oz2Problem)
        self.max_m = max(h.m for h in hs)
        self.max_n = max(h.n for h in hs)

    def prep(self):
        rc = G.lib().oz2_prep_grouped(self.d_desc.data_ptr(), len(self.hs), self.max_m, self.max_n, None)
        assert rc == 0, rc

    def i8_problems(self):
        probs = []
        for h, p in zip(self.hs, self.descs):
            if h.alpha == 0.0:
                continue
            for l in range(h.N + 1):
                probs.append(G.I8Problem(h.m, h.n, p.kp, p.A8 + l * p.a8_mod_stride, p.B8 + l * p.b8_mod_stride,
                                         p.C32 + 4 * l * p.c32_mod_stride, -1))
        return probs

    def gemm(self, tile_cfg=-1):
        probs = self.i8_problems()
        for q in probs:
            q.tile_cfg = tile_cfg
        d_probs = dev_struct_array(probs, G.I8Problem)
        nb = G.lib().i8_grouped_gemm_sched_ws_bytes(len(probs), 0)
        ws = dev_zeros(nb)
        arr = (G.I8Problem * max(len(probs), 1))(*probs)
        nl = C.c_int(0)
        rc = G.lib().i8_grouped_gemm_ex(d_probs.data_ptr(), len(probs), arr, ws.data_ptr(), nb, None, C.byref(nl))
        assert rc == 0, rc
        torch().cuda.synchronize()
        return nl.value

    def recon(self, mode):
        rc = G.lib().oz2_reconstruct_grouped(self.d_desc.data_ptr(), len(self.hs), self.max_m, self.max_n, None, mode)
        assert rc == 0, rc

    def run(self, mode=G.OZ2_REPAIR_ON):
        self.prep()
        self.gemm()
        self.recon(mode)
        torch().cuda.synchronize()

    # ---- readback in the oracle's layouts
    def planes(self, g):
        h, (oa, ob, oc, orr, occ) = self.hs[g], self.offs[g]
        kp = O.kp_of(h.k)
        NP = h.N + 1
        A8 = host(self.A8[oa:oa + NP * h.m * kp]).view(np.int8)
        B8 = host(self.B8[ob:ob + NP * h.n * kp]).view(np.int8)
        C32 = host(self.C32[oc:oc + NP * h.m * h.n])
        rs = host(self.rs[orr:orr + 4 * h.m])
        cs = host(self.cs[occ:occ + 4 * h.n])
        return A8, B8, C32, rs, cs

    def C(self, g):
        return host(self.dC[g])


def oracle_block(A_t, B_t, C0_t, k, alpha, beta, N, mode, I, J):
    """The oracle's emulated values of the entries (I x J) of one problem, and its counters
    [nonfinite vectors, uncertified, repaired, safety] over those entries.

    Every output entry (i, j) of the Ozaki-II pipeline depends only on row i of A, column j of B
    and C0(i, j): the row shift, abs shift and norm bounds are per row, the column ones per column,
    the CRT / certificate / repair per entry.  So the sub-problem made of rows I of A, columns J of B
    and C0(I, J) gives the oracle's exact bits for those entries at O(N k |I| |J|) cost.
    Torch layouts (column-major with leading dimension = the last axis): A_t (k, >= m),
    B_t (n, >= k), C0_t (n, >= m) or None when beta == 0.  Returns ((|J|, |I|) array, counters)."""
    t = torch()
    ii = t.as_tensor(np.asarray(I), device=A_t.device)
    jj = t.as_tensor(np.asarray(J), device=A_t.device)
    a = np.ascontiguousarray(A_t[:k][:, ii].cpu().numpy())          # (k, |I|): column-major |I| x k
    b = np.ascontiguousarray(B_t[jj][:, :k].cpu().numpy())          # (|J|, k): column-major k x |J|
    if C0_t is None or beta == 0.0:
        c = np.zeros((len(J), len(I)))
    else:
        c = np.ascontiguousarray(C0_t[jj][:, ii].cpu().numpy())     # (|J|, |I|): column-major |I| x |J|
    cnt = np.zeros(4, dtype=np.int64)
    rc = O.oracle().oz2o_emulate(len(I), len(J), k, N, a.reshape(-1), len(I), b.reshape(-1), k, c.reshape(-1),
                                 len(I), alpha, beta, mode, cnt)
    assert rc == 0, rc
    return c, cnt


def oracle_full_many(jobs, workers=16, batch=16):
    """Every entry of several problems through the oracle, on a thread pool (the oracle is a ctypes
    call, which releases the GIL; 16 workers = the host share of one GPU).  jobs: list of
    (key, A_t, B_t, C0_t, k, alpha, beta, N, mode, I, J, got) with torch layouts as in oracle_block,
    I / J row / column index arrays or None (all), got the device result's entries (|J|, |I|) as a
    host array.  Yields (key, equal, counters, first differing (j, i) or None) per job; jobs are
    taken in batches so that at most `batch` problems' host copies are alive at once."""
    from concurrent.futures import ThreadPoolExecutor
    t = torch()

    def host_inputs(A_t, B_t, C0_t, k, beta, I, J):
        if I is None:
            a = np.ascontiguousarray(A_t[:k].cpu().numpy())
            b = np.ascontiguousarray(B_t[:, :k].cpu().numpy())
            c = (np.zeros(B_t.shape[0] * A_t.shape[1]).reshape(B_t.shape[0], A_t.shape[1])
                 if C0_t is None or beta == 0.0 else np.ascontiguousarray(C0_t.cpu().numpy()))
            return a, b, c
        ii = t.as_tensor(np.asarray(I), device=A_t.device)
        jj = t.as_tensor(np.asarray(J), device=A_t.device)
        a = np.ascontiguousarray(A_t[:k][:, ii].cpu().numpy())
        b = np.ascontiguousarray(B_t[jj][:, :k].cpu().numpy())
        c = (np.zeros((len(J), len(I))) if C0_t is None or beta == 0.0 else
             np.ascontiguousarray(C0_t[jj][:, ii].cpu().numpy()))
        return a, b, c

    def work(item):
        key, (a, b, c), k, alpha, beta, N, mode, got = item
        m, n = a.shape[1], b.shape[0]
        cnt = np.zeros(4, dtype=np.int64)
        rc = O.oracle().oz2o_emulate(m, n, k, N, a.reshape(-1), m, b.reshape(-1), k, c.reshape(-1), m, alpha, beta,
                                     mode, cnt)
        assert rc == 0, (key, rc)
        eq = same_bits(got, c)
        where = None
        if not eq:
            bad = ~((got.view(np.int64) == c.view(np.int64)) | (np.isnan(got) & np.isnan(c)))
            where = tuple(int(x) for x in np.argwhere(bad)[0])
        return key, eq, cnt, where

    with ThreadPoolExecutor(max_workers=workers) as pool:
        for b0 in range(0, len(jobs), batch):
            items = []
            for (key, A_t, B_t, C0_t, k, alpha, beta, N, mode, I, J, got) in jobs[b0:b0 + batch]:
                items.append((key, host_inputs(A_t, B_t, C0_t, k, beta, I, J), k, alpha, beta, N, mode, got))
            for r in pool.map(work, items):
                yield r
            del items


def gpu_block(C_t, I, J):
    """Entries (I x J) of a device result in torch layout (n, >= m), as a (|J|, |I|) array."""
    t = torch()
    ii = t.as_tensor(np.asarray(I), device=C_t.device)
    jj = t.as_tensor(np.asarray(J), device=C_t.device)
    return C_t[jj][:, ii].cpu().numpy()
