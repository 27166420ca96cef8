// recon.hip -- CRT reconstruction, alpha/beta epilogue and componentwise certificate for a whole
// group (one launch), following src/ozaki2_numerics.cu:454-586.
//
// Per entry (i, j) of a problem with N moduli:
//   y_l = (C_l mod p_l) q_l mod p_l,   S1 = sum s1_l y_l (u64),  S2 = sum s2_l y_l (u32)
//   Q   = rint((S1 + S2 2^-18) u1/P),  X/u1 = (S1 - Q P1) + (S2 2^-18 - Q P2)
//   v   = 2^(log2 u1 - s_i - t_j) X/u1 (exact power-of-two scaling),  C = alpha v (+ beta C0)
//   certificate: E = 2^-(s+t) [da nb + na db + da db + u1 (N 255 2^-19 + 2^-10) + 4u |X|],
//   Lab = max(2^-(sigma+tau) L, |v| - E)(1 - 2^-40); certified iff
//   |alpha| E (1 + 2^-40) <= gamma' (|alpha| Lab + |beta C0|)(1 - 2^-40), gamma' = (gamma_n - 2u)(1 - 2^-40).
// Entries that fail (repair ON) or whose row / column holds NaN/Inf (every mode) are recomputed as
// a sequential FP64 fma dot product over k, exactly the value a native dot gives.
//
// Inputs: the production pipeline hands over the CRT digits y_l directly (one byte per entry and
// plane, written by the INT8 GEMM epilogue) and the int32 abs-plane product L; the kernel-level
// API hands over the int32 plane products C_l and the digits are formed here.  Both give the same
// y_l, hence the same output bits.
// Mapping: a workgroup covers 128 rows x 8 columns of one problem (blocked digits: four 16 x 16
// blocks, one per wave, lane = the block's MFMA lane, so a wave's per-plane digit read is one
// contiguous 256-byte block); a thread owns 4 consecutive rows of one column, so every per-plane
// digit read is one 32-bit load, L one 128-bit load, the row
// words (shift, sigma, norm bounds) four 128-bit loads and C0 two 128-bit loads (m % 4 == 0 and
// aligned operands; element-wise loads otherwise).  All loads are issued before the arithmetic and
// go through global-address-space pointers; the CRT constants are scalar.
// Two multiply-adds of the reference that its device compiler fuses are written as fma() here
// (s2d - Q P2 and |alpha| Lab + |beta C0|); every other operation is unfused (fp contract off),
// so the result is the reference's to the last bit.
#include <cmath>

#include "common.hpp"

#pragma clang fp contract(off)

namespace ggemm {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef double v2d __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kTileM = 128, kTileN = 8;   // rows x columns per workgroup (32 row quads x 8 columns)
constexpr int kBTileM = 64, kBTileN = 16;  // blocked layout: four 16 x 16 blocks stacked per workgroup

#define GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ const GLOBAL T* gp(const T* p) {
  return (const GLOBAL T*)p;
}
template <class T>
__device__ __forceinline__ GLOBAL T* gpw(T* p) {
  return (GLOBAL T*)p;
}

// x 2^e: one ldexp (the exact product, rounded once -- the reference's single multiply by 2^e)
// for |e| <= 1000, else the reference's steps of at most 2^+-1000
__device__ __forceinline__ double mul_pow2(double x, int e) {
  if (e >= -1000 && e <= 1000) return ldexp(x, e);
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    const int ee = max(-1000, min(1000, e));
    x = ldexp(x, ee);
    e -= ee;
  }
  return x;
}
__device__ __forceinline__ uint32_t mod_small(uint32_t u, uint32_t p, uint32_t magic) {
  uint32_t r = u - __umulhi(u, magic) * p;   // magic = floor(2^32/p): quotient low by at most 1
  r = r >= p ? r - p : r;
  return r >= p ? r - p : r;
}
__device__ __forceinline__ double fp64_dot(const oz2_problem& pr, int i, int j) {
  const GLOBAL double* a = gp(pr.A) + i;
  const GLOBAL double* b = gp(pr.B) + (size_t)j * pr.ldb;
  const size_t lda = (size_t)pr.lda;
  const int K = pr.k;
  double s = 0.0;
  int k = 0;
  for (; k + 8 <= K; k += 8) {   // 16 loads in flight, then the same fma chain
    double x[8], y[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      x[t] = a[(size_t)(k + t) * lda];
      y[t] = b[k + t];
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) s = fma(x[t], y[t], s);
  }
  for (; k < K; ++k) s = fma(a[(size_t)k * lda], b[k], s);
  return s;
}

struct Counts {
  unsigned uncert, repair, safety;
};

// One entry: CRT, scaling, alpha/beta, certificate.  Entries that need the FP64 dot product
// (safety fallback, repair) return with dot set; the caller computes it.  c0 is read only when
// beta != 0.
__device__ __forceinline__ double entry(const oz2_problem& pr, const CrtTables* __restrict__ tab, int N, int mode,
                                        int i, int j, uint64_t S1, uint32_t S2, int32_t L, int rsh, int csh,
                                        int sig, int tau, double da, double na, double db, double nb, double c0,
                                        double gam, Counts& cn, bool& dot) {
  const double alpha = pr.alpha, beta = pr.beta;
  if (alpha == 0.0) return (beta == 0.0) ? 0.0 : beta * c0;   // BLAS: A, B, workspace not referenced
  if (rsh == OZ2_SHIFT_NONFINITE || csh == OZ2_SHIFT_NONFINITE) {   // safety fallback
    ++cn.safety;
    dot = true;
    return 0.0;
  }
  if (sig == OZ2_SHIFT_ZERO || tau == OZ2_SHIFT_ZERO)   // zero row / column: AB_ij = 0
    return (beta == 0.0) ? alpha * 0.0 : fma(alpha, 0.0, beta * c0);
  const int64_t P1 = tab->P1[N];
  const double P2 = tab->P2[N], invPu = tab->inv_Pu[N];
  const int lu1 = tab->log2_u1[N];
  const double s2d = (double)S2 * 0x1p-18;
  const double Q = rint(((double)S1 + s2d) * invPu);
  const int64_t X1 = (int64_t)S1 - (int64_t)Q * P1;
  const double xr = (double)X1 + fma(-Q, P2, s2d);
  const int esc = lu1 - rsh - csh;
  const double v = mul_pow2(xr, esc);
  const double emu = (beta == 0.0) ? alpha * v : fma(alpha, v, beta * c0);
  if (mode == OZ2_REPAIR_OFF || (beta != 0.0 && !isfinite(c0))) return emu;
  const double u = 0x1p-53;
  const double crt_u = N * 255.0 * 0x1p-19 + 0x1p-10;
  const double aalpha = fabs(alpha);
  const double et = fma(da, nb, fma(na, db, da * db)) * (1.0 + 0x1p-40);
  const double Eu = (fma(et, ldexp(1.0, -lu1), crt_u) + 4.0 * u * fabs(xr)) * (1.0 + 0x1p-40);
  const double E = mul_pow2(Eu, esc);
  double lab = mul_pow2((double)L, -(sig + tau));
  lab = fmax(lab, fabs(v) - E) * (1.0 - 0x1p-40);
  if (lab < 0x1p-1000) lab = 0.0;
  const double lhs = aalpha * E * (1.0 + 0x1p-40);
  const double rhs = gam * fma(aalpha, lab, fabs(beta * c0)) * (1.0 - 0x1p-40);
  if (gam > 0.0 && E >= 0x1p-1000 && isfinite(lhs) && isfinite(v) && lhs <= rhs) return emu;
  if (mode == OZ2_REPAIR_COUNT) {
    ++cn.uncert;
    return emu;
  }
  ++cn.repair;
  dot = true;
  return 0.0;
}
// C from the FP64 dot product d (safety fallback and repair)
__device__ __forceinline__ double from_dot(double alpha, double beta, double d, double c0) {
  return (beta == 0.0) ? alpha * d : fma(alpha, d, beta * c0);
}

constexpr int kKC = 16;        // k-chunk of the tile dot products
constexpr int kTileDots = 8;   // threads needing dot products from which the tile computes them all
constexpr int kWaveDots = 4;   // lanes needing dot products from which a wave computes its whole block

// Blocked layout: the same for one wave's 16 x 16 block (rows wr0 .., columns wc0 ..; lane
// l = 16 q + c owns rows 4 q .. 4 q + 3 of column c), staged through the wave's own LDS: no
// workgroup barrier, so waves without such entries never wait.  The wave barrier and fences order
// the lanes' LDS writes before other lanes read them.
__device__ __forceinline__ void wave_dots(const oz2_problem& pr, int wr0, int wc0, int lane, double* wA, double* wB,
                                          double (&acc)[4]) {
  const GLOBAL double* A = gp(pr.A);
  const GLOBAL double* B = gp(pr.B);
  const size_t lda = (size_t)pr.lda, ldb = (size_t)pr.ldb;
  const int m = pr.m, n = pr.n, K = pr.k;
  const int q4 = 4 * (lane >> 4), c = lane & 15;
  const int sk = lane >> 2, sr = 4 * (lane & 3);   // staging: k-row sk, rows / k sr .. sr + 3
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = 0.0;
  if (K <= 0) return;
  // the chunk's 8 values per lane come from clamped (always valid) addresses, all loads in flight
  // at once (no prefetch across chunks: it would cost the kernel its fifth wave per SIMD); values
  // outside the problem stage as zero
  const int colB = min(wc0 + sk, n - 1);
  const bool inB = wc0 + sk < n;
  double va[4], vb[4];
  auto fetch = [&](int kc) {
    const size_t ka = (size_t)min(kc + sk, K - 1) * lda;
#pragma unroll
    for (int e = 0; e < 4; ++e) va[e] = A[(size_t)min(wr0 + sr + e, m - 1) + ka];
#pragma unroll
    for (int e = 0; e < 4; ++e) vb[e] = B[(size_t)min(kc + sr + e, K - 1) + (size_t)colB * ldb];
  };
  for (int kc = 0; kc < K; kc += kKC) {
    const int kn = min(kKC, K - kc);
    fetch(kc);
#pragma unroll
    for (int e = 0; e < 4; ++e) {   // A: wA[kk][r] (16 x 16), B: wB[col][kk] (16 x 17)
      wA[sk * 16 + sr + e] = (wr0 + sr + e < m && sk < kn) ? va[e] : 0.0;
      wB[sk * (kKC + 1) + sr + e] = (inB && sr + e < kn) ? vb[e] : 0.0;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll 4
    for (int kk = 0; kk < kn; ++kk) {
      const double b = wB[c * (kKC + 1) + kk];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = fma(wA[kk * 16 + q4 + e], b, acc[e]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// Sequential-fma dot products of every entry of an RM x CN tile (rows r0.., columns cb..), each
// thread its rows lr .. lr + 3 of column lc: k-chunks of A (kKC x RM, rows contiguous) and B
// (CN x kKC, padded rows against bank conflicts) staged in LDS; acc[e] = fma(a_k, b_k, acc[e]) in
// ascending k from 0, exactly fp64_dot's chain.  Rows / columns past the problem load zeros.
template <int RM, int CN>
__device__ __forceinline__ void tile_dots(const oz2_problem& pr, int r0, int cb, int lr, int lc, double* tA,
                                          double* tB, double (&acc)[4]) {
  const GLOBAL double* A = gp(pr.A);
  const GLOBAL double* B = gp(pr.B);
  const size_t lda = (size_t)pr.lda, ldb = (size_t)pr.ldb;
  const int m = pr.m, n = pr.n, K = pr.k;
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = 0.0;
  if (K <= 0) return;   // workgroup-uniform
  // a thread's staging elements: A x = tid + kThreads i (kk = x / RM, r = x % RM), B x = tid when
  // below CN kKC; loaded from clamped (always valid) addresses, all of a chunk in flight at once
  // (no prefetch across chunks: it would take this kernel past 102 VGPRs); values outside the
  // problem stage as zero
  constexpr int NA = kKC * RM / kThreads;
  static_assert(kKC * RM % kThreads == 0 && CN * kKC <= kThreads, "staging split");
  const int tid = threadIdx.x;
  const bool hasB = tid < CN * kKC;
  const int cB = tid / kKC, kB = tid % kKC;
  double va[NA], vb = 0.0;
  auto fetch = [&](int kc) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int x = tid + kThreads * i, kk = x / RM, r = x % RM;
      va[i] = A[(size_t)min(r0 + r, m - 1) + (size_t)min(kc + kk, K - 1) * lda];
    }
    if (hasB) vb = B[(size_t)min(kc + kB, K - 1) + (size_t)min(cb + cB, n - 1) * ldb];
  };
  for (int kc = 0; kc < K; kc += kKC) {
    const int kn = min(kKC, K - kc);
    fetch(kc);
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int x = tid + kThreads * i, kk = x / RM, r = x % RM;
      tA[x] = (r0 + r < m && kk < kn) ? va[i] : 0.0;
    }
    if (hasB) tB[cB * (kKC + 1) + kB] = (cb + cB < n && kB < kn) ? vb : 0.0;
    __syncthreads();
#pragma unroll 4
    for (int kk = 0; kk < kn; ++kk) {
      const double b = tB[lc * (kKC + 1) + kk];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = fma(tA[kk * RM + lr + e], b, acc[e]);
    }
    __syncthreads();
  }
}

template <bool kDigits, bool kBlocked>
__global__ void __launch_bounds__(kThreads) recon_kernel(const oz2_problem* __restrict__ probs,
                                                         const YDesc* __restrict__ yds, int mode,
                                                         const CrtTables* __restrict__ tab,
                                                         unsigned long long* __restrict__ cnt) {
  __shared__ unsigned long long red[3][kThreads / 64];
  const oz2_problem& pr = probs[blockIdx.y];
  const int N = pr.num_moduli;
  const int m = pr.m, n = pr.n, K = pr.k;
  Counts cn{0u, 0u, 0u};
  constexpr int RM = kBlocked ? kBTileM : kTileM, CN = kBlocked ? kBTileN : kTileN;   // tile rows, columns
  // dot products' k-chunks: per wave (blocked layout) or for the whole tile
  __shared__ double tA[kBlocked ? 4 * 16 * kKC : kKC * RM], tB[kBlocked ? 4 * 16 * (kKC + 1) : CN * (kKC + 1)];
  const int tiles_m = (m + RM - 1) / RM;
  const int r0 = ((int)blockIdx.x % max(tiles_m, 1)) * RM, cb = ((int)blockIdx.x / max(tiles_m, 1)) * CN;
  int lr, lc;   // the thread's rows lr .. lr + 3 and column lc inside the tile
  if (kBlocked) {   // a wave per 16 x 16 block, lane = the block's MFMA lane: 4 rows of one column
    const int lane = threadIdx.x & 63;
    lr = 16 * (threadIdx.x >> 6) + 4 * (lane >> 4);
    lc = lane & 15;
  } else {
    lr = 4 * (threadIdx.x & 31);
    lc = threadIdx.x >> 5;
  }
  const int i0 = r0 + lr, j = cb + lc;
  const bool active = N >= 1 && N <= kMaxModuli && m > 0 && n > 0 && i0 < m && j < n;
  const double alpha = pr.alpha, beta = pr.beta;
  const int ne = active ? min(4, m - i0) : 0;
  const bool full = ne == 4 && (m & 3) == 0;
  GLOBAL double* const cp = gpw(pr.C) + (active ? i0 + (size_t)j * pr.ldc : 0);
  unsigned dmask = 0;   // entries that take the FP64 dot product
  if (active) {
    double c0[4] = {0.0, 0.0, 0.0, 0.0};
    double out[4];
    // ---- loads
    if (beta != 0.0) {
      if (full && ((reinterpret_cast<uintptr_t>(cp) & 15) == 0)) {
        const v2d a = *reinterpret_cast<const GLOBAL v2d*>(cp);
        const v2d b = *reinterpret_cast<const GLOBAL v2d*>(cp + 2);
        c0[0] = a.x; c0[1] = a.y; c0[2] = b.x; c0[3] = b.y;
      } else {
        for (int e = 0; e < ne; ++e) c0[e] = cp[e];
      }
    }
    uint32_t yv[kMaxModuli];
    int32_t Lv[4] = {0, 0, 0, 0};
    int rsh[4] = {0, 0, 0, 0}, sig[4] = {0, 0, 0, 0}, dab[4] = {0, 0, 0, 0}, nab[4] = {0, 0, 0, 0};
    int csh = 0, tau = 0, dbb = 0, nbb = 0;
    if (alpha != 0.0) {
      const GLOBAL int32_t* rs = gp(pr.row_shift);
      const GLOBAL int32_t* cs = gp(pr.col_shift);
      if (full) {
        const v4i a = *reinterpret_cast<const GLOBAL v4i*>(rs + i0);
        const v4i b = *reinterpret_cast<const GLOBAL v4i*>(rs + m + i0);
        const v4i c = *reinterpret_cast<const GLOBAL v4i*>(rs + 2 * m + i0);
        const v4i d = *reinterpret_cast<const GLOBAL v4i*>(rs + 3 * m + i0);
        rsh[0] = a.x; rsh[1] = a.y; rsh[2] = a.z; rsh[3] = a.w;
        sig[0] = b.x; sig[1] = b.y; sig[2] = b.z; sig[3] = b.w;
        dab[0] = c.x; dab[1] = c.y; dab[2] = c.z; dab[3] = c.w;
        nab[0] = d.x; nab[1] = d.y; nab[2] = d.z; nab[3] = d.w;
      } else {
        for (int e = 0; e < ne; ++e) {
          rsh[e] = rs[i0 + e]; sig[e] = rs[m + i0 + e]; dab[e] = rs[2 * m + i0 + e]; nab[e] = rs[3 * m + i0 + e];
        }
      }
      csh = cs[j]; tau = cs[n + j]; dbb = cs[2 * n + j]; nbb = cs[3 * n + j];
      // blocked: the 4-entry word always exists (entries past m are padding, never used)
      const size_t off = kBlocked ? blocked_word(i0, j, (m + 15) / 16) : (size_t)i0 + (size_t)j * m;
      if (kDigits) {
        const YDesc yd = yds[blockIdx.y];
        const GLOBAL uint8_t* Y = gp(yd.Y) + off;
#pragma unroll
        for (int l = 0; l < kMaxModuli; ++l) {
          if (l < N) {
            const GLOBAL uint8_t* y = Y + (size_t)l * yd.y_stride;
            if (kBlocked || full) {
              yv[l] = *reinterpret_cast<const GLOBAL uint32_t*>(y);
            } else {
              uint32_t v = 0;
              for (int e = 0; e < ne; ++e) v |= (uint32_t)y[e] << (8 * e);
              yv[l] = v;
            }
          }
        }
        const GLOBAL int32_t* L = gp(yd.L) + off;
        if (kBlocked || full) {
          const v4i a = *reinterpret_cast<const GLOBAL v4i*>(L);
          Lv[0] = a.x; Lv[1] = a.y; Lv[2] = a.z; Lv[3] = a.w;
        } else {
          for (int e = 0; e < ne; ++e) Lv[e] = L[e];
        }
      } else {
        const GLOBAL int32_t* C32 = gp(pr.C32) + off;
        const size_t cst = pr.c32_mod_stride;
#pragma unroll
        for (int l = 0; l < kMaxModuli; ++l) {
          if (l < N) {
            const uint32_t p = (uint32_t)tab->p[l], mg = tab->magic[l], qi = (uint32_t)tab->qinv[N][l];
            uint32_t v = 0;
            for (int e = 0; e < ne; ++e) {
              const int32_t c = C32[l * cst + e];
              const uint32_t uc = c < 0 ? 0u - (uint32_t)c : (uint32_t)c;
              uint32_t r = mod_small(uc, p, mg);
              if (c < 0 && r) r = p - r;
              v |= mod_small(r * qi, p, mg) << (8 * e);
            }
            yv[l] = v;
          }
        }
        for (int e = 0; e < ne; ++e) Lv[e] = C32[N * cst + e];
      }
    }
    // ---- CRT sums of the 4 entries
    uint64_t S1[4] = {0, 0, 0, 0};
    uint32_t S2[4] = {0, 0, 0, 0};
    if (alpha != 0.0) {
#pragma unroll
      for (int l = 0; l < kMaxModuli; ++l) {
        if (l < N) {
          const uint64_t s1 = tab->s1[N][l];
          const uint32_t s2 = tab->s2[N][l];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t y = (yv[l] >> (8 * e)) & 0xffu;
            S1[e] += s1 * (uint64_t)y;
            S2[e] += s2 * y;
          }
        }
      }
    }
    const double u = 0x1p-53;
    const double nt = (double)K + (alpha != 1.0 ? 1.0 : 0.0) + (beta != 0.0 ? 1.0 : 0.0);
    const double gam = (nt * u / (1.0 - nt * u) - 2.0 * u) * (1.0 - 0x1p-40);
    const double db = __int_as_float(dbb), nb = __int_as_float(nbb);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (e < ne) {
        bool dot = false;
        out[e] = entry(pr, tab, N, mode, i0 + e, j, S1[e], S2[e], Lv[e], rsh[e], csh, sig[e], tau,
                       __int_as_float(dab[e]), __int_as_float(nab[e]), db, nb, c0[e], gam, cn, dot);
        dmask |= dot ? 1u << e : 0u;
      }
    // certified entries now; entries taking the dot product keep C0 in C until then
    if (dmask == 0u && full && ((reinterpret_cast<uintptr_t>(cp) & 15) == 0)) {
      *reinterpret_cast<GLOBAL v2d*>(cp) = v2d{out[0], out[1]};
      *reinterpret_cast<GLOBAL v2d*>(cp + 2) = v2d{out[2], out[3]};
    } else {
      for (int e = 0; e < ne; ++e)
        if (!((dmask >> e) & 1u)) cp[e] = out[e];
    }
  }
  // ---- FP64 dot products (sequential fma over k, the reference's fp64_dot order): one per entry
  // when few lanes need them, else a whole block / tile at once through LDS k-chunks (every lane
  // helps; values identical, since each entry is still one fma chain in ascending k).  Blocked
  // layout: per wave, without a workgroup barrier; column-major: per workgroup.
  bool many;
  if (kBlocked) {
    many = __popcll(__ballot(dmask != 0u)) >= kWaveDots;
    if (many) {
      const int w = threadIdx.x >> 6;
      double acc[4];
      wave_dots(pr, r0 + 16 * w, cb, threadIdx.x & 63, tA + w * 16 * kKC, tB + w * 16 * (kKC + 1), acc);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if ((dmask >> e) & 1u) cp[e] = from_dot(alpha, beta, acc[e], beta != 0.0 ? cp[e] : 0.0);
    }
  } else {
    many = __syncthreads_count(dmask != 0u) >= kTileDots;
    if (many) {
      double acc[4];
      tile_dots<RM, CN>(pr, r0, cb, lr, lc, tA, tB, acc);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if ((dmask >> e) & 1u) cp[e] = from_dot(alpha, beta, acc[e], beta != 0.0 ? cp[e] : 0.0);
    }
  }
  if (!many && dmask) {
    for (int e = 0; e < ne; ++e)
      if ((dmask >> e) & 1u) cp[e] = from_dot(alpha, beta, fp64_dot(pr, i0 + e, j), beta != 0.0 ? cp[e] : 0.0);
  }
  // counters: wave reduce, block reduce, one atomic per counter per block (exact integer sums)
  unsigned long long cu = cn.uncert, cr = cn.repair, cf = cn.safety;
#pragma unroll
  for (int o = 32; o; o >>= 1) {
    cu += __shfl_down(cu, o);
    cr += __shfl_down(cr, o);
    cf += __shfl_down(cf, o);
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) { red[0][wid] = cu; red[1][wid] = cr; red[2][wid] = cf; }
  __syncthreads();
  if (threadIdx.x < 3) {
    unsigned long long t = 0;
    for (int w = 0; w < kThreads / 64; ++w) t += red[threadIdx.x][w];
    if (t) atomicAdd(&cnt[1 + threadIdx.x], t);
  }
}

}  // namespace

int recon_launch(const oz2_problem* d, const YDesc* yd, int num, int max_m, int max_n, hipStream_t s, int mode,
                 bool blocked) {
  if (num <= 0) return 0;
  if (mode != OZ2_REPAIR_OFF && mode != OZ2_REPAIR_COUNT && mode != OZ2_REPAIR_ON) return 1;
  if (num > 65535 || max_m < 0 || max_n < 0) return 1;
  DevCtx* c = dev_ctx();
  if (!c) return 2;
  const size_t mn = (size_t)max_m * (size_t)max_n;
  if (mn == 0) return 0;
  // tiles of the largest problem; a problem with fewer tiles returns from the surplus workgroups
  const bool blk = blocked && yd;
  const int tm = blk ? kBTileM : kTileM, tn = blk ? kBTileN : kTileN;
  const size_t gx = (size_t)((max_m + tm - 1) / tm) * (size_t)((max_n + tn - 1) / tn);
  if (gx > 0x7fffffffu) return 1;
  if (blk)
    hipLaunchKernelGGL((recon_kernel<true, true>), dim3((unsigned)gx, num), dim3(kThreads), 0, s, d, yd, mode, c->tab,
                       c->counters);
  else if (yd)
    hipLaunchKernelGGL((recon_kernel<true, false>), dim3((unsigned)gx, num), dim3(kThreads), 0, s, d, yd, mode,
                       c->tab, c->counters);
  else
    hipLaunchKernelGGL((recon_kernel<false, false>), dim3((unsigned)gx, num), dim3(kThreads), 0, s, d, nullptr, mode,
                       c->tab, c->counters);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

}  // namespace ggemm

extern "C" int oz2_reconstruct_grouped(const oz2_problem* d, int num, int max_m, int max_n, hipStream_t s,
                                       int repair_mode) {
  return ggemm::recon_launch(d, nullptr, num, max_m, max_n, s, repair_mode);
}
