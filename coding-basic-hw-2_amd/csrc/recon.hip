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
// the same vectors at element alignment: one 16-byte access wherever its 4 / 2 elements lie (gfx950
// global memory takes dword-aligned vector accesses), for rows of C and of the shift arrays whose
// stride m is not a multiple of 4 -- element-wise accesses there cost the reconstruct of a ragged
// group a fifth of its time
typedef int v4i_e __attribute__((ext_vector_type(4), aligned(4)));
typedef double v2d_e __attribute__((ext_vector_type(2), aligned(8)));

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
  // at once (no prefetch across chunks: it would cost the kernel waves per SIMD); values
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

// The workgroup's problem and tile inside it.  ne > 0: compact grid (workgroup blockIdx.x of the
// tiles of all problems back to back; per > 0: every problem has per tiles, else the problem is the
// last one whose first tile, yds[p].t0 or .d0, is at most blockIdx.x); ne == 0: problem blockIdx.y,
// tile blockIdx.x.
// kGrid: 0 reconstruct tiles (t0), 1 dot-pass tiles (d0), 2 64-row bands (b0), 3 crossings workgroups
// (x0).
template <int kGrid>
__device__ __forceinline__ int grid_first(const YDesc& y) {
  return kGrid == 0 ? y.t0 : (kGrid == 1 ? y.d0 : (kGrid == 2 ? y.b0 : y.x0));
}
template <int kGrid>
__device__ __forceinline__ void grid_tile(const YDesc* __restrict__ yds, int ne, int per, int& p, int& lt) {
  const int g = blockIdx.x;
  if (ne == 0) {
    p = blockIdx.y;
    lt = g;
  } else if (per > 0) {
    p = g / per;
    lt = g - p * per;
  } else {
    int lo = 0, hi = ne - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (grid_first<kGrid>(yds[mid]) <= g) lo = mid; else hi = mid - 1;
    }
    p = lo;
    lt = g - grid_first<kGrid>(yds[lo]);
  }
}

template <bool kDigits, bool kBlocked>
__global__ void __launch_bounds__(kThreads) recon_kernel(const oz2_problem* __restrict__ probs,
                                                         const YDesc* __restrict__ yds, int mode,
                                                         const CrtTables* __restrict__ tab,
                                                         unsigned long long* __restrict__ cnt, int gne, int gper) {
  __shared__ unsigned long long red[3][kThreads / 64];
  int pi, lt;
  grid_tile<0>(yds, gne, gper, pi, lt);
  const oz2_problem& pr = probs[pi];
  const int N = pr.num_moduli;
  const int m = pr.m, n = pr.n, K = pr.k;
  Counts cn{0u, 0u, 0u};
  constexpr int RM = kBlocked ? kBTileM : kTileM, CN = kBlocked ? kBTileN : kTileN;   // tile rows, columns
  // dot products' k-chunks for the whole tile (column-major; the blocked layout leaves its dot
  // products to dots_kernel)
  __shared__ double tA[kBlocked ? 2 : kKC * RM], tB[kBlocked ? 2 : CN * (kKC + 1)];
  const int tiles_m = (m + RM - 1) / RM;
  const int r0 = (lt % max(tiles_m, 1)) * RM, cb = (lt / max(tiles_m, 1)) * CN;
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
  if (kBlocked && threadIdx.x == 0 && m > 0 && n > 0) {   // clear the crossings sets for dots_kernel
    GLOBAL uint64_t* const X = gpw(yds[pi].X);
    if (cb == 0 && r0 < m) X[r0 >> 6] = 0ull;
    if (r0 == 0 && (cb & 63) == 0 && cb < n) X[((m + 63) >> 6) + (cb >> 6)] = 0ull;
  }
  const bool active = N >= 1 && N <= kMaxModuli && m > 0 && n > 0 && i0 < m && j < n;
  const double alpha = pr.alpha, beta = pr.beta;
  const int ne = active ? min(4, m - i0) : 0;
  const bool four = ne == 4;                 // the thread's 4 rows exist
  const bool full = four && (m & 3) == 0;   // ... and column-major digits are 4-byte aligned
  GLOBAL double* const cp = gpw(pr.C) + (active ? i0 + (size_t)j * pr.ldc : 0);
  unsigned dmask = 0;   // entries that take the FP64 dot product
  if (active) {
    double c0[4] = {0.0, 0.0, 0.0, 0.0};
    double out[4];
    // ---- loads
    if (beta != 0.0) {
      if (four) {
        const v2d_e a = *reinterpret_cast<const GLOBAL v2d_e*>(cp);
        const v2d_e b = *reinterpret_cast<const GLOBAL v2d_e*>(cp + 2);
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
      if (four) {
        const v4i_e a = *reinterpret_cast<const GLOBAL v4i_e*>(rs + i0);
        const v4i_e b = *reinterpret_cast<const GLOBAL v4i_e*>(rs + m + i0);
        const v4i_e c = *reinterpret_cast<const GLOBAL v4i_e*>(rs + 2 * m + i0);
        const v4i_e d = *reinterpret_cast<const GLOBAL v4i_e*>(rs + 3 * m + i0);
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
        const YDesc yd = yds[pi];
        const GLOBAL uint8_t* Y = gp(yd.Y) + off;
        auto digits = [&]() {
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
        };
        if (yd.nff) {   // workgroup-uniform
          // a problem with non-finite rows / columns: the shifts first, and no digit for a lane
          // whose every entry takes the safety fallback (its column, or each of its rows, is
          // non-finite; such entries use neither S1, S2 nor L)
          bool fin = false;
#pragma unroll
          for (int e = 0; e < 4; ++e) fin = fin || (e < ne && rsh[e] != OZ2_SHIFT_NONFINITE);
          if (fin && csh != OZ2_SHIFT_NONFINITE) {
            digits();
          } else {
#pragma unroll
            for (int l = 0; l < kMaxModuli; ++l) yv[l] = 0u;
          }
        } else {
          digits();
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
    if (dmask == 0u && four) {
      *reinterpret_cast<GLOBAL v2d_e*>(cp) = v2d_e{out[0], out[1]};
      *reinterpret_cast<GLOBAL v2d_e*>(cp + 2) = v2d_e{out[2], out[3]};
    } else {
      for (int e = 0; e < ne; ++e)
        if (!((dmask >> e) & 1u)) cp[e] = out[e];
    }
  }
  // ---- FP64 dot products (sequential fma over k, the reference's fp64_dot order): one per entry
  // when few lanes need them, else a whole block / tile at once through LDS k-chunks (every lane
  // helps; values identical, since each entry is still one fma chain in ascending k).  Blocked
  // layout: per wave, without a workgroup barrier; column-major: per workgroup.
  bool many = false;
  if (kBlocked) {
    // the wave's block: flag words instead of dot products (the dot-product pass computes them);
    // written for every block of the problem, so no stale flag survives from an earlier call
    const uint64_t f0 = __ballot(dmask & 1u), f1 = __ballot((dmask >> 1) & 1u);
    const uint64_t f2 = __ballot((dmask >> 2) & 1u), f3 = __ballot((dmask >> 3) & 1u);
    const int br = r0 + 16 * (int)(threadIdx.x >> 6);
    if ((threadIdx.x & 63) == 0 && N >= 1 && N <= kMaxModuli && br < m && cb < n) {
      const size_t bidx = (size_t)(cb >> 4) * (size_t)((m + 15) >> 4) + (size_t)(br >> 4);
      GLOBAL uint64_t* F = gpw(yds[pi].F) + 4 * bidx;
      F[0] = f0; F[1] = f1; F[2] = f2; F[3] = f3;
      if (f0 | f1 | f2 | f3) *const_cast<int*>(&yds[pi].fla) = 1;   // (every writer stores the same value)
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
  if (!kBlocked && !many && dmask) {
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
    if (t) atomicAdd(counter_slot(cnt) + 1 + threadIdx.x, t);
  }
}

// ---------------------------------------------------------------- dot-product pass (blocked layout)
// The production reconstruct (blocked layout) computes no FP64 dot product: it leaves C0 in C for
// the entries that take one (safety fallback for rows / columns with NaN / Inf, repair of
// uncertified entries) and flags them, one bit per entry.  dots_kernel then covers a 64 x 64 tile of
// one problem per workgroup: a tile without flags returns after reading its 512 flag bytes;
// otherwise every flagged entry's dot product is one sequential fma chain over k in ascending order
// from 0, as the reference's fp64_dot, whichever of three forms computes it:
//   * dense: when at least a quarter of the tile's entries are flagged, the workgroup computes all 4096
//     chains of the tile at once, each thread a 4 x 4 register block (16 chains), the k-chunks of
//     A (64 rows) and B (64 columns) double-buffered in LDS and read as 32-byte row / column
//     quads that a wave's lanes share (broadcast reads): 4 LDS reads per 16 fmas;
//   * compact: when the flagged entries lie in nR rows and nC columns with nR nC <= kCompactMax,
//     the workgroup stages those rows of A and columns of B once per k-chunk and runs the nR nC
//     chains of their crossings, one per thread (compact_dots);
//   * per block: a block with flagged entries in at least kWaveDots lanes takes them all with 4
//     chains per lane (wave_dots: wave w the blocks of block column w);
//   * sparse: the remaining entries go to a per-workgroup list; for up to 16 entries at a time
//     all 256 threads stage their A rows and B columns through LDS in k-chunks of 64 to 1024 (all
//     of a chunk's loads in flight together, the next chunk's while the chains run), one lane per
//     chain -- instead of one lane loading its A row, lda apart, and its B column itself.
// Before that, the safety-fallback entries are evaluated from prep's non-finite summaries when the
// call has them (nf_dot below); only those it cannot decide, and the repairs, take the chains.
constexpr int kRT = 64;            // tile rows and columns
constexpr int kDenseMin = 1024;    // flagged entries of a tile from which it takes the dense form
constexpr int kDK = 8;             // dense k-chunk
constexpr int kSG = 16;            // sparse: entries per group
constexpr int kListCap = 256;      // sparse list capacity (16 blocks x 3 lanes x 4 entries fit)
constexpr int kCompactMax = 256;   // compact form: rows x columns of the flagged entries, one chain per thread
constexpr int kBandMin = 8;        // flagged entries from which a compact tile defers to the crossings pass
constexpr int kWaveLds = 16 * kKC + 16 * (kKC + 1);   // doubles of one wave's wave_dots staging
constexpr int kUnion = 4 * kWaveLds;                  // wave_dots x 4 waves; >= dense, sparse
static_assert(4 * kDK * kRT <= kUnion && 2 * 1024 <= kUnion, "dot-pass LDS union");

__device__ __forceinline__ void lds_sync() { __syncthreads(); }

// The fp64 dot product of a safety-fallback entry (row i of A or column j of B holds a NaN or an
// Inf) without its chain (the summary rule, applied in dots_kernel).  The chain s = fma(a_k, b_k, s)
// from s = 0 ends non-finite: a product with an infinite factor is +-Inf, or NaN when the other
// factor is 0 or NaN; an infinite s stays so under finite addends and turns NaN under the opposite
// infinity; NaN stays NaN.  Its value is therefore NaN if a NaN factor occurs, if an infinity meets
// a zero or if infinite products of both signs occur, and otherwise the one signed infinity --
// provided no finite partial sum overflows before the first infinite product.  Those sums stay
// below k 2^(eA + 1) 2^(eB + 1) (1 + u)^k < 2^(eA + eB + 3 + ceil(log2 k)) (eA, eB: ilogb of the
// largest finite magnitudes of the row and the column), so eA + eB + 3 + ceil(log2 k) <= 1023 rules
// overflow out.  Outside that bound, when the row or column has more infinities than its summary
// lists, or when none is listed, the entry takes its chain.  The result equals the chain's bit for
// bit except for a NaN's payload.  Row summary words 0 and 1 (or 0 and the exponent from sigma for
// a finite row) give hr / eA, likewise hc / eB for the column; a row infinity at k = w pairs with
// B(w, j), a column infinity with A(i, w).

__device__ __forceinline__ unsigned long long uniform_u64(unsigned long long v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return ((unsigned long long)hi << 32) | lo;
}

// Flagged entries of the tile counted into *c (threads 0 .. 63 read one flag word each).
__device__ __forceinline__ void count_flags(const uint64_t* fl, int* c) {
  const int t = threadIdx.x;
  if (t < 64) {
    int v = __popcll(fl[t]);
#pragma unroll
    for (int o = 32; o; o >>= 1) v += __shfl_down(v, o);
    if (t == 0) *c = v;
  }
}

// flag of tile entry (il, jl): block b = 4 (jl / 16) + il / 16, word il % 4, bit = MFMA lane
// 16 ((il % 16) / 4) + jl % 16
__device__ __forceinline__ bool tile_flag(const uint64_t* fl, int il, int jl) {
  return (fl[4 * (4 * (jl >> 4) + (il >> 4)) + (il & 3)] >> (16 * ((il & 15) >> 2) + (jl & 15))) & 1u;
}

// All 4096 chains of the tile (rows r0 .., columns c0 ..); thread t: tr = 4 (t / 64) + (t % 64) / 16,
// tc = t % 16 owns rows 4 tr .. 4 tr + 3 and columns 4 tc .. 4 tc + 3 of the tile.  The flagged
// entries (fl) are stored: C = alpha d (+ beta C0).
__device__ __forceinline__ void dense_dots(const oz2_problem& pr, int r0, int c0, const uint64_t* fl, double* buf) {
  const GLOBAL double* A = gp(pr.A);
  const GLOBAL double* B = gp(pr.B);
  const size_t lda = (size_t)pr.lda, ldb = (size_t)pr.ldb;
  const int m = pr.m, n = pr.n, K = pr.k;
  const int t = threadIdx.x;
  const int tr = 4 * (t >> 6) + ((t & 63) >> 4), tc = t & 15;
  double* sA = buf;                  // [2][kDK][64]: A chunk, rows contiguous
  double* sB = buf + 2 * kDK * kRT;  // [2][kDK][64]: B chunk, columns contiguous
  double acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = 0.0;
  // staging: A element x = t + 256 s (kk = x / 64, row = x % 64), B element x (col = x / kDK,
  // kk = x % kDK), NS of each per thread, from clamped (always valid) addresses; rows / columns past
  // the problem feed entries never stored, k past K is never read by the chains
  constexpr int NS = kDK * kRT / kThreads;
  static_assert(NS * kThreads == kDK * kRT, "dense staging split");
  double va[NS], vb[NS];
  auto fetch = [&](int kc) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int x = t + kThreads * s;
      va[s] = A[(size_t)min(r0 + x % kRT, m - 1) + (size_t)min(kc + x / kRT, K - 1) * lda];
      vb[s] = B[(size_t)min(kc + x % kDK, K - 1) + (size_t)min(c0 + x / kDK, n - 1) * ldb];
    }
  };
  auto put = [&](int slot) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int x = t + kThreads * s;
      sA[slot * kDK * kRT + x] = va[s];                                  // [kk][row], x = 64 kk + row
      sB[slot * kDK * kRT + (x % kDK) * kRT + x / kDK] = vb[s];          // [kk][col]
    }
  };
  if (K > 0) {
    fetch(0);
    put(0);
  }
  lds_sync();
  int slot = 0;
  for (int kc = 0; kc < K; kc += kDK) {
    const int kn = min(kDK, K - kc);
    const bool more = kc + kDK < K;
    if (more) fetch(kc + kDK);   // the next chunk's loads in flight while this chunk's fmas run
    const double* a_ = sA + slot * kDK * kRT + 4 * tr;
    const double* b_ = sB + slot * kDK * kRT + 4 * tc;
#pragma unroll 2
    for (int kk = 0; kk < kn; ++kk) {
      const v2d a01 = *reinterpret_cast<const v2d*>(a_ + kk * kRT);
      const v2d a23 = *reinterpret_cast<const v2d*>(a_ + kk * kRT + 2);
      const v2d b01 = *reinterpret_cast<const v2d*>(b_ + kk * kRT);
      const v2d b23 = *reinterpret_cast<const v2d*>(b_ + kk * kRT + 2);
      const double av[4] = {a01.x, a01.y, a23.x, a23.y}, bv[4] = {b01.x, b01.y, b23.x, b23.y};
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = fma(av[a], bv[b], acc[a][b]);
    }
    if (more) put(slot ^ 1);   // the other slot: every thread finished reading it before the last barrier
    lds_sync();
    slot ^= 1;
  }
  const double alpha = pr.alpha, beta = pr.beta;
  GLOBAL double* const C = gpw(pr.C);
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int jl = 4 * tc + b, j = c0 + jl;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int il = 4 * tr + a, i = r0 + il;
      if (i < m && j < n && tile_flag(fl, il, jl)) {
        GLOBAL double* cp = C + i + (size_t)j * pr.ldc;
        *cp = from_dot(alpha, beta, acc[a][b], beta != 0.0 ? *cp : 0.0);
      }
    }
  }
}

// The chains of the crossings of nR tile rows (rmap) and nC tile columns (cmap), nR nC <= kCompactMax:
// thread t < nR nC runs the chain of row rmap[t / nC], column cmap[t % nC] and stores it if that
// entry is flagged.  Per k-chunk of KC (the largest power of two with nRp + nC rows of KC + 2
// doubles in the LDS union and at most NS staging loads per thread; nRp = nR rounded up to a power
// of two) the rows of A are staged with consecutive threads on consecutive rows (A is column-major)
// and the columns of B with consecutive threads on consecutive k, the next chunk's loads in flight
// while the chains run; a chain reads its row and column two k at a time (16-byte LDS reads; KC + 2
// is even).
__device__ __forceinline__ void compact_dots(const oz2_problem& pr, int r0, int c0, const uint64_t* fl,
                                             const uint8_t* rmap, const uint8_t* cmap, int nR, int nC,
                                             double* buf) {
  const GLOBAL double* A = gp(pr.A);
  const GLOBAL double* B = gp(pr.B);
  const size_t lda = (size_t)pr.lda, ldb = (size_t)pr.ldb;
  const int K = pr.k;
  const int t = threadIdx.x;
  const int lr = nR > 1 ? 32 - __clz(nR - 1) : 0;   // nRp = 2^lr >= nR
  const int nq = (1 << lr) + nC;
  constexpr int NS = 4;   // staging loads per thread (6 cost the kernel its sixth wave per SIMD)
  const int kcap = min(kUnion / nq - 2, NS * kThreads / nq);
  const int lg = 31 - __clz(kcap);   // KC = 2^lg <= kcap
  const int KC = 1 << lg, S = KC + 2;
  const int nA = KC << lr, nS = nq * KC;   // staging elements: A rows (padded to nRp), B columns
  double v[NS];
  auto fetch = [&](int kc) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int x = t + kThreads * s;
      if (x < nA) {
        const int q = x & ((1 << lr) - 1), kk = x >> lr;
        if (q < nR) v[s] = A[(size_t)(r0 + rmap[q]) + (size_t)min(kc + kk, K - 1) * lda];
      } else if (x < nS) {
        const int y = x - nA, q = y >> lg, kk = y & (KC - 1);
        v[s] = B[(size_t)min(kc + kk, K - 1) + (size_t)(c0 + cmap[q]) * ldb];
      }
    }
  };
  auto put = [&](double* dst) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int x = t + kThreads * s;
      if (x < nA) {
        const int q = x & ((1 << lr) - 1);
        if (q < nR) dst[q * S + (x >> lr)] = v[s];
      } else if (x < nS) {
        const int y = x - nA;
        dst[(nR + (y >> lg)) * S + (y & (KC - 1))] = v[s];
      }
    }
  };
  // two chunk buffers when the LDS union holds them at this chunk length: chunk i + 1 is staged
  // into the other buffer while chunk i's chains run, one barrier per chunk; else one buffer, the
  // next chunk staged after a barrier
  const bool two = 2 * nq * S <= kUnion;
  const int nb = nq * S;   // doubles per chunk buffer
  const bool act = t < nR * nC;
  const int cr = act ? t / nC : 0, cc = act ? t - cr * nC : 0;
  const int ao = cr * S, bo = (nR + cc) * S;
  double acc = 0.0;
  if (K > 0) {
    fetch(0);
    put(buf);
    if (two && KC < K) fetch(KC);
  }
  lds_sync();
  int cur = 0;
  for (int kc = 0; kc < K; kc += KC) {
    const int kn = min(KC, K - kc);
    const bool more = kc + KC < K;
    if (!two && more) fetch(kc + KC);   // in flight while the chains run
    if (act) {
      const double* a_ = buf + cur * nb + ao;
      const double* b_ = buf + cur * nb + bo;
      int kk = 0;
#pragma unroll 2
      for (; kk + 2 <= kn; kk += 2) {
        const v2d a2 = *reinterpret_cast<const v2d*>(a_ + kk);
        const v2d b2 = *reinterpret_cast<const v2d*>(b_ + kk);
        acc = fma(a2.x, b2.x, acc);
        acc = fma(a2.y, b2.y, acc);
      }
      if (kk < kn) acc = fma(a_[kk], b_[kk], acc);
    }
    if (two) {
      if (more) {
        put(buf + (cur ^ 1) * nb);   // chunk kc + KC (the other buffer's last readers passed a barrier)
        if (kc + 2 * KC < K) fetch(kc + 2 * KC);
      }
      lds_sync();   // chunk kc's chains done, chunk kc + KC staged
      cur ^= 1;
    } else {
      lds_sync();   // every chain done with this chunk
      if (more) {
        put(buf);
        lds_sync();
      }
    }
  }
  if (act) {
    const int il = rmap[cr], jl = cmap[cc];
    if (tile_flag(fl, il, jl)) {
      GLOBAL double* cp = gpw(pr.C) + (size_t)(r0 + il) + (size_t)(c0 + jl) * pr.ldc;
      *cp = from_dot(pr.alpha, pr.beta, acc, pr.beta != 0.0 ? *cp : 0.0);
    }
  }
}

// The listed entries (tile-local row / column, packed 16 + 16 bits) in groups of at most kSG: lane e
// of the group runs entry e's chain; all threads stage the group's A rows and B columns through LDS
// in k-chunks of 1024 / (group size rounded up to a power of two) -- 4 loads of A and 4 of B per
// thread and chunk, the next chunk's in flight while the chains run on this one.
__device__ __forceinline__ void sparse_dots(const oz2_problem& pr, int r0, int c0, const uint32_t* list, int L,
                                            double* buf) {
  const GLOBAL double* A = gp(pr.A);
  const GLOBAL double* B = gp(pr.B);
  const size_t lda = (size_t)pr.lda, ldb = (size_t)pr.ldb;
  const int K = pr.k;
  const int t = threadIdx.x;
  double* sA = buf;          // [group entry][chunk]
  double* sB = buf + 1024;   // [group entry][chunk]
  for (int g0 = 0; g0 < L; g0 += kSG) {
    const int gl = min(kSG, L - g0);
    const int lg = 32 - __clz(gl - 1);   // ceil(log2 gl): gl <= 1 << lg
    const int ch = 1024 >> lg;           // k-chunk
    // staging element x = t + 256 s: entry x >> (10 - lg), kk = x & (ch - 1); entries >= gl load a
    // clamped copy of the last one (never read)
    double va[4], vb[4];
    auto fetch = [&](int kc) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int x = t + 256 * s;
        const int e = min(x >> (10 - lg), gl - 1), kk = min(kc + (x & (ch - 1)), K - 1);
        const uint32_t w = list[g0 + e];
        va[s] = A[(size_t)(r0 + (int)(w & 0xffffu)) + (size_t)kk * lda];
        vb[s] = B[(size_t)kk + (size_t)(c0 + (int)(w >> 16)) * ldb];
      }
    };
    auto put = [&]() {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        sA[t + 256 * s] = va[s];
        sB[t + 256 * s] = vb[s];
      }
    };
    double acc = 0.0;
    if (K > 0) {
      fetch(0);
      put();
    }
    lds_sync();
    for (int kc = 0; kc < K; kc += ch) {
      const int kn = min(ch, K - kc);
      const bool more = kc + ch < K;
      if (more) fetch(kc + ch);   // in flight while the chains run
      if (t < gl) {
        const double* a_ = sA + t * ch;
        const double* b_ = sB + t * ch;
        for (int kk = 0; kk < kn; ++kk) acc = fma(a_[kk], b_[kk], acc);
      }
      lds_sync();   // every chain done with this chunk
      if (more) {
        put();
        lds_sync();
      }
    }
    if (t < gl) {
      const uint32_t w = list[g0 + t];
      GLOBAL double* cp = gpw(pr.C) + (size_t)(r0 + (int)(w & 0xffffu)) + (size_t)(c0 + (int)(w >> 16)) * pr.ldc;
      *cp = from_dot(pr.alpha, pr.beta, acc, pr.beta != 0.0 ? *cp : 0.0);
    }
    lds_sync();   // the next group's staging overwrites this group's chunk
  }
}

// (launch bounds: seven waves per SIMD, which the summaries' partner loads and the chains' latency
// need, at a few spilled registers; six: 3-6 % slower on 32 x 2048^3 + 4 x 2048^2 x 65536 products
// with 0.1 % NaN / Inf entries)
__global__ void __launch_bounds__(kThreads, 7) dots_kernel(const oz2_problem* __restrict__ probs,
                                                        const YDesc* __restrict__ yds, int gne, int gper, int form) {
  __shared__ __attribute__((aligned(16))) double buf[kUnion];
  __shared__ uint64_t fl[64];       // flag words of the tile's 16 blocks (4 per block, column-major blocks)
  __shared__ uint32_t list[kListCap];
  __shared__ int cnt[2];            // flagged entries of the tile, listed entries
  __shared__ unsigned long long rcm[2];   // tile rows / columns holding flagged entries
  __shared__ uint8_t rmap[kRT], cmap[kRT];
  int pi, lt;
  grid_tile<1>(yds, gne, gper, pi, lt);
  const oz2_problem& pr = probs[pi];
  const int N = pr.num_moduli;
  const int m = pr.m, n = pr.n;
  const int tiles_m = (m + kRT - 1) / kRT;
  const int r0 = (lt % max(tiles_m, 1)) * kRT, c0 = (lt / max(tiles_m, 1)) * kRT;
  // workgroup-uniform: invalid problems, alpha = 0 (no dot product) and tiles past the problem
  if (N < 1 || N > kMaxModuli || m <= 0 || n <= 0 || r0 >= m || c0 >= n || pr.alpha == 0.0) return;
  if (!yds[pi].fla) return;   // the reconstruct flagged no entry of the problem
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const double alpha = pr.alpha, beta = pr.beta;
  const int mb = (m + 15) >> 4;
  // Problems with NaN / Inf rows or columns (nff; the only ones with safety-fallback entries):
  // the summaries of the thread's row (il = t % 64) and of the tile's column t (threads 0 .. 63) are
  // loaded with the flag words, whether or not the tile turns out to need them (in bounds for
  // every row and column; a finite row's words are never used), so that the safety evaluation
  // below starts without a chain of dependent loads.
  const GLOBAL int32_t* const nf = gp(yds[pi].nf);
  const bool nfp = nf != nullptr && yds[pi].nff != 0;   // workgroup-uniform
  const int il = t & 63, i = r0 + il;
  // word q of a summary held in four int4 values (passed by value: an array whose address a helper
  // takes stays in scratch; q is known at compile time after unrolling)
  static_assert(kNfWords == 16, "summaries of four int4");
  auto word = [](v4i a, v4i b, v4i c, v4i d, int q) __attribute__((always_inline)) {
    const v4i x = q < 4 ? a : (q < 8 ? b : (q < 12 ? c : d));
    return (q & 3) == 0 ? x.x : ((q & 3) == 1 ? x.y : ((q & 3) == 2 ? x.z : x.w));
  };
  int* const cinf = reinterpret_cast<int*>(buf);   // [64][4]: non-finite column, h word, exponent, listed
  int* const clst = cinf + 4 * kRT;                // [64][kNfCap]: the column's infinities
  v4i rw0 = v4i{0, 0, 0, 0}, rw1 = rw0, rw2 = rw0, rw3 = rw0;
  int rsh = 0, rsg = 0;
  if (nfp) {
    if (i < m) {
      const GLOBAL int32_t* rs = gp(pr.row_shift);
      rsh = rs[i];
      rsg = rs[m + i];
      const GLOBAL v4i* R = reinterpret_cast<const GLOBAL v4i*>(nf + (size_t)kNfWords * i);
      rw0 = R[0];
      rw1 = R[1];
      rw2 = R[2];
      rw3 = R[3];
    }
    if (t < kRT) {   // column c0 + t: its summary to LDS (read after the flag count's barrier)
      int cnf = 0, hc = 0, eB = kNfNoFinite, nc = 0;
      const int j = c0 + t;
      if (j < n) {
        const GLOBAL int32_t* cs = gp(pr.col_shift);
        const int csh = cs[j], ctau = cs[n + j];
        const GLOBAL v4i* Cl = reinterpret_cast<const GLOBAL v4i*>(nf + (size_t)kNfWords * ((size_t)m + j));
        const v4i cw0 = Cl[0], cw1 = Cl[1], cw2 = Cl[2], cw3 = Cl[3];
        if (csh == OZ2_SHIFT_NONFINITE) {
          cnf = 1;
          hc = cw0.x;
          eB = cw0.y;
          nc = min((hc >> 8) & 0xff, kNfCap);
#pragma unroll
          for (int s = 0; s < kNfCap; ++s)
            if (s < nc) clst[t * kNfCap + s] = word(cw0, cw1, cw2, cw3, 2 + s);
        } else {
          eB = ctau == OZ2_SHIFT_ZERO ? kNfNoFinite : 6 - ctau;
        }
      }
      cinf[4 * t] = cnf;
      cinf[4 * t + 1] = hc;
      cinf[4 * t + 2] = eB;
      cinf[4 * t + 3] = nc;
    }
  }
  if (t < 64) {   // word t % 4 of block t / 4 = (bi, bj) = (t / 4 % 4, t / 16)
    const int bi = (r0 >> 4) + ((t >> 2) & 3), bj = (c0 >> 4) + (t >> 4);
    fl[t] = (bi < mb && bj * 16 < n) ? gp(yds[pi].F)[4 * ((size_t)bj * mb + bi) + (t & 3)] : 0ull;
    if (t == 0) {
      cnt[1] = 0;
      rcm[0] = rcm[1] = 0ull;
    }
  }
  count_flags(fl, &cnt[0]);
  lds_sync();
  int total = cnt[0];
  if (total == 0) return;   // workgroup-uniform
  // The tile had flags.  On every way out it leaves in the global flags exactly the entries it
  // defers to the crossings pass (cross_kernel): the remaining flags when it defers, zeros otherwise.
  GLOBAL uint64_t* const Fg = gpw(yds[pi].F);
  auto publish = [&](bool deferred) {
    if (t < 64) {
      const int bi = (r0 >> 4) + ((t >> 2) & 3), bj = (c0 >> 4) + (t >> 4);
      if (bi < mb && bj * 16 < n) Fg[4 * ((size_t)bj * mb + bi) + (t & 3)] = deferred ? fl[t] : 0ull;
    }
  };
  if (nfp) {
    // safety-fallback entries from the summaries (nf_dot's rule): thread t takes row il of the tile
    // in columns jl = 16 (t / 64) .. + 15; decided entries are stored and their flags cleared.  The
    // tile's 64 column summaries are in LDS, a thread keeps its row's in registers, and the
    // partner loads for one listed infinity go out four entries at a time, row infinities and
    // column infinities together.
    const int jb = 16 * (t >> 6);
    const int K = pr.k;
    const int lk = K > 1 ? 32 - __clz(K - 1) : 0;
    unsigned cand = 0u, nanm = 0u, posm = 0u, negm = 0u;   // bit q: column jb + q
    int hr = 0, eA = kNfNoFinite, nr = 0;
    if (i < m) {
      const bool rnf = rsh == OZ2_SHIFT_NONFINITE;
      eA = rsg == OZ2_SHIFT_ZERO ? kNfNoFinite : 6 - rsg;
      if (rnf) {
        hr = rw0.x;
        eA = rw0.y;
      }
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int jl = jb + q;
        const int wi = 4 * (4 * (jl >> 4) + (il >> 4)) + (il & 3);
        const uint64_t bit = 1ull << (16 * ((il & 15) >> 2) + (jl & 15));
        if (c0 + jl >= n || !(fl[wi] & bit)) continue;
        const int cnf = cinf[4 * jl], hc = cinf[4 * jl + 1], eB = cinf[4 * jl + 2];
        if (!rnf && !cnf) continue;   // a repair
        if ((hr | hc) & 1) {          // a NaN factor: NaN
          nanm |= 1u << q;
          continue;
        }
        if (((hr | hc) & 2) || eA + eB + 3 + lk > 1023) continue;   // its chain decides
        cand |= 1u << q;
      }
      nr = cand ? min((hr >> 8) & 0xff, kNfCap) : 0;
    }
    // a partner x of an infinity of sign ng: NaN for 0 or NaN, else the product's sign
    auto cls = [&](double x, bool ng, int q) {   // selects, not branches (no mask array in scratch)
      const unsigned b = 1u << q;
      const bool z = x == 0.0 || isnan(x), o = ng != (x < 0.0);
      nanm |= z ? b : 0u;
      negm |= (!z && o) ? b : 0u;
      posm |= (!z && !o) ? b : 0u;
    };
    // listed infinity s of the row (B(w, j) for every candidate column j) and of each column
    // (A(i, w); a wave's 16 columns are the same in every lane)
    int nrm = nr, ncm = 0;
#pragma unroll
    for (int o = 32; o; o >>= 1) nrm = max(nrm, __shfl_xor(nrm, o));
#pragma unroll
    for (int q = 0; q < 16; ++q) ncm = max(ncm, cinf[4 * (jb + q) + 3]);
    const int sm = max(nrm, ncm);   // wave-uniform
    const GLOBAL double* const Bg = gp(pr.B);
    const GLOBAL double* const Ag = gp(pr.A);
    const size_t ldb = (size_t)pr.ldb, lda = (size_t)pr.lda;
    const int jbu = 16 * __builtin_amdgcn_readfirstlane(t >> 6);   // jb, known uniform
#pragma unroll 1
    for (int s = 0; s < sm; ++s) {   // wave-uniform trip count
      {
        const bool ract = s < nr;
        int wr = 0;   // word 2 + s of the row summary (s is not a compile-time index here)
#pragma unroll
        for (int q = 0; q < kNfCap; ++q) wr = q == s ? word(rw0, rw1, rw2, rw3, 2 + q) : wr;
        wr = ract ? wr : 0;
#pragma unroll
        for (int h = 0; h < 16; h += 4) {   // 4 + 4 loads at a time (the kernel's register budget)
          double xr[4], xc[4];
          int wc[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const bool rq = ract && ((cand >> (h + q)) & 1u);
            xr[q] = rq ? Bg[(size_t)(wr & 0x7fffffff) + (size_t)(c0 + jbu + h + q) * ldb] : 0.0;
            const bool cq = ((cand >> (h + q)) & 1u) && s < cinf[4 * (jb + h + q) + 3];
            wc[q] = cq ? clst[(jb + h + q) * kNfCap + s] : 0;
            xc[q] = cq ? Ag[(size_t)i + (size_t)(wc[q] & 0x7fffffff) * lda] : 0.0;
          }
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            if (ract && ((cand >> (h + q)) & 1u)) cls(xr[q], wr < 0, h + q);
            if (((cand >> (h + q)) & 1u) && s < cinf[4 * (jb + h + q) + 3]) cls(xc[q], wc[q] < 0, h + q);
          }
        }
      }
    }
    // decided entries: NaN if a NaN factor, a zero / NaN partner or products of both signs
    // occur, else the one signed infinity; a candidate with no partner keeps its chain
    const unsigned dec = nanm | posm | negm;
#pragma unroll
    for (int h = 0; h < 16; h += 8) {
      double cv[8];
#pragma unroll
      for (int q = 0; q < 8; ++q)
        cv[q] = (beta != 0.0 && ((dec >> (h + q)) & 1u)) ? gp(pr.C)[(size_t)i + (size_t)(c0 + jb + h + q) * pr.ldc] : 0.0;
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if ((dec >> (h + q)) & 1u) {
          const int jl = jb + h + q;
          const bool isnan_ = ((nanm >> (h + q)) & 1u) || (((posm & negm) >> (h + q)) & 1u);
          const double d = isnan_ ? __builtin_nan("") : (((posm >> (h + q)) & 1u) ? __builtin_inf() : -__builtin_inf());
          gpw(pr.C)[(size_t)i + (size_t)(c0 + jl) * pr.ldc] = from_dot(alpha, beta, d, cv[q]);
        }
    }
    // clear the decided flags: lanes il, il + 4, il + 8, il + 12 share the flag word of their
    // block row and quarter -- their 16-bit masks merged by two shuffles, one LDS and per word
    {
      const int wi = 4 * (4 * (jb >> 4) + (il >> 4)) + (il & 3);
      uint64_t mk = (uint64_t)(dec & 0xffffu) << (16 * ((il & 15) >> 2));
      mk |= __shfl_xor(mk, 4);
      mk |= __shfl_xor(mk, 8);
      if (((il >> 2) & 3) == 0 && mk) atomicAnd(reinterpret_cast<unsigned long long*>(&fl[wi]), ~(unsigned long long)mk);
    }
    lds_sync();
    count_flags(fl, &cnt[0]);
    lds_sync();
    total = cnt[0];
    if (total == 0) {   // workgroup-uniform
      publish(false);
      return;
    }
  }
  const bool autof = form == kDotFormAuto || form == kDotFormTile;
  if (form == kDotFormDense || (autof && total >= kDenseMin)) {
    publish(false);
    dense_dots(pr, r0, c0, fl, buf);
    return;
  }
  if (autof && t < 64) {   // rows and columns of the flagged entries: word t covers rows 16 bi + 4 q + e, columns 16 bj + c
    const uint64_t v = fl[t];
    const int bi = (t >> 2) & 3, bj = t >> 4, e = t & 3;
    unsigned long long rb = 0ull;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if ((v >> (16 * q)) & 0xffffull) rb |= 1ull << (16 * bi + 4 * q + e);
    const unsigned long long cbits = ((v | (v >> 16) | (v >> 32) | (v >> 48)) & 0xffffull) << (16 * bj);
    if (rb) atomicOr(&rcm[0], rb);
    if (cbits) atomicOr(&rcm[1], cbits);
  }
  lds_sync();
  // workgroup-uniform: moved to scalar registers, and everything derived from them with them
  const unsigned long long rmask = uniform_u64(rcm[0]), cmask = uniform_u64(rcm[1]);
  const int nR = __popcll(rmask), nC = __popcll(cmask);
  if (autof && nR * nC <= kCompactMax) {   // workgroup-uniform
    // dense crossings with enough chains go to the crossings pass, which runs the crossings of all
    // deferred rows and columns of the problem as one GEMM on the matrix cores (needs the gather
    // workspace AT)
    const bool defer = form == kDotFormAuto && yds[pi].AT && total >= kBandMin && 2 * total >= nR * nC;
    publish(defer);
    if (defer) {
      if (t == 0) {
        unsigned long long* const X = reinterpret_cast<unsigned long long*>(yds[pi].X);
        atomicOr(&X[r0 >> 6], rmask);
        atomicOr(&X[((m + 63) >> 6) + (c0 >> 6)], cmask);
      }
      return;
    }
    if (t < 64) {
      if ((rmask >> t) & 1ull) rmap[__popcll(rmask & ((1ull << t) - 1ull))] = (uint8_t)t;
      if ((cmask >> t) & 1ull) cmap[__popcll(cmask & ((1ull << t) - 1ull))] = (uint8_t)t;
    }
    lds_sync();
    compact_dots(pr, r0, c0, fl, rmap, cmap, nR, nC, buf);
    return;
  }
  publish(false);
  const int j = c0 + 16 * w + (lane & 15);
  for (int bi = 0; bi < 4; ++bi) {   // wave w: the blocks (bi, w)
    const int i0 = r0 + 16 * bi + 4 * (lane >> 4);
    unsigned dm = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) dm |= (unsigned)((fl[4 * (4 * w + bi) + e] >> lane) & 1u) << e;
    GLOBAL double* const cp = gpw(pr.C) + (dm ? i0 + (size_t)j * pr.ldc : 0);
    if (form != kDotFormList && __popcll(__ballot(dm != 0u)) >= kWaveDots) {   // wave-uniform
      double acc[4];
      wave_dots(pr, r0 + 16 * bi, c0 + 16 * w, lane, buf + w * kWaveLds, buf + w * kWaveLds + 16 * kKC, acc);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if ((dm >> e) & 1u) cp[e] = from_dot(alpha, beta, acc[e], beta != 0.0 ? cp[e] : 0.0);
    } else if (dm) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if ((dm >> e) & 1u) {
          const int x = atomicAdd(&cnt[1], 1);
          if (x < kListCap) list[x] = (uint32_t)(i0 + e - r0) | ((uint32_t)(j - c0) << 16);
          else cp[e] = from_dot(alpha, beta, fp64_dot(pr, i0 + e, j), beta != 0.0 ? cp[e] : 0.0);
        }
    }
  }
  lds_sync();
  const int L = min(cnt[1], kListCap);
  if (L > 0) sparse_dots(pr, r0, c0, list, L, buf);   // L is workgroup-uniform
}


// ---------------------------------------------------------------- crossings pass of the dot products
// The chains dots_kernel deferred: 64 x 64 tiles whose remaining flagged entries form dense
// crossings of a few rows and columns leave exactly those flags in the global flag words (the
// other tiles leave zeros) and add their rows and columns to the problem's crossings sets X (bit
// words: ceil(m / 64) for the rows, then ceil(n / 64) for the columns, cleared by the
// reconstruct).  The crossings of the two sets, R x C, then run as one small GEMM per problem on
// the FP64 matrix cores: gather_kernel copies the rows of R row-major and compact (row x of R at
// AT + x k), as each deferred chain would otherwise read its row of column-major A a line per
// value, and cross_kernel computes 64 x 64 tiles of R x C, 16 x 16 blocks per MFMA.
//
// v_mfma_f64_16x16x4f64 adds its four products to each accumulator as four sequential IEEE fmas in
// k order (c -> k0 -> k1 -> k2 -> k3, each rounded; signed zeros, subnormals and infinities
// included), so a block's chains over k = 4 t + g, t = 0, 1, .. from a zero accumulator are bit for
// bit the sequential fma chains in ascending k from 0 of the reference's fp64_dot
// (src/ozaki2_numerics.cu:445-452); k past the problem's k pads A with +0 and B with -0, whose
// product -0 leaves every accumulator unchanged (+0 + -0 = +0 and -0 + -0 = -0 included).
// Crossings whose flag is set are stored, the others are computed and dropped.

// Sum of v over the workgroup (every thread gets it); ws: 4 ints of LDS, free again on return.
__device__ __forceinline__ int block_sum(int v, int* ws) {
#pragma unroll
  for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o);
  if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = v;
  lds_sync();
  int s = 0;
#pragma unroll
  for (int x = 0; x < kThreads / 64; ++x) s += ws[x];
  lds_sync();
  return s;
}

// Positions lo .. lo + 63 of the set bits of the nw words at Xw (bit b of word w is position
// 64 w + b, counted in ascending order) into map[0 .. 63]; ws: 4 ints of LDS.  Thread t takes the
// words [t per, (t + 1) per): its count, the workgroup's exclusive prefix of the counts, then the
// walk of its words' bits that fall in the window.  Free of races on map and ws on return.
__device__ void select_bits(const GLOBAL uint64_t* __restrict__ Xw, int nw, int lo, int* map, int* ws) {
  const int t = threadIdx.x, lane = t & 63;
  const int per = (nw + kThreads - 1) / kThreads, w0 = min(nw, t * per), w1 = min(nw, w0 + per);
  int c = 0;
  for (int x = w0; x < w1; ++x) c += __popcll(Xw[x]);
  int inc = c;   // inclusive prefix in the wave
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(inc, o);
    if (lane >= o) inc += y;
  }
  if (lane == 63) ws[t >> 6] = inc;
  lds_sync();
  int pos = inc - c;
#pragma unroll
  for (int x = 0; x < kThreads / 64; ++x) pos += x < (t >> 6) ? ws[x] : 0;
  for (int x = w0; x < w1 && pos < lo + 64; ++x) {
    uint64_t v = Xw[x];
    const int pc = __popcll(v);
    if (pos + pc <= lo) {
      pos += pc;
      continue;
    }
    while (v) {
      if (pos >= lo && pos < lo + 64) map[pos - lo] = 64 * x + __builtin_ctzll(v);
      ++pos;
      v &= v - 1;
    }
  }
  lds_sync();
}

constexpr int kGK = 64;   // gather: k per round

// One workgroup per 64-row band of a problem (the row words of X): the band's rows of R copied to
// AT at their positions in R, kGK values of k per round -- every lane loads one row of the band at
// consecutive addresses (16-row groups without a row of R skipped), then each wave writes a row's
// kGK values contiguously.  Band 0 also stores |R| and |C| in X's last word.
__global__ void __launch_bounds__(kThreads) gather_kernel(const oz2_problem* __restrict__ probs,
                                                         const YDesc* __restrict__ yds, int gne, int gper) {
  __shared__ double T[kGK][kRT + 1];   // [k][band row], padded
  __shared__ int rl[kRT];
  __shared__ int ws[kThreads / 64];
  int pi, band;
  grid_tile<2>(yds, gne, gper, pi, band);
  const oz2_problem& pr = probs[pi];
  const int N = pr.num_moduli, m = pr.m, n = pr.n, K = pr.k;
  const int r0 = band * kRT;
  // workgroup-uniform: invalid problems, alpha = 0, bands past the problem, no deferral possible
  if (N < 1 || N > kMaxModuli || m <= 0 || n <= 0 || K <= 0 || r0 >= m || pr.alpha == 0.0) return;
  if (!yds[pi].fla || !yds[pi].AT) return;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int m64 = (m + 63) >> 6, n64 = (n + 63) >> 6;
  GLOBAL uint64_t* const X = gpw(yds[pi].X);
  if (band == 0) {
    int cr = 0, cc = 0;
    for (int x = t; x < m64; x += kThreads) cr += __popcll(X[x]);
    for (int x = t; x < n64; x += kThreads) cc += __popcll(X[m64 + x]);
    cr = block_sum(cr, ws);
    cc = block_sum(cc, ws);
    if (t == 0) X[m64 + n64] = (uint64_t)(uint32_t)cr | ((uint64_t)(uint32_t)cc << 32);
  }
  const uint64_t bits = X[band];
  if (bits == 0ull) return;   // workgroup-uniform
  int before = 0;   // rows of R in the bands before
  for (int x = t; x < band; x += kThreads) before += __popcll(X[x]);
  before = block_sum(before, ws);
  const int nb = __popcll(bits);
  if ((bits >> lane) & 1ull && w == 0) rl[__popcll(bits & ((1ull << lane) - 1ull))] = lane;
  lds_sync();
  const GLOBAL double* const A = gp(pr.A);
  GLOBAL double* const AT = gpw(yds[pi].AT);
  const size_t lda = (size_t)pr.lda;
  const bool load = r0 + lane < m && ((bits >> (lane & ~15)) & 0xffffull) != 0ull;
  for (int k0 = 0; k0 < K; k0 += kGK) {
    if (load) {
      double v[kGK / 4];
#pragma unroll
      for (int s2 = 0; s2 < kGK / 4; ++s2) {
        const int kk = w + 4 * s2;
        v[s2] = k0 + kk < K ? A[(size_t)(r0 + lane) + (size_t)(k0 + kk) * lda] : 0.0;
      }
#pragma unroll
      for (int s2 = 0; s2 < kGK / 4; ++s2) T[w + 4 * s2][lane] = v[s2];
    }
    lds_sync();
    for (int q = w; q < nb; q += kThreads / 64) {
      if (k0 + lane < K) AT[(size_t)(before + q) * (size_t)K + (size_t)(k0 + lane)] = T[lane][rl[q]];
    }
    lds_sync();
  }
}

constexpr int kXK = 16;        // k per staged chunk
constexpr int kXS = kXK + 2;   // LDS doubles per staged row / column (padded)
constexpr int kXLoads = 2 * kRT * kXK / kThreads;   // staging loads per thread and chunk
typedef double v4d __attribute__((ext_vector_type(4)));

// The 64 x 64 tiles (ti, tj) of R x C, a few workgroups per problem (yds[p].xn of them, in
// proportion to its dot-pass tiles; tiles t = workgroup, + xn, ..): rows 64 ti .. of R (from AT)
// and columns 64 tj .. of C (B's columns) staged through LDS in k-chunks of kXK, row / column slot
// major, double-buffered with the next chunk's loads in registers while the matrix cores run; wave w
// owns the 2 x 2 blocks of block rows 2 (w % 2) .. and block columns 2 (w / 2) .., its next k-step's
// operands read from LDS while the current step's MFMAs run.
__global__ void __launch_bounds__(kThreads, 4) cross_kernel(const oz2_problem* __restrict__ probs,
                                                           const YDesc* __restrict__ yds, int gne, int gper) {
  __shared__ __attribute__((aligned(16))) double xs[2][2 * kRT * kXS];   // [buffer][A slots | B slots]
  __shared__ int rmap[kRT], cmap[kRT];
  __shared__ int ws[kThreads / 64];
  int pi, wi;
  grid_tile<3>(yds, gne, gper, pi, wi);
  const int P = gne == 0 ? (int)gridDim.x : yds[pi].xn;   // the problem's workgroups
  const oz2_problem& pr = probs[pi];
  const int N = pr.num_moduli, m = pr.m, n = pr.n, K = pr.k;
  // workgroup-uniform: invalid problems, alpha = 0 (no dot product), nothing deferred
  if (N < 1 || N > kMaxModuli || m <= 0 || n <= 0 || K <= 0 || pr.alpha == 0.0) return;
  if (!yds[pi].fla || !yds[pi].AT) return;
  const int m64 = (m + 63) >> 6, n64 = (n + 63) >> 6;
  const GLOBAL uint64_t* const X = gp(yds[pi].X);
  const uint64_t tot = X[m64 + n64];
  const int nR = (int)(uint32_t)tot, nC = (int)(uint32_t)(tot >> 32);
  const int ntr = (nR + kRT - 1) / kRT, ntiles = ntr * ((nC + kRT - 1) / kRT);
  if (wi >= ntiles) return;   // workgroup-uniform
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const GLOBAL double* const B = gp(pr.B);
  const size_t ldb = (size_t)pr.ldb;
  const int mb = (m + 15) >> 4;
  const GLOBAL uint64_t* const F = gp(yds[pi].F);
  const double alpha = pr.alpha, beta = pr.beta;
  const int r16 = lane & 15, g = lane >> 4;
  const int rb0 = 2 * (w & 1), cb0 = 2 * (w >> 1);
  for (int tile = wi; tile < ntiles; tile += P) {   // workgroup-uniform
    const int ti = tile % ntr, tj = tile / ntr;
    select_bits(X, m64, kRT * ti, rmap, ws);
    select_bits(X + m64, n64, kRT * tj, cmap, ws);
    const int nr = min(kRT, nR - kRT * ti), nc = min(kRT, nC - kRT * tj);
    const GLOBAL double* const AT = gp(yds[pi].AT) + (size_t)(kRT * ti) * (size_t)K;
    // staging element x = t + kThreads s: slot x / kXK of A (x < kRT kXK) or of B, at k x % kXK
    double v[kXLoads];
    // (inlined: a staging array passed to an outlined lambda by reference would live in scratch)
    auto fetch = [&](int kc) __attribute__((always_inline)) {
#pragma unroll
      for (int s = 0; s < kXLoads; ++s) {
        const int x = t + kThreads * s, slot = (x / kXK) % kRT, kk = x % kXK, k = kc + kk;
        if (x < kRT * kXK)
          v[s] = (slot < nr && k < K) ? AT[(size_t)slot * (size_t)K + (size_t)k] : 0.0;
        else
          v[s] = (slot < nc && k < K) ? B[(size_t)k + (size_t)cmap[slot] * ldb] : -0.0;
      }
    };
    auto put = [&](double* dst) __attribute__((always_inline)) {
#pragma unroll
      for (int s = 0; s < kXLoads; ++s) {
        const int x = t + kThreads * s;
        dst[(x / kXK) * kXS + x % kXK] = v[s];   // B's slots follow A's (x / kXK >= kRT)
      }
    };
    // wave-uniform: the wave's blocks that hold rows of R / columns of C
    const bool rowA = 16 * rb0 < nr, rowB = 16 * (rb0 + 1) < nr;
    const bool colA = 16 * cb0 < nc, colB = 16 * (cb0 + 1) < nc;
    v4d acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = v4d{0.0, 0.0, 0.0, 0.0};
    fetch(0);
    put(xs[0]);
    if (kXK < K) fetch(kXK);
    lds_sync();
    int cur = 0;
    for (int kc = 0; kc < K; kc += kXK) {
      const int steps = (min(kXK, K - kc) + 3) >> 2;   // k-steps of 4 (the last padded)
      if (rowA && colA) {
        const double* const As = xs[cur] + (16 * rb0 + r16) * kXS + g;
        const double* const Bs = xs[cur] + (kRT + 16 * cb0 + r16) * kXS + g;
        double a0 = As[0], a1 = As[16 * kXS], b0 = Bs[0], b1 = Bs[16 * kXS];
        for (int st = 0; st < steps; ++st) {
          const int nx = 4 * min(st + 1, steps - 1);   // the next step's operands (the last reads its own)
          const double na0 = As[nx], na1 = As[16 * kXS + nx], nb0 = Bs[nx], nb1 = Bs[16 * kXS + nx];
          acc[0][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0, b0, acc[0][0], 0, 0, 0);
          if (colB) acc[0][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0, b1, acc[0][1], 0, 0, 0);
          if (rowB) acc[1][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1, b0, acc[1][0], 0, 0, 0);
          if (rowB && colB) acc[1][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1, b1, acc[1][1], 0, 0, 0);
          a0 = na0;
          a1 = na1;
          b0 = nb0;
          b1 = nb1;
        }
      }
      if (kc + kXK < K) {
        put(xs[cur ^ 1]);   // chunk kc + kXK (the other buffer's last readers passed a barrier)
        if (kc + 2 * kXK < K) fetch(kc + 2 * kXK);
      }
      lds_sync();   // chunk kc's steps done, chunk kc + kXK staged
      cur ^= 1;
    }
    // accumulator element e of lane l: block row l / 16 + 4 e, block column l % 16
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int cs = 16 * (cb0 + j) + r16;
        if (cs >= nc) continue;
        const int col = cmap[cs];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int rs = 16 * (rb0 + i) + g + 4 * e;
          if (rs >= nr) continue;
          const int row = rmap[rs];
          const uint64_t wv = F[4 * ((size_t)(col >> 4) * mb + (row >> 4)) + (row & 3)];
          if ((wv >> (16 * ((row & 15) >> 2) + (col & 15))) & 1ull) {
            const double d = e == 0 ? acc[i][j].x : (e == 1 ? acc[i][j].y : (e == 2 ? acc[i][j].z : acc[i][j].w));
            GLOBAL double* cp = gpw(pr.C) + (size_t)row + (size_t)col * pr.ldc;
            *cp = from_dot(alpha, beta, d, beta != 0.0 ? *cp : 0.0);
          }
        }
      }
    lds_sync();   // rmap / cmap and the staging are free for the next tile
  }
}

// Kernel of oz2_mfma_f64_chains: the accumulation the crossings pass relies on, for the tests.
__global__ void __launch_bounds__(64) mfma_chain_kernel(const double* __restrict__ A, const double* __restrict__ B,
                                                        double* __restrict__ D, int steps) {
  const int w = blockIdx.x, l = threadIdx.x;
  v4d acc = v4d{0.0, 0.0, 0.0, 0.0};
  for (int t = 0; t < steps; ++t) {
    const size_t x = ((size_t)w * steps + t) * 64 + l;
    acc = __builtin_amdgcn_mfma_f64_16x16x4f64(A[x], B[x], acc, 0, 0, 0);
  }
  double* d = D + 256 * (size_t)w + 4 * l;
  d[0] = acc.x;
  d[1] = acc.y;
  d[2] = acc.z;
  d[3] = acc.w;
}

}  // namespace

int recon_launch(const oz2_problem* d, const YDesc* yd, int num, int max_m, int max_n, hipStream_t s, int mode,
                 bool blocked, int* launches, const ReconGrid* grid, int dot_form) {
  if (launches) *launches = 0;
  if (num <= 0) return 0;
  if (mode != OZ2_REPAIR_OFF && mode != OZ2_REPAIR_COUNT && mode != OZ2_REPAIR_ON) return 1;
  if (num > 65535 || max_m < 0 || max_n < 0) return 1;
  DevCtx* c = dev_ctx();
  if (!c) return 2;
  const size_t mn = (size_t)max_m * (size_t)max_n;
  if (mn == 0) return 0;
  const bool blk = blocked && yd;
  const bool compact = grid && yd && grid->ne == num;
  const int tm = blk ? kBTileM : kTileM, tn = blk ? kBTileN : kTileN;
  static_assert(kBTileM == kReconTileMB && kBTileN == kReconTileNB && kTileM == kReconTileMC && kTileN == kReconTileNC &&
                    kRT == kDotTile, "reconstruct tile shapes");
  // compact grid: the tiles of all problems; else a row per problem as wide as the largest problem
  // (a problem with fewer tiles returns from the surplus workgroups)
  const size_t gx = compact ? (size_t)grid->tiles : (size_t)((max_m + tm - 1) / tm) * (size_t)((max_n + tn - 1) / tn);
  const size_t gd = compact ? (size_t)grid->dtiles : (size_t)((max_m + kRT - 1) / kRT) * (size_t)((max_n + kRT - 1) / kRT);
  const size_t gb = compact ? (size_t)grid->bands : (size_t)((max_m + kRT - 1) / kRT);
  if (gx > 0x7fffffffu || gd > 0x7fffffffu || gb > 0x7fffffffu) return 1;
  const unsigned gy = compact ? 1u : (unsigned)num;
  const int gne = compact ? num : 0, gper = compact ? grid->per : 0, dper = compact ? grid->dper : 0;
  const int bper = compact ? grid->bper : 0;
  int nl = 0;
  if (gx > 0) {
    if (blk)
      hipLaunchKernelGGL((recon_kernel<true, true>), dim3((unsigned)gx, gy), dim3(kThreads), 0, s, d, yd, mode, c->tab,
                         c->counters, gne, gper);
    else if (yd)
      hipLaunchKernelGGL((recon_kernel<true, false>), dim3((unsigned)gx, gy), dim3(kThreads), 0, s, d, yd, mode,
                         c->tab, c->counters, gne, gper);
    else
      hipLaunchKernelGGL((recon_kernel<false, false>), dim3((unsigned)gx, gy), dim3(kThreads), 0, s, d, nullptr, mode,
                         c->tab, c->counters, 0, 0);
    ++nl;
  }
  if (blk && gd > 0) {
    hipLaunchKernelGGL(dots_kernel, dim3((unsigned)gd, gy), dim3(kThreads), 0, s, d, yd, gne, dper, dot_form);
    ++nl;
  }
  // crossings workgroups: the compact grid's, else 64 per problem
  const size_t gc = compact ? (size_t)grid->xwgs : (size_t)std::min<size_t>(gd, 64);
  if (blk && gb > 0 && gc > 0) {   // the deferred chains: rows gathered, then the crossings
    hipLaunchKernelGGL(gather_kernel, dim3((unsigned)gb, gy), dim3(kThreads), 0, s, d, yd, gne, bper);
    hipLaunchKernelGGL(cross_kernel, dim3((unsigned)gc, gy), dim3(kThreads), 0, s, d, yd, gne, compact ? grid->xper : 0);
    nl += 2;
  }
  if (launches) *launches = nl;
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

}  // namespace ggemm

extern "C" int oz2_mfma_f64_chains(const double* A, const double* B, double* D, int waves, int steps, hipStream_t s) {
  if (waves < 1 || steps < 1) return 1;
  hipLaunchKernelGGL(ggemm::mfma_chain_kernel, dim3((unsigned)waves), dim3(64), 0, s, A, B, D, steps);
  if (hipGetLastError() != hipSuccess || hipStreamSynchronize(s) != hipSuccess) return 3;
  return 0;
}

extern "C" int oz2_reconstruct_grouped(const oz2_problem* d, int num, int max_m, int max_n, hipStream_t s,
                                       int repair_mode) {
  return ggemm::recon_launch(d, nullptr, num, max_m, max_n, s, repair_mode);
}
