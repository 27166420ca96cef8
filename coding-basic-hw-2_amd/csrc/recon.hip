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
// y_l, hence the same output bits.  A thread handles 4 consecutive entries of the column-major
// m x n index space: one 32-bit load per digit plane, one 128-bit load of L, all issued before
// the arithmetic.
// Two multiply-adds of the reference that its device compiler fuses are written as fma() here
// (s2d - Q P2 and |alpha| Lab + |beta C0|); every other operation is unfused (fp contract off),
// so the result is the reference's to the last bit.
#include <cmath>

#include "common.hpp"

#pragma clang fp contract(off)

namespace ggemm {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ double pow2d(int e) { return __longlong_as_double((long long)(e + 1023) << 52); }
__device__ __forceinline__ double mul_pow2(double x, int e) {
  if (e >= -1000 && e <= 1000) return x * pow2d(e);
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    const int ee = max(-1000, min(1000, e));
    x *= pow2d(ee);
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
  const double* __restrict__ a = pr.A + i;
  const double* __restrict__ b = pr.B + (size_t)j * pr.ldb;
  const size_t lda = (size_t)pr.lda;
  double s = 0.0;
  for (int k = 0; k < pr.k; ++k) s = fma(a[(size_t)k * lda], b[k], s);
  return s;
}

struct Shared {
  uint32_t p[kMaxModuli], mg[kMaxModuli], q[kMaxModuli], s2[kMaxModuli];
  uint64_t s1[kMaxModuli];
  unsigned long long cnt[3][kThreads / 64];
};

template <bool kDigits>
__global__ void __launch_bounds__(kThreads) recon_kernel(const oz2_problem* __restrict__ probs,
                                                         const YDesc* __restrict__ yds, int mode,
                                                         const CrtTables* __restrict__ tab,
                                                         unsigned long long* __restrict__ cnt) {
  __shared__ Shared sh;
  const oz2_problem& pr = probs[blockIdx.y];
  const int N = pr.num_moduli;
  if (N < 1 || N > kMaxModuli) return;
  const int m = pr.m, n = pr.n, K = pr.k;
  const size_t total = (size_t)m * (size_t)n;
  if (total == 0) return;
  if (threadIdx.x < (unsigned)N) {
    const int l = threadIdx.x;
    sh.p[l] = (uint32_t)tab->p[l];
    sh.mg[l] = tab->magic[l];
    sh.q[l] = (uint32_t)tab->qinv[N][l];
    sh.s1[l] = tab->s1[N][l];
    sh.s2[l] = tab->s2[N][l];
  }
  __syncthreads();
  const double alpha = pr.alpha, beta = pr.beta, aalpha = fabs(alpha);
  const int64_t P1 = tab->P1[N];
  const double P2 = tab->P2[N], invPu = tab->inv_Pu[N];
  const int lu1 = tab->log2_u1[N];
  const double inv_u1 = ldexp(1.0, -lu1);
  const double crt_u = N * 255.0 * 0x1p-19 + 0x1p-10;
  const double u = 0x1p-53;
  const double nt = (double)K + (alpha != 1.0 ? 1.0 : 0.0) + (beta != 0.0 ? 1.0 : 0.0);
  const double gam = (nt * u / (1.0 - nt * u) - 2.0 * u) * (1.0 - 0x1p-40);
  const int32_t* __restrict__ rs = pr.row_shift;
  const int32_t* __restrict__ cs = pr.col_shift;
  const int32_t* __restrict__ C32 = pr.C32;
  const size_t cst = pr.c32_mod_stride;
  YDesc yd{nullptr, 0, nullptr};
  if (kDigits) yd = yds[blockIdx.y];
  unsigned n_uncert = 0, n_repair = 0, n_safety = 0;

  // quads of entries: qd covers linear indices 4 qd .. 4 qd + 3 (column-major, ld m);
  // (i, j) of the first entry advances by G = 4 * stride = di m + dr with one carry
  const size_t nq = (total + 3) / 4;
  const size_t stride = (size_t)gridDim.x * kThreads;
  const size_t q0 = (size_t)blockIdx.x * kThreads + threadIdx.x;
  const size_t G4 = 4 * stride;
  const int di = (int)(G4 / (size_t)m), dr = (int)(G4 % (size_t)m);
  int i0 = (int)((4 * q0) % (size_t)m);
  int j0 = (int)((4 * q0) / (size_t)m);
  for (size_t qd = q0; qd < nq; qd += stride) {
    const size_t idx0 = 4 * qd;
    const bool full = idx0 + 4 <= total;
    uint32_t yv[kMaxModuli];
    int32_t Lv[4] = {0, 0, 0, 0};
    if (alpha != 0.0) {
      if (kDigits) {
#pragma unroll
        for (int l = 0; l < kMaxModuli; ++l) {
          if (l < N) {
            const uint8_t* y = yd.Y + (size_t)l * yd.y_stride + idx0;
            if (full) {
              yv[l] = *reinterpret_cast<const uint32_t*>(y);
            } else {
              uint32_t v = 0;
              for (int e = 0; e < 4; ++e)
                if (idx0 + e < total) v |= (uint32_t)y[e] << (8 * e);
              yv[l] = v;
            }
          }
        }
        if (full) {
          const int4 L4 = *reinterpret_cast<const int4*>(yd.L + idx0);
          Lv[0] = L4.x; Lv[1] = L4.y; Lv[2] = L4.z; Lv[3] = L4.w;
        } else {
          for (int e = 0; e < 4; ++e)
            if (idx0 + e < total) Lv[e] = yd.L[idx0 + e];
        }
      } else {
#pragma unroll
        for (int l = 0; l < kMaxModuli; ++l) {
          if (l < N) {
            const uint32_t p = sh.p[l], mg = sh.mg[l], qi = sh.q[l];
            uint32_t v = 0;
            for (int e = 0; e < 4; ++e) {
              if (idx0 + e >= total) break;
              const int32_t c = C32[l * cst + idx0 + e];
              const uint32_t uc = c < 0 ? 0u - (uint32_t)c : (uint32_t)c;
              uint32_t r = mod_small(uc, p, mg);
              if (c < 0 && r) r = p - r;
              v |= mod_small(r * qi, p, mg) << (8 * e);
            }
            yv[l] = v;
          }
        }
        for (int e = 0; e < 4; ++e)
          if (idx0 + e < total) Lv[e] = C32[N * cst + idx0 + e];
      }
    }
    // coordinates, C0 and the row / column shifts of the 4 entries, loaded before any arithmetic
    int ie[4], je[4], rsv[4], csv[4], sgv[4], tav[4];
    float dav[4], nav[4], dbv[4], nbv[4];
    double c0v[4];
    {
      int i = i0, j = j0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ie[e] = i;
        je[e] = j;
        if (++i == m) { i = 0; ++j; }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool in = idx0 + e < total;
        c0v[e] = (in && beta != 0.0) ? pr.C[ie[e] + (size_t)je[e] * pr.ldc] : 0.0;
        const bool ld = in && alpha != 0.0;
        rsv[e] = ld ? rs[ie[e]] : 0;
        csv[e] = ld ? cs[je[e]] : 0;
        sgv[e] = ld ? rs[m + ie[e]] : 0;
        tav[e] = ld ? cs[n + je[e]] : 0;
        const bool lc = ld && mode != OZ2_REPAIR_OFF;
        dav[e] = lc ? __int_as_float(rs[2 * m + ie[e]]) : 0.f;
        nav[e] = lc ? __int_as_float(rs[3 * m + ie[e]]) : 0.f;
        dbv[e] = lc ? __int_as_float(cs[2 * n + je[e]]) : 0.f;
        nbv[e] = lc ? __int_as_float(cs[3 * n + je[e]]) : 0.f;
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (idx0 + e >= total) break;
      const int i = ie[e], j = je[e];
      double* cp = pr.C + i + (size_t)j * pr.ldc;
      const double c0 = c0v[e];
      double out;
      if (alpha == 0.0) {   // BLAS: A, B and the workspace are not referenced
        out = (beta == 0.0) ? 0.0 : beta * c0;
      } else {
        const int rsh = rsv[e], csh = csv[e];
        if (rsh == OZ2_SHIFT_NONFINITE || csh == OZ2_SHIFT_NONFINITE) {   // safety fallback
          const double d = fp64_dot(pr, i, j);
          out = (beta == 0.0) ? alpha * d : fma(alpha, d, beta * c0);
          ++n_safety;
        } else {
          const int sig = sgv[e], tau = tav[e];
          if (sig == OZ2_SHIFT_ZERO || tau == OZ2_SHIFT_ZERO) {   // zero row / column: AB_ij = 0
            out = (beta == 0.0) ? alpha * 0.0 : fma(alpha, 0.0, beta * c0);
          } else {
            uint64_t S1 = 0;
            uint32_t S2 = 0;
#pragma unroll
            for (int l = 0; l < kMaxModuli; ++l) {
              if (l < N) {
                const uint32_t y = (yv[l] >> (8 * e)) & 0xffu;
                S1 += sh.s1[l] * (uint64_t)y;
                S2 += sh.s2[l] * y;
              }
            }
            const double s2d = (double)S2 * 0x1p-18;
            const double Q = rint(((double)S1 + s2d) * invPu);
            const int64_t X1 = (int64_t)S1 - (int64_t)Q * P1;
            const double xr = (double)X1 + fma(-Q, P2, s2d);
            const int esc = lu1 - rsh - csh;
            const double v = mul_pow2(xr, esc);
            const double emu = (beta == 0.0) ? alpha * v : fma(alpha, v, beta * c0);
            if (mode == OZ2_REPAIR_OFF || (beta != 0.0 && !isfinite(c0))) {
              out = emu;
            } else {
              const double da = dav[e], na = nav[e];
              const double db = dbv[e], nb = nbv[e];
              const double et = fma(da, nb, fma(na, db, da * db)) * (1.0 + 0x1p-40);
              const double Eu = (fma(et, inv_u1, crt_u) + 4.0 * u * fabs(xr)) * (1.0 + 0x1p-40);
              const double E = mul_pow2(Eu, esc);
              double lab = mul_pow2((double)Lv[e], -(sig + tau));
              lab = fmax(lab, fabs(v) - E) * (1.0 - 0x1p-40);
              if (lab < 0x1p-1000) lab = 0.0;
              const double lhs = aalpha * E * (1.0 + 0x1p-40);
              const double rhs = gam * fma(aalpha, lab, fabs(beta * c0)) * (1.0 - 0x1p-40);
              const bool cert = gam > 0.0 && E >= 0x1p-1000 && isfinite(lhs) && isfinite(v) && lhs <= rhs;
              if (cert) {
                out = emu;
              } else if (mode == OZ2_REPAIR_COUNT) {
                out = emu;
                ++n_uncert;
              } else {
                const double d = fp64_dot(pr, i, j);
                out = (beta == 0.0) ? alpha * d : fma(alpha, d, beta * c0);
                ++n_repair;
              }
            }
          }
        }
      }
      *cp = out;
    }
    i0 += dr;
    j0 += di;
    if (i0 >= m) { i0 -= m; ++j0; }
  }
  // counters: wave reduce, block reduce, one atomic per counter per block (exact integer sums)
  unsigned long long cu = n_uncert, cr = n_repair, cf = n_safety;
#pragma unroll
  for (int o = 32; o; o >>= 1) {
    cu += __shfl_down(cu, o);
    cr += __shfl_down(cr, o);
    cf += __shfl_down(cf, o);
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) { sh.cnt[0][wid] = cu; sh.cnt[1][wid] = cr; sh.cnt[2][wid] = cf; }
  __syncthreads();
  if (threadIdx.x < 3) {
    unsigned long long t = 0;
    for (int w = 0; w < kThreads / 64; ++w) t += sh.cnt[threadIdx.x][w];
    if (t) atomicAdd(&cnt[1 + threadIdx.x], t);
  }
}

}  // namespace

int recon_launch(const oz2_problem* d, const YDesc* yd, int num, int max_m, int max_n, hipStream_t s, int mode) {
  if (num <= 0) return 0;
  if (mode != OZ2_REPAIR_OFF && mode != OZ2_REPAIR_COUNT && mode != OZ2_REPAIR_ON) return 1;
  if (num > 65535 || max_m < 0 || max_n < 0) return 1;
  DevCtx* c = dev_ctx();
  if (!c) return 2;
  const size_t mn = (size_t)max_m * (size_t)max_n;
  if (mn == 0) return 0;
  size_t gx = (mn / 4 + kThreads - 1) / kThreads + 1;
  if (gx > 1024) gx = 1024;
  if (yd)
    hipLaunchKernelGGL(recon_kernel<true>, dim3((unsigned)gx, num), dim3(kThreads), 0, s, d, yd, mode, c->tab,
                       c->counters);
  else
    hipLaunchKernelGGL(recon_kernel<false>, dim3((unsigned)gx, num), dim3(kThreads), 0, s, d, nullptr, mode, c->tab,
                       c->counters);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

}  // namespace ggemm

extern "C" int oz2_reconstruct_grouped(const oz2_problem* d, int num, int max_m, int max_n, hipStream_t s,
                                       int repair_mode) {
  return ggemm::recon_launch(d, nullptr, num, max_m, max_n, s, repair_mode);
}
