// prep.hip -- Ozaki-II residue preparation for a whole group (one launch).
//
// Per problem (alpha != 0, N moduli):
//   s_i   = largest s with 2^s ||A(i,:)||_2 (1+2^-30)^(1/2) <= T_N   (t_j likewise for B(:,j))
//   A'    = trunc(2^s A)                      (toward zero, so ||A'_i|| <= T_N)
//   plane l < N : sym(A' mod p_l) in [-(p-1)/2, (p-1)/2]   (p = 256: [-128, 127])
//   plane N     : floor(2^sigma |A|) in [0, 127], sigma = 6 - ilogb(max_k |A_ik|)
//   workspace   : {s, sigma, ||2^s A - A'|| float-rounded-up, ||A'|| float-rounded-up}
// following src/ozaki2_numerics.cu:112-231 (element arithmetic) and :242-442 (kernel).
// Rows / columns with NaN/Inf get s = OZ2_SHIFT_NONFINITE (zero residues); all-zero ones get
// sigma = OZ2_SHIFT_ZERO.
//
// Bit-exactness of s, sigma and the two norm bounds requires the reference's summation order:
//   A rows   : 8 chains, chain c = k (mod 8) accumulated in ascending k with fma, then the chain
//              sums added c = 0..7 (src/ozaki2_numerics.cu:274-305, :356-363);
//   B columns: 32 chains k = L (mod 32) for the norm; for the residue-pass sums lane L owns
//              k = 4L + 128c + e (c ascending, e = 0..3); lane values combined by the XOR
//              butterfly o = 16, 8, 4, 2, 1 (src/ozaki2_numerics.cu:373-440).
// Everything else (residues, abs plane) is elementwise and mapped freely for the hardware:
//   * A (column-major in HBM, row-major residues out): a block owns 32 rows.  The chain threads
//     load a 32 x 128 k-tile with 256-byte coalesced reads, keep the ordered chain sums, and
//     park the doubles in LDS k-major; then every thread takes 16 consecutive k of one row,
//     computes the residues and writes each plane with one 128-bit store.
//   * B (column-major = K contiguous): 32 lanes per column, 4 consecutive k per lane: 1 KB
//     coalesced loads, 128 contiguous residue bytes per plane per store.
// Floating-point contraction is off in this file: the only fused operations are the explicit
// fma() calls, which are the reference's own.
#include <cmath>

#include "common.hpp"

#pragma clang fp contract(off)

namespace ggemm {
namespace {

constexpr int kThreads = 256;
constexpr int kARows = 32;      // rows of A per block
constexpr int kATile = 128;     // k tile of the A residue pass
constexpr int kBCols = 8;       // columns of B per block (32 lanes each)
constexpr int kChains = 8;      // A-row reduction chains

__device__ __forceinline__ double pow2d(int e) {   // 2^e, e in [-1022, 1023]
  return __longlong_as_double((long long)(e + 1023) << 52);
}
// x * 2^e: one exact multiply for |e| <= 1000, else three clamped steps.
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

// Largest s with 2^s * nrm <= T, nrm = f 2^(g + add) (frexp), T = F 2^G.
__device__ __forceinline__ int choose_shift(double nrm, int add, double T) {
  int g, G;
  const double f = frexp(nrm, &g);
  const double F = frexp(T, &G);
  return G - (g + add) - (f > F ? 1 : 0);
}
__device__ __forceinline__ int shift_from_norm(double maxabs, double ssq, bool rescaled, double T) {
  if (isinf(maxabs) || isnan(ssq)) return OZ2_SHIFT_NONFINITE;
  if (!(maxabs > 0.0)) return 0;
  const double nm = sqrt(ssq * (1.0 + 0x1p-30));
  return choose_shift(nm, rescaled ? ilogb(maxabs) : 0, T);
}
__device__ __forceinline__ int abs_shift(double maxabs, int sh) {
  if (sh == OZ2_SHIFT_NONFINITE) return 0;
  if (!(maxabs > 0.0)) return OZ2_SHIFT_ZERO;
  return 6 - ilogb(maxabs);
}
__device__ __forceinline__ bool needs_rescale(double maxabs) {
  return maxabs > 0.0 && (maxabs > 0x1p400 || maxabs < 0x1p-400);
}
// Float round-up of sqrt(x (1 + 2^-30)), returned as the float's bit pattern (x >= 0 finite).
__device__ __forceinline__ int32_t norm_ub_bits(double x) {
  const double s = sqrt(x * (1.0 + 0x1p-30));
  float f = (float)s;
  int32_t b = __float_as_int(f);
  if ((double)f < s) ++b;   // next float up (f >= 0)
  return b;
}

// Residues of an integer-valued double x (|x| < 2^81): x = sign M 2^E with M < 2^53 split in
// 18-bit chunks; x mod p = sign (c0 [2^E] + c1 [2^(E+18)] + c2 [2^(E+36)]) mod p.
struct Split {
  uint32_t c0, c1, c2;
  int E;
  bool neg;
};
__device__ __forceinline__ Split split_int(double x) {
  Split d;
  const double ax = fabs(x);
  d.neg = x < 0.0;
  uint64_t M;
  int E;
  if (ax < 9007199254740992.0) {
    M = (uint64_t)ax;
    E = 0;
  } else {
    const uint64_t b = (uint64_t)__double_as_longlong(ax);
    E = min((int)((b >> 52) & 0x7ff) - 1075, kPow2Table - 37);
    M = (b & ((1ull << 52) - 1)) | (1ull << 52);
  }
  d.c0 = (uint32_t)(M & 0x3ffff);
  d.c1 = (uint32_t)((M >> 18) & 0x3ffff);
  d.c2 = (uint32_t)(M >> 36);
  d.E = E;
  return d;
}
// Symmetric residues sym(x mod p) in [-h, p - 1 - h] (h = floor(p / 2)) of integers
// x = c0 2^E + c1 2^(E+18) + c2 2^(E+36) given as signed 18-bit chunks (the sign of x on each):
//   u = c0 w0 + c1 w1 + c2 w2 + K p,  w_i = 2^(E + 18 i) mod p (times q for folded planes)
//       (24-bit multiply-adds; |c_i w_i| < 2^26, K p >= 2^28, so 0 < u < 2^30)
//   q = trunc(fma(u, ip, hip)) = floor((u + h) / p)
//       exact: ip = 1/p and hip = h ip are rounded up, so the fma's exact value is >= (u + h)/p,
//       and it exceeds it by less than 2^-21 / p while (u + h)/p <= floor + 1 - 1/p
//   r = fma(-q, p, u)                 (exact: an integer in [-h, p - 1 - h])
// The byte equals the reference's reduce / negate / symmetric-map sequence; every operation is
// full rate (24-bit integer and FP64 arithmetic, no 32-bit integer multiply).  When no lane of the
// wave has E > 0 the weights are per-plane constants (scalar registers), otherwise per-element
// LDS table lookups.
struct PlaneC {
  int Kp, w0, w1, w2;
  double p, ip, hip;
};
__device__ __forceinline__ PlaneC plane_c(const CrtTables* __restrict__ tab, int l, int widx) {
  return PlaneC{tab->Kp[l], tab->w3[widx][l][0], tab->w3[widx][l][1], tab->w3[widx][l][2],
                (double)tab->p[l], tab->inv_p_up[l], tab->h_ip_up[l]};
}
template <int NE>
__device__ __forceinline__ void residue_bytes(const int* c0, const int* c1, const int* c2, const int* E, bool anyE,
                                              const PlaneC& k, const uint8_t* pw, uint32_t* out) {
  int u[NE];
  if (!anyE) {
#pragma unroll
    for (int e = 0; e < NE; ++e) u[e] = __mul24(c0[e], k.w0) + __mul24(c1[e], k.w1) + __mul24(c2[e], k.w2) + k.Kp;
  } else {
#pragma unroll
    for (int e = 0; e < NE; ++e)
      u[e] = __mul24(c0[e], (int)pw[E[e]]) + __mul24(c1[e], (int)pw[E[e] + 18]) + __mul24(c2[e], (int)pw[E[e] + 36]) + k.Kp;
  }
#pragma unroll
  for (int w = 0; w < NE / 4; ++w) {
    uint32_t v = 0u;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const double ud = (double)u[4 * w + e];
      const double q = trunc(fma(ud, k.ip, k.hip));
      const int r = (int)fma(-q, k.p, ud);
      v |= ((uint32_t)r & 0xffu) << (8 * e);
    }
    out[w] = v;
  }
}
// signed chunks of an integer-valued double (|x| < 2^81)
__device__ __forceinline__ void chunks(double x, int& c0, int& c1, int& c2, int& E) {
  const Split d = split_int(x);
  c0 = d.neg ? -(int)d.c0 : (int)d.c0;
  c1 = d.neg ? -(int)d.c1 : (int)d.c1;
  c2 = d.neg ? -(int)d.c2 : (int)d.c2;
  E = d.E;
}
__device__ __forceinline__ uint32_t abs_u8(double a, int sig) {
  if (sig == OZ2_SHIFT_ZERO) return 0;
  return (uint32_t)(int)fmin(127.0, trunc(mul_pow2(fabs(a), sig)));
}

struct PrepShared {
  uint8_t pow2[kMaxModuli][kPow2Table];
  double red0[kChains][kARows];
  double red1[kChains][kARows];
  int shift[kARows], sig[kARows];
  double rowmax[kARows];
  double tile[kATile][kARows];      // A values of the current k-tile, k-major
};

// ------------------------------------------------------------------------------- A rows
__device__ void prep_rows(const oz2_problem& pr, const CrtTables* __restrict__ tab, int blk, int split,
                          int nsplit, PrepShared& sm, unsigned long long* cnt, int widx, bool packed) {
  const int tid = threadIdx.x;
  const int N = pr.num_moduli, K = pr.k, Kp = pr.kp, m = pr.m;
  const int row0 = blk * kARows;
  const int r = tid & 31, c = tid >> 5;          // chain role: row r, chain c
  const int i = row0 + r;
  const bool valid = i < m;
  const double* __restrict__ A = pr.A;
  const size_t lda = (size_t)pr.lda;
  const double T = tab->T[N];

  // ---- pass 1: row max and sum of squares, chain c = k mod 8 ascending
  double mx = 0.0, ss = 0.0;
  if (valid) {
    int k = c;
    for (; k + 8 * 15 < K; k += 8 * 16) {   // 16 loads in flight, then the ordered chain
      double a[16];
#pragma unroll
      for (int t = 0; t < 16; ++t) a[t] = A[i + (size_t)(k + 8 * t) * lda];
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        mx = fmax(mx, fabs(a[t]));
        ss = fma(a[t], a[t], ss);
      }
    }
    for (; k < K; k += 8) {
      const double a = A[i + (size_t)k * lda];
      mx = fmax(mx, fabs(a));
      ss = fma(a, a, ss);
    }
  }
  sm.red0[c][r] = mx;
  __syncthreads();
  if (c == 0) {
    double M = 0.0;
    for (int q = 0; q < kChains; ++q) M = fmax(M, sm.red0[q][r]);
    sm.rowmax[r] = M;
  }
  __syncthreads();
  const double rowmax = sm.rowmax[r];
  const bool resc = valid && needs_rescale(rowmax);
  if (resc) {   // rare: exact power-of-two prescaling so the squares cannot overflow / underflow
    const int e = -ilogb(rowmax);
    ss = 0.0;
    for (int k = c; k < K; k += kChains) {
      const double a = mul_pow2(A[i + (size_t)k * lda], e);
      ss = fma(a, a, ss);
    }
  }
  sm.red1[c][r] = ss;
  __syncthreads();
  if (c == 0) {
    double S = 0.0;
    for (int q = 0; q < kChains; ++q) S += sm.red1[q][r];
    const int sh = valid ? shift_from_norm(rowmax, S, resc, T) : 0;
    const int sg = valid ? abs_shift(rowmax, sh) : OZ2_SHIFT_ZERO;
    sm.shift[r] = sh;
    sm.sig[r] = sg;
    if (valid && split == 0) {
      pr.row_shift[i] = sh;
      pr.row_shift[m + i] = sg;
      if (sh == OZ2_SHIFT_NONFINITE) atomicAdd(&cnt[0], 1ull);
    }
  }
  __syncthreads();

  // ---- pass 2: residues of this split's k-tiles; split 0 also walks every tile for the
  //      ordered ||dA||, ||A'|| chain sums (the residue values do not depend on the split)
  const int sh_c = sm.shift[r];
  const bool nf_c = sh_c == OZ2_SHIFT_NONFINITE;
  const int rr = tid & 31, seg = tid >> 5;   // residue role: row rr, k = 16 seg .. 16 seg + 15
  const int sh_r = sm.shift[rr], sg_r = sm.sig[rr];
  const bool nf_r = sh_r == OZ2_SHIFT_NONFINITE;
  const bool rvalid = row0 + rr < m;
  double da2 = 0.0, na2 = 0.0;
  const int ntile = (Kp + kATile - 1) / kATile;
  const int per = (ntile + nsplit - 1) / nsplit;
  const int w0 = min(ntile, split * per), w1 = min(ntile, w0 + per);   // tiles written here
  const int l0 = split == 0 ? 0 : w0, l1 = split == 0 ? ntile : w1;   // tiles walked here
  for (int t = l0; t < l1; ++t) {
    const int k0 = t * kATile;
    double av[kATile / kChains];
#pragma unroll
    for (int jj = 0; jj < kATile / kChains; ++jj) {
      const int k = k0 + c + kChains * jj;
      av[jj] = (valid && k < K) ? A[i + (size_t)k * lda] : 0.0;
    }
#pragma unroll
    for (int jj = 0; jj < kATile / kChains; ++jj) {
      const int kk = c + kChains * jj;
      const double a = av[jj];
      if (!nf_c && split == 0) {
        const double xs = mul_pow2(a, sh_c);
        const double xt = trunc(xs);
        const double fr = xs - xt;
        da2 = fma(fr, fr, da2);
        na2 = fma(xt, xt, na2);
      }
      sm.tile[kk][r] = a;
    }
    __syncthreads();
    const int kb = k0 + 16 * seg;
    if (t >= w0 && t < w1 && rvalid && kb < Kp) {
      int8_t* dst = pr.A8 + (packed ? packed_offset(row0 + rr, kb, m, Kp) : (size_t)(row0 + rr) * Kp + kb);
      if (nf_r) {
        for (int l = 0; l <= N; ++l)
          *reinterpret_cast<uint4*>(dst + (size_t)l * pr.a8_mod_stride) = make_uint4(0u, 0u, 0u, 0u);
      } else {
        int c0[16], c1[16], c2[16], E[16];
        int anyE = 0;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          chunks(trunc(mul_pow2(sm.tile[16 * seg + e][rr], sh_r)), c0[e], c1[e], c2[e], E[e]);
          anyE |= E[e];
        }
        const bool wE = __any(anyE != 0);
        for (int l = 0; l < N; ++l) {
          const PlaneC pc = plane_c(tab, l, widx);
          uint32_t q[4];
          residue_bytes<16>(c0, c1, c2, E, wE, pc, sm.pow2[l], q);
          *reinterpret_cast<uint4*>(dst + (size_t)l * pr.a8_mod_stride) = make_uint4(q[0], q[1], q[2], q[3]);
        }
        uint32_t q[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          q[w] = 0u;
#pragma unroll
          for (int e = 0; e < 4; ++e) q[w] |= abs_u8(sm.tile[16 * seg + 4 * w + e][rr], sg_r) << (8 * e);
        }
        *reinterpret_cast<uint4*>(dst + (size_t)N * pr.a8_mod_stride) = make_uint4(q[0], q[1], q[2], q[3]);
      }
    }
    __syncthreads();
  }
  if (split != 0) return;   // block-uniform
  sm.red0[c][r] = da2;
  sm.red1[c][r] = na2;
  __syncthreads();
  if (c == 0 && valid) {
    double D = 0.0, Nn = 0.0;
    for (int q = 0; q < kChains; ++q) { D += sm.red0[q][r]; Nn += sm.red1[q][r]; }
    pr.row_shift[2 * m + i] = norm_ub_bits(D);
    pr.row_shift[3 * m + i] = norm_ub_bits(Nn);
  }
}

// ---------------------------------------------------------------------------- B columns
__device__ void prep_cols(const oz2_problem& pr, const CrtTables* __restrict__ tab, int blk, int split,
                          int nsplit, PrepShared& sm, unsigned long long* cnt, bool packed) {
  const int lane = threadIdx.x & 31, w = threadIdx.x >> 5;
  const int j = blk * kBCols + w;
  const int n = pr.n, N = pr.num_moduli, K = pr.k, Kp = pr.kp;
  if (j >= n) return;   // no barriers below; the 32-lane group is column-uniform
  const double* __restrict__ b = pr.B + (size_t)j * pr.ldb;
  const double T = tab->T[N];

  double mx = 0.0, ss = 0.0;
  int k = lane;
  for (; k + 32 * 7 < K; k += 32 * 8) {   // 8 loads in flight, then the ordered chain
    double a[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) a[t] = b[k + 32 * t];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      mx = fmax(mx, fabs(a[t]));
      ss = fma(a[t], a[t], ss);
    }
  }
  for (; k < K; k += 32) {
    const double a = b[k];
    mx = fmax(mx, fabs(a));
    ss = fma(a, a, ss);
  }
#pragma unroll
  for (int o = 16; o; o >>= 1) mx = fmax(mx, __shfl_xor(mx, o, 32));
  const bool resc = needs_rescale(mx);
  if (resc) {
    const int e = -ilogb(mx);
    ss = 0.0;
    for (int k = lane; k < K; k += 32) {
      const double a = mul_pow2(b[k], e);
      ss = fma(a, a, ss);
    }
  }
#pragma unroll
  for (int o = 16; o; o >>= 1) ss += __shfl_xor(ss, o, 32);
  const int sh = shift_from_norm(mx, ss, resc, T);
  const int sg = abs_shift(mx, sh);
  if (lane == 0 && split == 0) {
    pr.col_shift[j] = sh;
    pr.col_shift[n + j] = sg;
    if (sh == OZ2_SHIFT_NONFINITE) atomicAdd(&cnt[0], 1ull);
  }
  const bool nf = sh == OZ2_SHIFT_NONFINITE;

  double da2 = 0.0, na2 = 0.0;
  int8_t* const B8 = pr.B8;
  const int nchunk = (Kp + 127) / 128;
  const int per = (nchunk + nsplit - 1) / nsplit;
  const int c0 = min(nchunk, split * per), c1 = min(nchunk, c0 + per);
  // split 0 walks every chunk (ordered sums) but writes residues only for its own range; lane L
  // owns k = 128 ch + 4 L + e
  for (int ch = (split == 0 ? 0 : c0); ch < (split == 0 ? nchunk : c1); ++ch) {
    const int k0 = 128 * ch + 4 * lane;
    if (k0 >= Kp) continue;
    int8_t* const base = B8 + (packed ? packed_offset(j, k0, n, Kp) : (size_t)j * Kp + k0);
    double a[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] = (k0 + e < K) ? b[k0 + e] : 0.0;
    const bool write = ch >= c0 && ch < c1;
    if (nf) {
      if (write)
        for (int l = 0; l <= N; ++l) *reinterpret_cast<uint32_t*>(base + (size_t)l * pr.b8_mod_stride) = 0u;
      continue;
    }
    int q0[4], q1[4], q2[4], E[4];
    int anyE = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const double xs = mul_pow2(a[e], sh);
      const double xt = trunc(xs);
      const double fr = xs - xt;
      if (split == 0) {
        da2 = fma(fr, fr, da2);
        na2 = fma(xt, xt, na2);
      }
      chunks(xt, q0[e], q1[e], q2[e], E[e]);
      anyE |= E[e];
    }
    if (!write) continue;
    const bool wE = __any(anyE != 0);
    for (int l = 0; l < N; ++l) {
      uint32_t q;
      residue_bytes<4>(q0, q1, q2, E, wE, plane_c(tab, l, 0), sm.pow2[l], &q);
      *reinterpret_cast<uint32_t*>(base + (size_t)l * pr.b8_mod_stride) = q;
    }
    uint32_t q = 0u;
#pragma unroll
    for (int e = 0; e < 4; ++e) q |= abs_u8(a[e], sg) << (8 * e);
    *reinterpret_cast<uint32_t*>(base + (size_t)N * pr.b8_mod_stride) = q;
  }
  if (split != 0) return;
#pragma unroll
  for (int o = 16; o; o >>= 1) {
    da2 += __shfl_xor(da2, o, 32);
    na2 += __shfl_xor(na2, o, 32);
  }
  if (lane == 0) {
    pr.col_shift[2 * n + j] = norm_ub_bits(da2);
    pr.col_shift[3 * n + j] = norm_ub_bits(na2);
  }
}

__global__ void __launch_bounds__(kThreads) prep_kernel(const oz2_problem* __restrict__ probs, int a_blocks,
                                                        const CrtTables* __restrict__ tab,
                                                        unsigned long long* __restrict__ cnt, int fold_q,
                                                        int packed) {
  __shared__ PrepShared sm;
  const oz2_problem& pr = probs[blockIdx.y];
  const int N = pr.num_moduli;
  if (N < 1 || N > kMaxModuli || pr.alpha == 0.0) return;   // alpha == 0: A, B never referenced
  const bool fold = fold_q && (int)blockIdx.x < a_blocks;
  // 2^e mod p; for folded A residues (q 2^e) mod p, so that sum c_i [q 2^(E_i)] = q x (mod p)
  for (int q = threadIdx.x; q < kMaxModuli * kPow2Table; q += kThreads) {
    const int l = q / kPow2Table;
    uint32_t v = tab->pow2[l][q % kPow2Table];
    if (fold && l < N) v = (v * (uint32_t)tab->qinv[N][l]) % (uint32_t)tab->p[l];
    (&sm.pow2[0][0])[q] = (uint8_t)v;
  }
  __syncthreads();
  const int blk = (int)blockIdx.x;
  if (blk < a_blocks) {
    if (blk * kARows >= pr.m) return;
    prep_rows(pr, tab, blk, blockIdx.z, gridDim.z, sm, cnt, fold ? N : 0, packed != 0);
  } else {
    prep_cols(pr, tab, blk - a_blocks, blockIdx.z, gridDim.z, sm, cnt, packed != 0);
  }
}

int g_force_split = 0;

}  // namespace

int prep_launch(const oz2_problem* d, int num, int max_m, int max_n, hipStream_t s, int fold_q, int packed) {
  if (num <= 0) return 0;
  if (num > 65535 || max_m < 0 || max_n < 0) return 1;
  DevCtx* c = dev_ctx();
  if (!c) return 2;
  const int a_blocks = (max_m + kARows - 1) / kARows;
  const int b_blocks = (max_n + kBCols - 1) / kBCols;
  if (a_blocks + b_blocks == 0) return 0;
  const long long blocks = (long long)(a_blocks + b_blocks) * num;
  const long long target = 4LL * c->num_cus;
  int S = (int)std::min<long long>(16, std::max<long long>(1, (target + blocks - 1) / blocks));
  if (g_force_split > 0) S = g_force_split;
  hipLaunchKernelGGL(prep_kernel, dim3(a_blocks + b_blocks, num, S), dim3(kThreads), 0, s, d, a_blocks,
                     c->tab, c->counters, fold_q, packed);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

}  // namespace ggemm

extern "C" int oz2_prep_grouped(const oz2_problem* d, int num, int max_m, int max_n, hipStream_t s) {
  return ggemm::prep_launch(d, num, max_m, max_n, s, 0);
}

extern "C" void oz2_debug_force_prep_split(int S) { ggemm::g_force_split = (S >= 1 && S <= 64) ? S : 0; }
