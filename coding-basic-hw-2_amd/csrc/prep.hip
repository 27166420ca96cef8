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
//     coalesced loads, 128 contiguous residue bytes per plane per store.  With two-word digits and
//     k <= 1024 a column is read once: lane l keeps k = l (mod 32) in registers (its norm chain)
//     and receives each chunk's 4 consecutive k through a 1 KB LDS exchange row of its column.
//     The kernel is bounded to 128 VGPRs (four workgroups per compute unit).
// Floating-point contraction is off in this file: the only fused operations are the explicit
// fma() calls, which are the reference's own.
#include <cmath>

#include "common.hpp"

// global address space for every HBM access: the descriptor pointers would otherwise compile to
// flat accesses, which also count in lgkmcnt, so the LDS waits of the reductions and of the
// exchange row would wait for the HBM loads in flight as well
#define GLOBAL __attribute__((address_space(1)))
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#pragma clang fp contract(off)

namespace ggemm {
namespace {

constexpr int kThreads = 256;
constexpr int kARows = 32;      // rows of A per block
constexpr int kATile = 128;     // k tile of the A residue pass
constexpr int kBCols = 8;       // columns of B per block (32 lanes each)
constexpr int kChains = 8;      // A-row reduction chains
static_assert(kARows == kPrepRows && kBCols == kPrepCols, "prep block shapes");

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

// Residues from the bytes of an integer-valued double x, |x| <= T_N < 2^77 (every row / column is
// scaled into the norm budget T_N).  Exact floor splits at 2^32 write x in 32-bit words,
//   narrow (T_N < 1.5 2^62, N <= 16): x = L + H 2^32,            L in [0, 2^32), |H| < 2^31
//   wide:                             x = L + M 2^32 + H 2^64,   L, M in [0, 2^32), |H| < 2^13
// L and M are used as unsigned bytes, H as balanced signed digits: the bytes of H + 0x80808080
// minus 128 (H + 0x80808080 lies in [0, 2^32), so nothing wraps).  For a modulus p, with byte
// weights 2^(8 i) mod p for the unsigned words and sym(2^(8 i) mod p) for H (times q for folded
// planes):
//   u = v_dot4_u32_u8 over L (and M), then v_dot4_i32_i8 over H; u = x (mod p) and
//       -2^16 <= u < 2^19 + 2^16 (unsigned words give [0, 8 255^2], the signed one [-2^16, 2^16])
//   q = trunc(fmaf(u, ipf, cf)) = floor((u + h) / p) + 2048, h = floor(p / 2), where ipf and
//       cf = (h + 1/2)/p + 2048 are the nearest floats: the exact value (u + h + 1/2)/p + 2048 is
//       positive and below 2^13, its fractional part (j + 1/2)/p is at least 1/(2p) >= 2^-9 from an
//       integer, and the computed one is within |u| 2^-32 + 2^-13 + 2^-12 < 2^-10 of it (checked
//       exhaustively over every u and p on the host)
//   r = u - q p = sym(x mod p) - 2048 p, and 2048 p = 0 (mod 256): its low byte is the stored
//       byte of the symmetric residue in [-h, p - 1 - h]
// Full-rate 32-bit operations only: two or three dot products, three float operations and one
// 24-bit multiply-add per residue, no table lookups.  The bytes equal the reference's
// reduce / negate / symmetric-map sequence (sym(x mod p) is unique).
template <bool kWide>
struct Digits {
  uint32_t w[kWide ? 3 : 2];   // L, (M,) balanced H
};
template <bool kWide>
__device__ __forceinline__ Digits<kWide> digits_of(double x) {
  Digits<kWide> d;
  double h = floor(x * 0x1p-32);   // x = h 2^32 + L: exact
  d.w[0] = (uint32_t)fma(-h, 0x1p32, x);
  if (kWide) {
    const double t = floor(h * 0x1p-32);
    d.w[1] = (uint32_t)fma(-t, 0x1p32, h);
    h = t;
  }
  d.w[kWide ? 2 : 1] = ((uint32_t)(int)h + 0x80808080u) ^ 0x80808080u;
  return d;
}
struct PlaneW {
  uint32_t w0, w1;
  int wh, p;
  float ip, c;
};
template <bool kWide>
__device__ __forceinline__ PlaneW plane_w(const CrtTables* __restrict__ tab, int l, int widx) {
  const uint32_t* w = tab->wb[widx][l];
  return PlaneW{w[0], w[1], (int)w[kWide ? 3 : 2], tab->p[l], tab->ipf[l], tab->cf[l]};
}
__device__ __forceinline__ uint32_t pack4(int r0, int r1, int r2, int r3) {   // low bytes
  const uint32_t lo = __builtin_amdgcn_perm((uint32_t)r1, (uint32_t)r0, 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm((uint32_t)r3, (uint32_t)r2, 0x0c0c0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}
template <int NE, bool kWide>
__device__ __forceinline__ void residue_bytes(const Digits<kWide>* x, const PlaneW& k, uint32_t* out) {
  // groups of up to 8 values, phase by phase, so that dependent dot products are not back to
  // back and few temporaries are live
  constexpr int G = NE < 8 ? NE : 8;
#pragma unroll
  for (int g = 0; g < NE; g += G) {
    uint32_t s[G];
    int u[G], r[G];
#pragma unroll
    for (int e = 0; e < G; ++e) s[e] = __builtin_amdgcn_udot4(x[g + e].w[0], k.w0, 0u, false);
    if (kWide) {
#pragma unroll
      for (int e = 0; e < G; ++e) s[e] = __builtin_amdgcn_udot4(x[g + e].w[1], k.w1, s[e], false);
    }
#pragma unroll
    for (int e = 0; e < G; ++e) u[e] = __builtin_amdgcn_sdot4((int)x[g + e].w[kWide ? 2 : 1], k.wh, (int)s[e], false);
#pragma unroll
    for (int e = 0; e < G; ++e) r[e] = (int)__builtin_fmaf((float)u[e], k.ip, k.c);
#pragma unroll
    for (int e = 0; e < G; ++e) r[e] = __mul24(r[e], -k.p) + u[e];
#pragma unroll
    for (int w = 0; w < G / 4; ++w) out[g / 4 + w] = pack4(r[4 * w], r[4 * w + 1], r[4 * w + 2], r[4 * w + 3]);
  }
}
// x 2^sh for NE values (mul_pow2 of each), the scale formed once when |sh| <= 1000 (the common case)
template <int NE>
__device__ __forceinline__ void scaled(const double* x, int sh, double* out) {
  if (sh >= -1000 && sh <= 1000) {
    const double sc = pow2d(sh);
#pragma unroll
    for (int e = 0; e < NE; ++e) out[e] = x[e] * sc;
  } else {
#pragma unroll
    for (int e = 0; e < NE; ++e) out[e] = mul_pow2(x[e], sh);
  }
}
// Residue planes 0..N-1 of NE consecutive k (integer-valued doubles) of one row / column: NE bytes
// per plane at dst + l * stride (one 128-bit or 32-bit store).  Three-word digits of 16 values
// take two passes of 8 (64-bit stores), which keeps the kernel's register count for the common
// two-word case.
template <int NE, bool kWide>
__device__ __forceinline__ void planes(const double* xt, int N, const CrtTables* __restrict__ tab, int widx,
                                       GLOBAL int8_t* dst, size_t stride) {
  constexpr int P = (kWide && NE > 8) ? 8 : NE;   // values per pass
#pragma unroll
  for (int h = 0; h < NE; h += P) {
    Digits<kWide> x[P];
#pragma unroll
    for (int e = 0; e < P; ++e) x[e] = digits_of<kWide>(xt[h + e]);
    for (int l = 0; l < N; ++l) {
      uint32_t q[P / 4];
      residue_bytes<P, kWide>(x, plane_w<kWide>(tab, l, widx), q);
      GLOBAL int8_t* d = dst + (size_t)l * stride + h;
      if constexpr (P == 16)
        *(GLOBAL u32x4*)(d) = u32x4{q[0], q[1], q[2], q[3]};
      else if constexpr (P == 8)
        *(GLOBAL u32x2*)(d) = u32x2{q[0], q[1]};
      else
        *(GLOBAL uint32_t*)(d) = q[0];
    }
  }
}
__device__ __forceinline__ uint32_t abs_u8(double a, int sig) {
  if (sig == OZ2_SHIFT_ZERO) return 0;
  return (uint32_t)(int)fmin(127.0, trunc(mul_pow2(fabs(a), sig)));
}

struct PrepShared {
  double red0[kChains][kARows];
  double red1[kChains][kARows];
  int shift[kARows], sig[kARows];
  double rowmax[kARows];
  double tile[kATile][kARows];      // A values of the current k-tile, k-major
  // non-finite summaries of the block's rows (A) or columns (B, slot = the column's 32-lane group):
  // infinities listed so far, NaN seen, largest finite magnitude (bits of a non-negative double)
  int nfcnt[kARows], nfnan[kARows];
  unsigned long long nfmx[kARows];
};

// The summary's words 0 and 1 from the LDS state.
__device__ __forceinline__ void nf_header(GLOBAL int32_t* nfw, int ni, int nan, unsigned long long mx) {
  nfw[0] = (nan ? 1 : 0) | (ni > kNfCap ? 2 : 0) | (min(ni, kNfCap) << 8);
  nfw[1] = mx ? ilogb(__longlong_as_double((long long)mx)) : kNfNoFinite;
}

// ------------------------------------------------------------------------------- A rows
template <bool kWide>
__device__ void prep_rows(const oz2_problem& pr, const CrtTables* __restrict__ tab, int blk, int split,
                          int nsplit, PrepShared& sm, unsigned long long* cnt, int widx, bool packed, int32_t* nfo,
                          int* nff, bool zero_nf, const YDesc* yds, int pi) {
  const int tid = threadIdx.x;
  // split 0, when the call asks for summaries: pass 1, which reads every value of the block's rows,
  // also collects each row's non-finite summary state (NaN seen, largest finite magnitude,
  // infinity positions); it is written for the rows whose shift turns out non-finite
  const bool trk = nfo && split == 0;   // block-uniform
  if (trk) {
    if (tid < kARows) {
      sm.nfcnt[tid] = 0;
      sm.nfnan[tid] = 0;
      sm.nfmx[tid] = 0ull;
    }
    __syncthreads();
  }
  const int N = pr.num_moduli, K = pr.k, Kp = pr.kp, m = pr.m;
  const int row0 = blk * kARows;
  const int r = tid & 31, c = tid >> 5;          // chain role: row r, chain c
  const int i = row0 + r;
  const bool valid = i < m;
  const GLOBAL double* __restrict__ A = (const GLOBAL double*)pr.A;
  const size_t lda = (size_t)pr.lda;
  const double T = tab->T[N];

  // ---- pass 1: row max and sum of squares, chain c = k mod 8 ascending.  With trk, mx is the
  // largest FINITE magnitude and every infinity is listed instead; the row max is then infinite
  // exactly when the row's infinity count is nonzero, so the shift is the same
  double mx = 0.0, ss = 0.0;
  auto step = [&](double a, int k) {
    ss = fma(a, a, ss);
    if (!trk) {
      mx = fmax(mx, fabs(a));
      return;
    }
    const double aa = fabs(a);
    const bool inf = aa == __builtin_inf();
    mx = fmax(mx, inf ? 0.0 : aa);
    if (inf) {   // rare: the summary's address is formed here, not kept live through the pass
      const int x = atomicAdd(&sm.nfcnt[r], 1);
      if (x < kNfCap) ((GLOBAL int32_t*)nfo)[(size_t)kNfWords * i + 2 + x] = k | (a < 0.0 ? (int)0x80000000u : 0);
    }
  };
  if (valid) {
    int k = c;
    // groups of 16 k per chain, software-pipelined: the next group's loads are issued before this
    // group's chain, so 16 to 32 loads stay in flight (a long-k block is one of few workgroups and
    // streams megabytes); the load past the last group re-reads it (in bounds) so that the load
    // count between two waits is the same on every path
    auto ld16 = [&](double (&a)[16], int k0) {
#pragma unroll
      for (int t = 0; t < 16; ++t) a[t] = A[i + (size_t)(k0 + 8 * t) * lda];
    };
    auto chain16 = [&](const double (&a)[16], int k0) {
#pragma unroll
      for (int t = 0; t < 16; ++t) step(a[t], k0 + 8 * t);
    };
    if (k + 8 * 15 < K) {
      double a[16], b[16];
      ld16(a, k);
      for (;;) {
        bool more = k + 8 * 31 < K;
        ld16(b, more ? k + 128 : k);
        chain16(a, k);
        k += 128;
        if (!more) break;
        more = k + 8 * 31 < K;
        ld16(a, more ? k + 128 : k);
        chain16(b, k);
        k += 128;
        if (!more) break;
      }
    }
    for (; k < K; k += 8) step(A[i + (size_t)k * lda], k);
    if (trk && isnan(ss)) sm.nfnan[r] = 1;   // a sum of squares turns NaN only through a NaN
  }
  sm.red0[c][r] = mx;
  __syncthreads();
  if (c == 0) {
    double M = 0.0;
    for (int q = 0; q < kChains; ++q) M = fmax(M, sm.red0[q][r]);
    if (trk) {   // M is the largest finite magnitude: the summary's, and infinite row max if any Inf
      sm.nfmx[r] = (unsigned long long)__double_as_longlong(M);
      if (sm.nfcnt[r] > 0) M = __builtin_inf();
    }
    sm.rowmax[r] = M;
  }
  __syncthreads();
  const double rowmax = sm.rowmax[r];
  // (an infinite row max already makes the shift non-finite: no rescaled second read of the row)
  const bool resc = valid && isfinite(rowmax) && needs_rescale(rowmax);
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
      ((GLOBAL int32_t*)pr.row_shift)[i] = sh;
      ((GLOBAL int32_t*)pr.row_shift)[m + i] = sg;
      if (sh == OZ2_SHIFT_NONFINITE) {
        atomicAdd(counter_slot(cnt), 1ull);
        if (nff) *nff = 1;   // (every writer stores the same value)
      }
    }
  }
  __syncthreads();
  // the rows' finite flags (the descriptor is formed here, not kept live through the pass)
  uint8_t* const frw = (split == 0 && yds) ? yds[pi].fr : nullptr;
  if (frw && tid < kARows && row0 + tid < m) frw[row0 + tid] = sm.shift[tid] != OZ2_SHIFT_NONFINITE ? 1 : 0;

  // ---- pass 2: residues of this split's k-tiles; split 0 also walks every tile for the
  //      ordered ||dA||, ||A'|| chain sums (the residue values do not depend on the split)
  const int sh_c = sm.shift[r];
  const bool nf_c = sh_c == OZ2_SHIFT_NONFINITE;
  const int rr = tid & 31, seg = tid >> 5;   // residue role: row rr, k = 16 seg .. 16 seg + 15
  const int sh_r = sm.shift[rr], sg_r = sm.sig[rr];
  const bool nf_r = sh_r == OZ2_SHIFT_NONFINITE;
  const bool rvalid = row0 + rr < m;
  double da2 = 0.0, na2 = 0.0;
  const bool nfr = trk && nf_c && valid;   // the row's summary is written (state from pass 1)
  const int ntile = (Kp + kATile - 1) / kATile;
  const int per = (ntile + nsplit - 1) / nsplit;
  const int w0 = min(ntile, split * per), w1 = min(ntile, w0 + per);   // tiles written here
  int l0 = split == 0 ? 0 : w0, l1 = split == 0 ? ntile : w1;   // tiles walked here
  // without zero residues, a block whose every row is non-finite has nothing to walk (its rows'
  // sums stay 0, as the walk leaves them)
  if (!zero_nf && __syncthreads_and(!valid || nf_c)) l1 = l0;
  for (int t = l0; t < l1; ++t) {
    const int k0 = t * kATile;
    double av[kATile / kChains];
#pragma unroll
    for (int jj = 0; jj < kATile / kChains; ++jj) {   // non-finite rows: zero residues, nothing to read
      const int k = k0 + c + kChains * jj;
      av[jj] = (valid && !nf_c && k < K) ? A[i + (size_t)k * lda] : 0.0;
    }
    if (!nf_c && split == 0) {
      double xs[kATile / kChains];
      scaled<kATile / kChains>(av, sh_c, xs);
#pragma unroll
      for (int jj = 0; jj < kATile / kChains; ++jj) {
        const double xt = trunc(xs[jj]);
        const double fr = xs[jj] - xt;
        da2 = fma(fr, fr, da2);
        na2 = fma(xt, xt, na2);
      }
    }
#pragma unroll
    for (int jj = 0; jj < kATile / kChains; ++jj) sm.tile[c + kChains * jj][r] = av[jj];
    __syncthreads();
    const int kb = k0 + 16 * seg;
    if (t >= w0 && t < w1 && rvalid && kb < Kp) {
      GLOBAL int8_t* dst = (GLOBAL int8_t*)pr.A8 + (packed ? packed_offset(row0 + rr, kb, m, Kp) : (size_t)(row0 + rr) * Kp + kb);
      if (nf_r) {
        if (zero_nf)
          for (int l = 0; l <= N; ++l)
            *(GLOBAL u32x4*)(dst + (size_t)l * pr.a8_mod_stride) = u32x4{0u, 0u, 0u, 0u};
      } else {
        double av[16], xt[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) av[e] = sm.tile[16 * seg + e][rr];
        uint32_t q[4];   // abs plane first, so the A values are dead during the residue planes
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          q[w] = 0u;
#pragma unroll
          for (int e = 0; e < 4; ++e) q[w] |= abs_u8(av[4 * w + e], sg_r) << (8 * e);
        }
        *(GLOBAL u32x4*)(dst + (size_t)N * pr.a8_mod_stride) = u32x4{q[0], q[1], q[2], q[3]};
        scaled<16>(av, sh_r, xt);
#pragma unroll
        for (int e = 0; e < 16; ++e) xt[e] = trunc(xt[e]);
        planes<16, kWide>(xt, N, tab, widx, dst, pr.a8_mod_stride);
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
    if (nfr) nf_header((GLOBAL int32_t*)nfo + (size_t)kNfWords * i, sm.nfcnt[r], sm.nfnan[r], sm.nfmx[r]);
    ((GLOBAL int32_t*)pr.row_shift)[2 * m + i] = norm_ub_bits(D);
    ((GLOBAL int32_t*)pr.row_shift)[3 * m + i] = norm_ub_bits(Nn);
  }
}

// ---------------------------------------------------------------------------- B columns
constexpr int kBReg = 32;   // column values per lane held in registers (K <= 32 kBReg: one read of B)

template <bool kWide>
__device__ void prep_cols(const oz2_problem& pr, const CrtTables* __restrict__ tab, int blk, int split,
                          int nsplit, PrepShared& sm, unsigned long long* cnt, bool packed, int32_t* nfo, int* nff,
                          bool zero_nf, const YDesc* yds, int pi) {
  const int lane = threadIdx.x & 31, w = threadIdx.x >> 5;
  const int j = blk * kBCols + w;
  const int n = pr.n, N = pr.num_moduli, K = pr.k, Kp = pr.kp;
  if (j >= n) return;   // no barriers below; the 32-lane group is column-uniform
  if (nfo && lane == 0) {   // the column's summary state (used by this 32-lane group only)
    sm.nfcnt[w] = 0;
    sm.nfnan[w] = 0;
    sm.nfmx[w] = 0ull;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const GLOBAL double* __restrict__ b = (const GLOBAL double*)pr.B + (size_t)j * pr.ldb;
  const double T = tab->T[N];
  // split 0 with summaries: pass 1 collects the column's summary state, as for the A rows (mx the
  // largest finite magnitude, the infinities listed)
  const bool trk = nfo && split == 0;   // column-uniform
  // (the summary's address is formed where it is used: a pointer live through the passes would
  // take the kernel past its register budget)
  auto nfw = [&]() { return (GLOBAL int32_t*)nfo + (size_t)kNfWords * ((size_t)pr.m + j); };

  // K <= 32 kBReg: the column is read once; lane l keeps k = l + 32 t in registers (its norm chain,
  // zeros past K change neither the max nor the sums) and gets the residue pass's 4 consecutive k
  // per chunk through a wave-private LDS exchange row
  // (two-word digits only: with three-word digits the kernel would exceed 128 VGPRs)
  const bool single = !kWide && K <= 32 * kBReg;
  double v[kBReg];
  double mx = 0.0, ss = 0.0;
  auto step = [&](double a, int k) {   // as for the A rows
    ss = fma(a, a, ss);
    if (!trk) {
      mx = fmax(mx, fabs(a));
      return;
    }
    const double aa = fabs(a);
    const bool inf = aa == __builtin_inf();
    mx = fmax(mx, inf ? 0.0 : aa);
    if (inf) {
      const int x = atomicAdd(&sm.nfcnt[w], 1);
      if (x < kNfCap) nfw()[2 + x] = k | (a < 0.0 ? (int)0x80000000u : 0);
    }
  };
  if (single) {
#pragma unroll
    for (int t = 0; t < kBReg; ++t) v[t] = lane + 32 * t < K ? b[lane + 32 * t] : 0.0;
#pragma unroll
    for (int t = 0; t < kBReg; ++t) {
      mx = fmax(mx, fabs(v[t]));
      ss = fma(v[t], v[t], ss);
    }
    // the values are still in registers: the summary state is collected only when the column
    // turns out non-finite (any lane), from them
    if (trk && __any(!isfinite(mx) || isnan(ss))) {
      double mf = 0.0;
#pragma unroll
      for (int t = 0; t < kBReg; ++t) {
        const double aa = fabs(v[t]);
        const bool inf = aa == __builtin_inf();
        mf = fmax(mf, inf ? 0.0 : aa);
        if (inf) {
          const int x = atomicAdd(&sm.nfcnt[w], 1);
          if (x < kNfCap) nfw()[2 + x] = (lane + 32 * t) | (v[t] < 0.0 ? (int)0x80000000u : 0);
        }
      }
      mx = mf;   // with trk, mx is the largest finite magnitude (the infinities are counted)
    }
  } else {
    int k = lane;
    // groups of 16 k per lane, software-pipelined as in the A-row pass (16 to 32 loads in flight)
    auto ld16 = [&](double (&a)[16], int k0) {
#pragma unroll
      for (int t = 0; t < 16; ++t) a[t] = b[k0 + 32 * t];
    };
    auto chain16 = [&](const double (&a)[16], int k0) {
#pragma unroll
      for (int t = 0; t < 16; ++t) step(a[t], k0 + 32 * t);
    };
    if (k + 32 * 15 < K) {
      double a[16], c[16];
      ld16(a, k);
      for (;;) {
        bool more = k + 32 * 31 < K;
        ld16(c, more ? k + 512 : k);
        chain16(a, k);
        k += 512;
        if (!more) break;
        more = k + 32 * 31 < K;
        ld16(a, more ? k + 512 : k);
        chain16(c, k);
        k += 512;
        if (!more) break;
      }
    }
    for (; k < K; k += 32) step(b[k], k);
  }
  if (trk && isnan(ss)) sm.nfnan[w] = 1;   // a sum of squares turns NaN only through a NaN
#pragma unroll
  for (int o = 16; o; o >>= 1) mx = fmax(mx, __shfl_xor(mx, o, 32));
  if (trk) {   // every lane's counter update precedes the reads; mx is the largest finite magnitude
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane == 0) sm.nfmx[w] = (unsigned long long)__double_as_longlong(mx);
    if (sm.nfcnt[w] > 0) mx = __builtin_inf();
  }
  // (an infinite column max already makes the shift non-finite: no rescaled second read)
  const bool resc = isfinite(mx) && needs_rescale(mx);
  if (resc) {
    const int e = -ilogb(mx);
    ss = 0.0;
    if (single) {
#pragma unroll
      for (int t = 0; t < kBReg; ++t) {
        const double a = mul_pow2(v[t], e);
        ss = fma(a, a, ss);
      }
    } else {
      for (int k = lane; k < K; k += 32) {
        const double a = mul_pow2(b[k], e);
        ss = fma(a, a, ss);
      }
    }
  }
#pragma unroll
  for (int o = 16; o; o >>= 1) ss += __shfl_xor(ss, o, 32);
  const int sh = shift_from_norm(mx, ss, resc, T);
  const int sg = abs_shift(mx, sh);
  if (lane == 0 && split == 0) {
    ((GLOBAL int32_t*)pr.col_shift)[j] = sh;
    ((GLOBAL int32_t*)pr.col_shift)[n + j] = sg;
    if (sh == OZ2_SHIFT_NONFINITE) {
      atomicAdd(counter_slot(cnt), 1ull);
      if (nff) *nff = 1;
    }
  }
  if (split == 0 && yds && lane == 0) {   // the column's finite flag
    uint8_t* const fcw = yds[pi].fc;
    if (fcw) fcw[j] = sh != OZ2_SHIFT_NONFINITE ? 1 : 0;
  }
  const bool nf = sh == OZ2_SHIFT_NONFINITE;

  const bool nfc = trk && nf;   // the column's summary is written (state from pass 1; column-uniform)

  double da2 = 0.0, na2 = 0.0;
  GLOBAL int8_t* const B8 = (GLOBAL int8_t*)pr.B8;
  const int nchunk = (Kp + 127) / 128;
  const int per = (nchunk + nsplit - 1) / nsplit;
  const int c0 = min(nchunk, split * per), c1 = min(nchunk, c0 + per);
  // split 0 walks every chunk (ordered sums) but writes residues only for its own range; lane L
  // owns k = 128 ch + 4 L + e
  // chunk ch's residues from its values a (lane l: k = 128 ch + 4 l + e)
  auto chunk = [&](int ch, const double (&a)[4]) {
    const int k0 = 128 * ch + 4 * lane;
    if (k0 >= Kp) return;
    GLOBAL int8_t* const base = B8 + (packed ? packed_offset(j, k0, n, Kp) : (size_t)j * Kp + k0);
    const bool write = ch >= c0 && ch < c1;
    if (nf) {
      if (write && zero_nf)
        for (int l = 0; l <= N; ++l) *(GLOBAL uint32_t*)(base + (size_t)l * pr.b8_mod_stride) = 0u;
      return;
    }
    double xs[4], xt[4];
    scaled<4>(a, sh, xs);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xt[e] = trunc(xs[e]);
      const double fr = xs[e] - xt[e];
      if (split == 0) {
        da2 = fma(fr, fr, da2);
        na2 = fma(xt[e], xt[e], na2);
      }
    }
    if (!write) return;
    planes<4, kWide>(xt, N, tab, 0, base, pr.b8_mod_stride);
    uint32_t q = 0u;
#pragma unroll
    for (int e = 0; e < 4; ++e) q |= abs_u8(a[e], sg) << (8 * e);
    *(GLOBAL uint32_t*)(base + (size_t)N * pr.b8_mod_stride) = q;
  };
  const int ch0 = split == 0 ? 0 : c0, ch1 = split == 0 ? nchunk : c1;   // chunks walked here
  if (single) {
    // lane l holds k = 128 ch + 32 jj + l (jj < 4) of chunk ch in v[4 ch + jj]: through this column's
    // LDS exchange row to k = 128 ch + 4 l + e; unrolled so that the register indices are static
    double* const xb = reinterpret_cast<double*>(&sm.tile[0][0]) + 128 * w;
#pragma unroll
    for (int ch = 0; ch < kBReg / 4; ++ch) {
      if (ch < ch0 || ch >= ch1) continue;   // column-uniform
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) xb[32 * jj + lane] = v[4 * ch + jj];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      double a[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) a[e] = xb[4 * lane + e];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");   // the reads precede the next chunk's writes
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      chunk(ch, a);
    }
  } else if (nf) {   // a non-finite column: zero residues (when asked for), nothing to read
    for (int ch = c0; ch < (zero_nf ? c1 : c0); ++ch) {
      const int k0 = 128 * ch + 4 * lane;
      if (k0 < Kp)
        for (int l = 0; l <= N; ++l)
          *(GLOBAL uint32_t*)(B8 + (packed ? packed_offset(j, k0, n, Kp) : (size_t)j * Kp + k0) +
                              (size_t)l * pr.b8_mod_stride) = 0u;
    }
  } else {
    for (int ch = ch0; ch < ch1; ++ch) {
      const int k0 = 128 * ch + 4 * lane;
      double a[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) a[e] = (k0 + e < K) ? b[k0 + e] : 0.0;
      chunk(ch, a);
    }
  }
  if (split != 0) return;
#pragma unroll
  for (int o = 16; o; o >>= 1) {
    da2 += __shfl_xor(da2, o, 32);
    na2 += __shfl_xor(na2, o, 32);
  }
  if (lane == 0) {
    ((GLOBAL int32_t*)pr.col_shift)[2 * n + j] = norm_ub_bits(da2);
    ((GLOBAL int32_t*)pr.col_shift)[3 * n + j] = norm_ub_bits(na2);
  }
  if (nfc) {   // every lane's LDS updates precede lane 0's reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane == 0) nf_header(nfw(), sm.nfcnt[w], sm.nfnan[w], sm.nfmx[w]);
  }
}

// kWide: three-word digits (any N); the two-word kernel is launched only for calls whose every
// problem has T_N < 1.5 2^62.
// Grid: compact (pofs != nullptr) -- blockIdx.x runs over the real blocks of all problems, problem
// order[i] owning blocks pofs[i] .. pofs[i + 1] - 1, its A-row blocks first; else blockIdx.y is the
// problem (through order when given) and blockIdx.x one of a_blocks A-row blocks or a B-column
// block, as wide as the largest problem.
template <bool kWide>
__global__ void __launch_bounds__(kThreads, 4) prep_kernel(const oz2_problem* __restrict__ probs, int a_blocks,
                                                        const CrtTables* __restrict__ tab,
                                                        unsigned long long* __restrict__ cnt, int fold_q,
                                                        int packed_kp, const YDesc* __restrict__ yds,
                                                        const int* __restrict__ order, const int* __restrict__ pofs,
                                                        int nprob) {
  __shared__ PrepShared sm;
  int pi, blk = (int)blockIdx.x;
  if (pofs) {   // the last problem whose first block is at most blockIdx.x (empty problems are skipped)
    int lo = 0, hi = nprob - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (pofs[mid] <= blk) lo = mid; else hi = mid - 1;
    }
    pi = order[lo];
    blk -= pofs[lo];
    a_blocks = (probs[pi].m + kARows - 1) / kARows;
  } else {
    pi = order ? order[blockIdx.y] : (int)blockIdx.y;
  }
  const oz2_problem& pr = probs[pi];
  int32_t* const nfo = yds ? yds[pi].nf : nullptr;
  // the problem's non-finite flag (the descriptors are device memory of this call)
  int* const nff = yds ? const_cast<int*>(&yds[pi].nff) : nullptr;
  const int N = pr.num_moduli;
  if (N < 1 || N > kMaxModuli || pr.alpha == 0.0) return;   // alpha == 0: A, B never referenced
  // folded A residues use the weights q 2^(8 i) mod p, so that sum b_i [q 2^(8 i)] = q x (mod p)
  const bool fold = fold_q && blk < a_blocks;
  const bool packed = pr.kp <= packed_kp;   // packed_kp = 0: row-major (every Kp >= 32)
  // the residues of a non-finite row / column: zeros for the kernel-level API (fold_q = 0), which
  // hands the planes over; the grouped pipeline (fold_q = 1) leaves them unwritten, since every
  // entry in such a row or column takes the safety fallback, which uses neither its digits nor its
  // L (the GEMM's int32 sums over whatever bytes the planes hold are dropped with those entries)
  const bool zero_nf = !fold_q;
  if (blk < a_blocks) {
    if (blk * kARows >= pr.m) return;
    prep_rows<kWide>(pr, tab, blk, blockIdx.z, gridDim.z, sm, cnt, fold ? N : 0, packed, nfo, nff, zero_nf, yds, pi);
  } else {
    prep_cols<kWide>(pr, tab, blk - a_blocks, blockIdx.z, gridDim.z, sm, cnt, packed, nfo, nff, zero_nf, yds, pi);
  }
}

int g_force_split = 0;

}  // namespace

int prep_launch(const oz2_problem* d, int num, int max_m, int max_n, hipStream_t s, int fold_q, int packed_kp,
                int max_moduli, const YDesc* yd, const int* order, const int* pofs, long long total_blocks) {
  if (num <= 0) return 0;
  if (num > 65535 || max_m < 0 || max_n < 0 || max_moduli < 1 || max_moduli > kMaxModuli) return 1;
  if (pofs && (!order || total_blocks < 0 || total_blocks > 0x7fffffffLL)) return 1;
  DevCtx* c = dev_ctx();
  if (!c) return 2;
  const int a_blocks = (max_m + kARows - 1) / kARows;
  const int b_blocks = (max_n + kBCols - 1) / kBCols;
  if (a_blocks + b_blocks == 0) return 0;
  const long long blocks = pofs ? total_blocks : (long long)(a_blocks + b_blocks) * num;
  if (blocks == 0) return 0;
  const dim3 grid = pofs ? dim3((unsigned)blocks, 1, 1) : dim3(a_blocks + b_blocks, num, 1);
  const long long target = 4LL * c->num_cus;
  int S = (int)std::min<long long>(16, std::max<long long>(1, (target + blocks - 1) / blocks));
  if (g_force_split > 0) S = g_force_split;
  const CrtTables* ht = host_tables();
  if (!ht) return 2;
  const dim3 g3(grid.x, grid.y, S);
  if (ht->T[max_moduli] < 0x1.8p62)
    hipLaunchKernelGGL(prep_kernel<false>, g3, dim3(kThreads), 0, s, d, a_blocks, c->tab, c->counters, fold_q,
                       packed_kp, yd, order, pofs, num);
  else
    hipLaunchKernelGGL(prep_kernel<true>, g3, dim3(kThreads), 0, s, d, a_blocks, c->tab, c->counters, fold_q,
                       packed_kp, yd, order, pofs, num);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

}  // namespace ggemm

extern "C" int oz2_prep_grouped(const oz2_problem* d, int num, int max_m, int max_n, hipStream_t s) {
  return ggemm::prep_launch(d, num, max_m, max_n, s, 0, 0, ggemm::kMaxModuli);   // N is device-side only
}

extern "C" void oz2_debug_force_prep_split(int S) { ggemm::g_force_split = (S >= 1 && S <= 64) ? S : 0; }
