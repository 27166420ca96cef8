/* oz2_oracle.c -- CPU oracle for the grouped Ozaki-II FP64 GEMM (TEST INFRASTRUCTURE ONLY).
 *
 * Plain C restatement of the reference's behaviour, written from its formulas and operation
 * order; what tests/, smoke() and bench.py's cpu_baseline leg compare against.  See oz2_oracle.h
 * for what pins each part.  Build: oracle/Makefile (gcc, -ffp-contract=off so that only the
 * fma() calls written below fuse, matching the reference's explicit fma()s and the two
 * multiply-adds its device compiler contracts).
 */
#include "oz2_oracle.h"

#include <float.h>
#include <limits.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ moduli and CRT tables */
/* src/moduli.h:39-41: the 16 INT8 moduli of Ozaki scheme II followed by 181, 179, 173, 167. */
static const int kModuli[OZ2O_MAX_MODULI] = {256, 255, 253, 251, 247, 239, 233, 229, 227, 223,
                                             217, 211, 199, 197, 193, 191, 181, 179, 173, 167};

/* Fixed-width little-endian big integer (P_N < 2^160). */
#define BW 8
typedef struct { uint32_t w[BW]; } big;

static void big_set(big* a, uint64_t v) {
  memset(a, 0, sizeof *a);
  a->w[0] = (uint32_t)v;
  a->w[1] = (uint32_t)(v >> 32);
}
static void big_mul_u32(big* a, uint32_t m) {
  uint64_t c = 0;
  for (int i = 0; i < BW; ++i) {
    uint64_t t = (uint64_t)a->w[i] * m + c;
    a->w[i] = (uint32_t)t;
    c = t >> 32;
  }
}
static uint32_t big_div_u32(const big* a, uint32_t d, big* q) {
  uint64_t r = 0;
  big out;
  memset(&out, 0, sizeof out);
  for (int i = BW - 1; i >= 0; --i) {
    uint64_t cur = (r << 32) | a->w[i];
    out.w[i] = (uint32_t)(cur / d);
    r = cur % d;
  }
  if (q) *q = out;
  return (uint32_t)r;
}
static int big_bits(const big* a) {
  for (int i = BW - 1; i >= 0; --i)
    if (a->w[i]) {
      int b = 0;
      uint32_t t = a->w[i];
      while (t) { ++b; t >>= 1; }
      return 32 * i + b;
    }
  return 0;
}
static int big_bit(const big* a, int i) {
  if (i < 0 || i >= 32 * BW) return 0;
  return (a->w[i / 32] >> (i % 32)) & 1u;
}
/* floor(a / 2^s) for s >= 0, or a * 2^-s for s < 0 */
static big big_shift_right(const big* a, int s) {
  big r;
  memset(&r, 0, sizeof r);
  int nb = big_bits(a);
  for (int i = 0; i < nb; ++i)
    if (big_bit(a, i)) {
      int j = i - s;
      if (j >= 0 && j < 32 * BW) r.w[j / 32] |= 1u << (j % 32);
    }
  return r;
}
static big big_low_bits(const big* a, int s) { /* a mod 2^s */
  big r;
  memset(&r, 0, sizeof r);
  for (int i = 0; i < s && i < 32 * BW; ++i)
    if (big_bit(a, i)) r.w[i / 32] |= 1u << (i % 32);
  return r;
}
static uint64_t big_u64(const big* a) { return ((uint64_t)a->w[1] << 32) | a->w[0]; }
/* src/moduli.h:115-118: Horner over 32-bit limbs in x87 long double, then rounded to double. */
static double big_double(const big* a) {
  long double v = 0.0L;
  for (int i = BW - 1; i >= 0; --i) v = v * 4294967296.0L + (long double)a->w[i];
  return (double)v;
}
static int gcd_int(int a, int b) {
  while (b) { int t = a % b; a = b; b = t; }
  return a;
}

/* src/moduli.h:124-181 */
int oz2o_build_tables(oz2o_tables* t) {
  memset(t, 0, sizeof *t);
  for (int a = 0; a < OZ2O_MAX_MODULI; ++a)
    for (int b = a + 1; b < OZ2O_MAX_MODULI; ++b)
      if (gcd_int(kModuli[a], kModuli[b]) != 1) return 1;
  for (int l = 0; l < OZ2O_MAX_MODULI; ++l) {
    const int p = kModuli[l];
    t->p[l] = p;
    t->magic[l] = (uint32_t)((1ull << 32) / (uint64_t)p);
    unsigned v = 1u % (unsigned)p;
    for (int e = 0; e < OZ2O_POW2_TABLE; ++e) { t->pow2[l][e] = (uint8_t)v; v = (v * 2u) % (unsigned)p; }
  }
  for (int N = 1; N <= OZ2O_MAX_MODULI; ++N) {
    big P, M[OZ2O_MAX_MODULI];
    big_set(&P, 1);
    for (int l = 0; l < N; ++l) big_mul_u32(&P, (uint32_t)kModuli[l]);
    int maxbits = 0;
    for (int l = 0; l < N; ++l) {
      const int p = kModuli[l];
      if (big_div_u32(&P, (uint32_t)p, &M[l]) != 0) return 3;
      const int mr = (int)big_div_u32(&M[l], (uint32_t)p, NULL);
      int inv = -1;
      for (int x = 0; x < p; ++x)
        if ((mr * x) % p == 1 % p) { inv = x; break; }
      if (inv < 0) return 4;
      t->qinv[N][l] = inv;
      const int b = big_bits(&M[l]);
      if (b > maxbits) maxbits = b;
    }
    const int sh = maxbits - 49; /* u1 = 2^sh, every M_l / u1 < 2^49 */
    t->log2_u1[N] = sh;
    for (int l = 0; l < N; ++l) {
      if (sh >= 0) {
        big hi = big_shift_right(&M[l], sh);
        t->s1[N][l] = big_u64(&hi);
        big low = big_low_bits(&M[l], sh);
        uint64_t s2;
        if (sh >= OZ2O_S2_BITS) {
          big top = big_shift_right(&low, sh - OZ2O_S2_BITS);
          s2 = big_u64(&top) + (uint64_t)big_bit(&low, sh - OZ2O_S2_BITS - 1); /* round half up */
        } else {
          s2 = big_u64(&low) << (OZ2O_S2_BITS - sh);
        }
        if (s2 > (1u << OZ2O_S2_BITS)) return 5;
        t->s2[N][l] = (uint32_t)s2;
      } else {
        big hi = big_shift_right(&M[l], sh);
        t->s1[N][l] = big_u64(&hi);
        t->s2[N][l] = 0;
      }
      if (t->s1[N][l] >= (1ull << 49)) return 6;
    }
    big P1 = big_shift_right(&P, sh);
    if (big_bits(&P1) > 57) return 7;
    t->P1[N] = (int64_t)big_u64(&P1);
    if (sh > 0) {
      big low = big_low_bits(&P, sh);
      t->P2[N] = ldexp(big_double(&low), -sh);
    } else {
      t->P2[N] = 0.0;
    }
    t->inv_Pu[N] = 1.0 / ((double)t->P1[N] + t->P2[N]);
    const double Pd = big_double(&P);
    t->log2P[N] = log2(Pd);
    t->T[N] = sqrt(Pd * 0.5 * (1.0 - ldexp(1.0, -20))) * (1.0 - ldexp(1.0, -40));
  }
  return 0;
}

static oz2o_tables g_tab;
static int g_tab_state = -1;
const oz2o_tables* oz2o_tables_get(void) {
  if (g_tab_state < 0) g_tab_state = oz2o_build_tables(&g_tab);
  return g_tab_state == 0 ? &g_tab : NULL;
}

/* ----------------------------------------------------------- a-priori bound and choice of N */
/* src/ozaki2_numerics.cu:639-650 */
double oz2o_error_bound(int k, int N) {
  const oz2o_tables* t = oz2o_tables_get();
  if (!t || N < 1 || N > OZ2O_MAX_MODULI || k < 0) return INFINITY;
  const double T = t->T[N];
  const double T2 = T * T;
  const double kk = (double)k;
  const double u = ldexp(1.0, -53);
  const double u1 = ldexp(1.0, t->log2_u1[N]);
  return 4.0 * sqrt(kk) / T + 4.0 * kk / T2 +
         4.0 * u1 * (N * 255.0 * ldexp(1.0, -19) + ldexp(1.0, -10)) / T2 + u;
}
/* src/ozaki2_numerics.cu:652-657 */
int oz2o_choose_num_moduli(int k, double target) {
  if (k < 0 || k > OZ2O_MAX_K) return -1;
  for (int N = 2; N <= OZ2O_MAX_MODULI; ++N)
    if (oz2o_error_bound(k, N) <= target) return N;
  return -1;
}
/* src/ozaki2_numerics.cu:665-673 */
int oz2o_choose_num_moduli_cw(int k, double rho) {
  if (k < 0 || k > OZ2O_MAX_K) return -1;
  if (rho < 1.0) rho = 1.0;
  const double u = ldexp(1.0, -53);
  const double budget = 0.5 * (k > 2 ? (double)(k - 2) : 1.0) * u;
  for (int N = 2; N <= OZ2O_MAX_MODULI; ++N)
    if ((oz2o_error_bound(k, N) - u) * rho <= budget) return N;
  return OZ2O_MAX_MODULI;
}

/* -------------------------------------------------------------------------------- prep */
/* src/ozaki2_numerics.cu:112-121: x * 2^e, one exact multiply for |e| <= 1000, else 3 steps. */
static double mul_pow2(double x, int e) {
  if (e >= -1000 && e <= 1000) return x * ldexp(1.0, e);
  for (int r = 0; r < 3; ++r) {
    int ee = e < -1000 ? -1000 : (e > 1000 ? 1000 : e);
    x *= ldexp(1.0, ee);
    e -= ee;
  }
  return x;
}
/* src/ozaki2_numerics.cu:132-138 */
static int choose_shift(double nrm, int add, double T) {
  int g, G;
  const double f = frexp(nrm, &g);
  const double F = frexp(T, &G);
  g += add;
  return G - g - (f > F ? 1 : 0);
}
/* src/ozaki2_numerics.cu:140-152 */
static int shift_from_norm(double maxabs, double ssq, int rescaled, double T) {
  if (isinf(maxabs) || isnan(ssq)) return OZ2O_SHIFT_NONFINITE;
  if (!(maxabs > 0.0)) return 0;
  const double nm = sqrt(ssq * (1.0 + ldexp(1.0, -30)));
  return choose_shift(nm, rescaled ? ilogb(maxabs) : 0, T);
}
/* src/ozaki2_numerics.cu:155-163 */
static int abs_shift(double maxabs, int sh) {
  if (sh == OZ2O_SHIFT_NONFINITE) return 0;
  if (!(maxabs > 0.0)) return OZ2O_SHIFT_ZERO;
  return 6 - ilogb(maxabs);
}
static int needs_rescale(double maxabs) {
  return maxabs > 0.0 && (maxabs > ldexp(1.0, 400) || maxabs < ldexp(1.0, -400));
}
/* src/ozaki2_numerics.cu:171-201: residue of an integer-valued double |x| < 2^81 modulo p_l,
 * mapped to the symmetric int8 range. */
static void residues_of(double x, int N, const oz2o_tables* t, int8_t* out, size_t plane_stride) {
  const double ax = fabs(x);
  const int neg = x < 0.0;
  uint64_t M;
  int E;
  if (ax < 9007199254740992.0) {
    M = (uint64_t)ax;
    E = 0;
  } else {
    uint64_t b;
    memcpy(&b, &ax, sizeof b);
    E = (int)((b >> 52) & 0x7ff) - 1023 - 52;
    M = (b & ((1ull << 52) - 1)) | (1ull << 52);
    if (E > OZ2O_POW2_TABLE - 37) E = OZ2O_POW2_TABLE - 37;
  }
  const uint32_t c0 = (uint32_t)(M & 0x3ffff), c1 = (uint32_t)((M >> 18) & 0x3ffff),
                 c2 = (uint32_t)(M >> 36);
  for (int l = 0; l < N; ++l) {
    const uint32_t p = (uint32_t)t->p[l];
    const uint32_t s = c0 * t->pow2[l][E] + c1 * t->pow2[l][E + 18] + c2 * t->pow2[l][E + 36];
    uint32_t r = s % p;
    if (neg && r) r = p - r;
    int ri = (int)r;
    if (ri > (int)((p - 1) >> 1)) ri -= (int)p;
    out[(size_t)l * plane_stride] = (int8_t)ri;
  }
}
/* src/ozaki2_numerics.cu:209-226 */
static void prep_elem(double a, int sh, int sig, double* da2, double* na2, int N,
                      const oz2o_tables* t, int8_t* out, size_t plane_stride) {
  if (sh == OZ2O_SHIFT_NONFINITE) {
    for (int l = 0; l <= N; ++l) out[(size_t)l * plane_stride] = 0;
    return;
  }
  const double xs = mul_pow2(a, sh);
  const double xt = trunc(xs);
  const double fr = xs - xt;
  *da2 = fma(fr, fr, *da2);
  *na2 = fma(xt, xt, *na2);
  residues_of(xt, N, t, out, plane_stride);
  out[(size_t)N * plane_stride] =
      (sig == OZ2O_SHIFT_ZERO) ? (int8_t)0 : (int8_t)(int)fmin(127.0, trunc(mul_pow2(fabs(a), sig)));
}
/* float round-up of sqrt(x (1 + 2^-30)) as int bits, src/ozaki2_numerics.cu:229-231 */
static int32_t norm_ub_bits(double x) {
  const double s = sqrt(x * (1.0 + ldexp(1.0, -30)));
  float f = (float)s;
  if ((double)f < s) f = nextafterf(f, INFINITY);
  int32_t b;
  memcpy(&b, &f, sizeof b);
  return b;
}

/* One row of A: the reference's A-path reduction order (src/ozaki2_numerics.cu:274-364):
 * 8 chains, chain c sums k = c, c+8, ... ascending with fma; chains summed c = 0..7. */
static void prep_row(const double* x, size_t stride, int K, int Kp, int N, const oz2o_tables* t,
                     int8_t* out, size_t plane_stride, int32_t* ws, size_t ws_stride,
                     long long* nonfinite) {
  const double T = t->T[N];
  double mx[8], ss[8], da2[8], na2[8];
  for (int c = 0; c < 8; ++c) { mx[c] = ss[c] = da2[c] = na2[c] = 0.0; }
  for (int c = 0; c < 8; ++c)
    for (int k = c; k < K; k += 8) {
      const double a = x[(size_t)k * stride];
      mx[c] = fmax(mx[c], fabs(a));
      ss[c] = fma(a, a, ss[c]);
    }
  double rowmax = 0.0;
  for (int c = 0; c < 8; ++c) rowmax = fmax(rowmax, mx[c]);
  const int resc = needs_rescale(rowmax);
  if (resc) {
    const int e = -ilogb(rowmax);
    for (int c = 0; c < 8; ++c) {
      ss[c] = 0.0;
      for (int k = c; k < K; k += 8) {
        const double a = mul_pow2(x[(size_t)k * stride], e);
        ss[c] = fma(a, a, ss[c]);
      }
    }
  }
  double S = 0.0;
  for (int c = 0; c < 8; ++c) S += ss[c];
  const int sh = shift_from_norm(rowmax, S, resc, T);
  const int sg = abs_shift(rowmax, sh);
  if (sh == OZ2O_SHIFT_NONFINITE && nonfinite) ++*nonfinite;
  for (int k = 0; k < Kp; ++k) {
    const double a = k < K ? x[(size_t)k * stride] : 0.0;
    prep_elem(a, sh, sg, &da2[k & 7], &na2[k & 7], N, t, out + k, plane_stride);
  }
  double D = 0.0, Nn = 0.0;
  for (int c = 0; c < 8; ++c) { D += da2[c]; Nn += na2[c]; }
  ws[0] = sh;
  ws[ws_stride] = sg;
  ws[2 * ws_stride] = norm_ub_bits(D);
  ws[3 * ws_stride] = norm_ub_bits(Nn);
}

/* XOR butterfly over 32 lanes: lane i <- v[i] + v[i^o] for o = 16, 8, 4, 2, 1 (lane 0 result). */
static double butterfly32(const double* v0) {
  double v[32], w[32];
  memcpy(v, v0, sizeof v);
  for (int o = 16; o; o >>= 1) {
    for (int i = 0; i < 32; ++i) w[i] = v[i] + v[i ^ o];
    memcpy(v, w, sizeof v);
  }
  return v[0];
}

/* One column of B: the reference's B-path order (src/ozaki2_numerics.cu:373-440): 32 lane chains
 * k = L, L+32, ... for the norm; lane L covers k = 4L + 128c + e (c ascending, e = 0..3) for the
 * ||dB||, ||B'|| sums; lane partials combined by the XOR butterfly. */
static void prep_col(const double* x, int K, int Kp, int N, const oz2o_tables* t, int8_t* out,
                     size_t plane_stride, int32_t* ws, size_t ws_stride, long long* nonfinite) {
  const double T = t->T[N];
  double mx[32], ss[32], da2[32], na2[32];
  for (int L = 0; L < 32; ++L) {
    mx[L] = ss[L] = da2[L] = na2[L] = 0.0;
    for (int k = L; k < K; k += 32) {
      const double a = x[k];
      mx[L] = fmax(mx[L], fabs(a));
      ss[L] = fma(a, a, ss[L]);
    }
  }
  double colmax = 0.0;
  for (int L = 0; L < 32; ++L) colmax = fmax(colmax, mx[L]);
  const int resc = needs_rescale(colmax);
  if (resc) {
    const int e = -ilogb(colmax);
    for (int L = 0; L < 32; ++L) {
      ss[L] = 0.0;
      for (int k = L; k < K; k += 32) {
        const double a = mul_pow2(x[k], e);
        ss[L] = fma(a, a, ss[L]);
      }
    }
  }
  const double S = butterfly32(ss);
  const int sh = shift_from_norm(colmax, S, resc, T);
  const int sg = abs_shift(colmax, sh);
  if (sh == OZ2O_SHIFT_NONFINITE && nonfinite) ++*nonfinite;
  for (int L = 0; L < 32; ++L)
    for (int k0 = 4 * L; k0 < Kp; k0 += 128)
      for (int e = 0; e < 4; ++e) {
        const int k = k0 + e;
        prep_elem(k < K ? x[k] : 0.0, sh, sg, &da2[L], &na2[L], N, t, out + k, plane_stride);
      }
  ws[0] = sh;
  ws[ws_stride] = sg;
  ws[2 * ws_stride] = norm_ub_bits(butterfly32(da2));
  ws[3 * ws_stride] = norm_ub_bits(butterfly32(na2));
}

static int kp_of(int k) { return (k + 31) / 32 * 32; }

void oz2o_prep_rows(int m, int k, int N, const double* A, int lda, int8_t* A8, int32_t* ws,
                    long long* nonfinite) {
  const oz2o_tables* t = oz2o_tables_get();
  const int kp = kp_of(k);
  const size_t ps = (size_t)m * kp;
  for (int i = 0; i < m; ++i)
    prep_row(A + i, (size_t)lda, k, kp, N, t, A8 + (size_t)i * kp, ps, ws + i, (size_t)m, nonfinite);
}

void oz2o_prep_cols(int n, int k, int N, const double* B, int ldb, int8_t* B8, int32_t* ws,
                    long long* nonfinite) {
  const oz2o_tables* t = oz2o_tables_get();
  const int kp = kp_of(k);
  const size_t ps = (size_t)n * kp;
  for (int j = 0; j < n; ++j)
    prep_col(B + (size_t)j * ldb, k, kp, N, t, B8 + (size_t)j * kp, ps, ws + j, (size_t)n, nonfinite);
}

/* ------------------------------------------------------------------------------ int GEMM */
/* tests/test_i8_grouped.cu:89-96 (int64 brute force); the range check is the kp <= 131040 bound.
 * The exact dot products come from oz2_i8dot.c (vectorised; four columns of B per pass over a row
 * of A). */
int oz2o_i8_gemm(int m, int n, int kp, const int8_t* A8, const int8_t* B8, int32_t* C32) {
  int bad = 0;
  int j = 0;
  for (; j + 4 <= n; j += 4) {
    const int8_t* b = B8 + (size_t)j * kp;
    for (int i = 0; i < m; ++i) {
      int64_t acc[4];
      oz2o_dot4_i8(A8 + (size_t)i * kp, b, b + kp, b + 2 * (size_t)kp, b + 3 * (size_t)kp, kp, acc);
      for (int c = 0; c < 4; ++c) {
        if (acc[c] > INT32_MAX || acc[c] < INT32_MIN) bad = 1;
        C32[i + (size_t)(j + c) * m] = (int32_t)acc[c];
      }
    }
  }
  for (; j < n; ++j)
    for (int i = 0; i < m; ++i) {
      const int64_t acc = oz2o_dot_i8(A8 + (size_t)i * kp, B8 + (size_t)j * kp, kp);
      if (acc > INT32_MAX || acc < INT32_MIN) bad = 1;
      C32[i + (size_t)j * m] = (int32_t)acc;
    }
  return bad;
}

/* --------------------------------------------------------------------------- reconstruct */
/* src/ozaki2_numerics.cu:445-452: sequential FMA dot. */
double oz2o_fp64_dot(int k, const double* a, int lda, const double* b) {
  double s = 0.0;
  for (int q = 0; q < k; ++q) s = fma(a[(size_t)q * lda], b[q], s);
  return s;
}

static float f32_of_bits(int32_t b) {
  float f;
  memcpy(&f, &b, sizeof f);
  return f;
}

/* src/ozaki2_numerics.cu:454-563, per entry.  Two multiply-adds the reference's device compiler
 * contracts are written as fma(): s2d - Q*P2 and |alpha| lab + |beta C0|. */
void oz2o_reconstruct(int m, int n, int k, int N, const double* A, int lda, const double* B, int ldb,
                      double* C, int ldc, double alpha, double beta, const int32_t* C32,
                      const int32_t* rws, const int32_t* cws, int mode, long long* cnt) {
  const oz2o_tables* t = oz2o_tables_get();
  const size_t cst = (size_t)m * n;
  const double aalpha = fabs(alpha);
  const int64_t P1 = t->P1[N];
  const double P2 = t->P2[N], invPu = t->inv_Pu[N];
  const int lu1 = t->log2_u1[N];
  const double inv_u1 = ldexp(1.0, -lu1);
  const double crt_u = N * 255.0 * ldexp(1.0, -19) + ldexp(1.0, -10);
  const double u = ldexp(1.0, -53);
  const double nt = (double)k + (alpha != 1.0 ? 1.0 : 0.0) + (beta != 0.0 ? 1.0 : 0.0);
  const double gam = (nt * u / (1.0 - nt * u) - 2.0 * u) * (1.0 - ldexp(1.0, -40));
  for (int j = 0; j < n; ++j)
    for (int i = 0; i < m; ++i) {
      const size_t idx = (size_t)i + (size_t)j * m;
      double* cp = C + i + (size_t)j * ldc;
      const double c0 = (beta == 0.0) ? 0.0 : *cp;
      if (alpha == 0.0) {
        *cp = (beta == 0.0) ? 0.0 : beta * c0;
        continue;
      }
      const int rsh = rws[i], csh = cws[j];
      if (rsh == OZ2O_SHIFT_NONFINITE || csh == OZ2O_SHIFT_NONFINITE) {
        const double d = oz2o_fp64_dot(k, A + i, lda, B + (size_t)j * ldb);
        *cp = (beta == 0.0) ? alpha * d : fma(alpha, d, beta * c0);
        cnt[3] += 1;
        continue;
      }
      const int sig = rws[m + i], tau = cws[n + j];
      if (sig == OZ2O_SHIFT_ZERO || tau == OZ2O_SHIFT_ZERO) {
        *cp = (beta == 0.0) ? alpha * 0.0 : fma(alpha, 0.0, beta * c0);
        continue;
      }
      uint64_t S1 = 0;
      uint32_t S2 = 0;
      for (int l = 0; l < N; ++l) {
        const uint32_t p = (uint32_t)t->p[l];
        const int32_t c = C32[(size_t)l * cst + idx];
        const uint32_t uc = c < 0 ? 0u - (uint32_t)c : (uint32_t)c;
        uint32_t r = uc % p;
        if (c < 0 && r) r = p - r;
        const uint32_t y = (r * (uint32_t)t->qinv[N][l]) % p;
        S1 += t->s1[N][l] * (uint64_t)y;
        S2 += t->s2[N][l] * y;
      }
      const double s2d = (double)S2 * (1.0 / (double)(1u << OZ2O_S2_BITS));
      const double Q = rint(((double)S1 + s2d) * invPu);
      const int64_t X1 = (int64_t)S1 - (int64_t)Q * P1;
      const double xr = (double)X1 + fma(-Q, P2, s2d);
      const int esc = lu1 - rsh - csh;
      const double v = mul_pow2(xr, esc);
      const double emu = (beta == 0.0) ? alpha * v : fma(alpha, v, beta * c0);
      if (mode == OZ2O_REPAIR_OFF || (beta != 0.0 && !isfinite(c0))) {
        *cp = emu;
        continue;
      }
      const double da = f32_of_bits(rws[2 * m + i]), na = f32_of_bits(rws[3 * m + i]);
      const double db = f32_of_bits(cws[2 * n + j]), nb = f32_of_bits(cws[3 * n + j]);
      const double et = fma(da, nb, fma(na, db, da * db)) * (1.0 + ldexp(1.0, -40));
      const double Eu = (fma(et, inv_u1, crt_u) + 4.0 * u * fabs(xr)) * (1.0 + ldexp(1.0, -40));
      const double E = mul_pow2(Eu, esc);
      const double L = (double)C32[(size_t)N * cst + idx];
      double lab = mul_pow2(L, -(sig + tau));
      lab = fmax(lab, fabs(v) - E) * (1.0 - ldexp(1.0, -40));
      if (lab < ldexp(1.0, -1000)) lab = 0.0;
      const double lhs = aalpha * E * (1.0 + ldexp(1.0, -40));
      const double rhs = gam * fma(aalpha, lab, fabs(beta * c0)) * (1.0 - ldexp(1.0, -40));
      const int cert = gam > 0.0 && E >= ldexp(1.0, -1000) && isfinite(lhs) && isfinite(v) && lhs <= rhs;
      if (cert) {
        *cp = emu;
      } else if (mode == OZ2O_REPAIR_COUNT) {
        *cp = emu;
        cnt[1] += 1;
      } else {
        const double d = oz2o_fp64_dot(k, A + i, lda, B + (size_t)j * ldb);
        *cp = (beta == 0.0) ? alpha * d : fma(alpha, d, beta * c0);
        cnt[2] += 1;
      }
    }
}

int oz2o_emulate(int m, int n, int k, int N, const double* A, int lda, const double* B, int ldb,
                 double* C, int ldc, double alpha, double beta, int mode, long long* cnt) {
  if (N < 1 || N > OZ2O_MAX_MODULI || m <= 0 || n <= 0) return 1;
  const int kp = kp_of(k);
  const size_t np = (size_t)N + 1;
  int8_t* A8 = (int8_t*)calloc(np * (size_t)m * kp + 1, 1);
  int8_t* B8 = (int8_t*)calloc(np * (size_t)n * kp + 1, 1);
  int32_t* C32 = (int32_t*)calloc(np * (size_t)m * n + 1, sizeof(int32_t));
  int32_t* rws = (int32_t*)calloc(4 * (size_t)m + 1, sizeof(int32_t));
  int32_t* cws = (int32_t*)calloc(4 * (size_t)n + 1, sizeof(int32_t));
  int rc = 0;
  if (!A8 || !B8 || !C32 || !rws || !cws) { rc = 2; goto out; }
  if (alpha != 0.0) {
    oz2o_prep_rows(m, k, N, A, lda, A8, rws, &cnt[0]);
    oz2o_prep_cols(n, k, N, B, ldb, B8, cws, &cnt[0]);
    for (size_t l = 0; l < np; ++l)
      rc |= oz2o_i8_gemm(m, n, kp, A8 + l * (size_t)m * kp, B8 + l * (size_t)n * kp,
                         C32 + l * (size_t)m * n);
  }
  oz2o_reconstruct(m, n, k, N, A, lda, B, ldb, C, ldc, alpha, beta, C32, rws, cws, mode, cnt);
out:
  free(A8); free(B8); free(C32); free(rws); free(cws);
  return rc;
}

/* -------------------------------------------------------------------------------- planner */
/* src/planner.h:27-30 */
int oz2o_route_is_fallback(int r) {
  return r != OZ2O_ROUTE_EMU && r != OZ2O_ROUTE_EMPTY && r != OZ2O_ROUTE_K_ZERO &&
         r != OZ2O_ROUTE_ALPHA_ZERO;
}
static int tile_dim(int cfg) { return cfg == 0 ? 128 : (cfg == 1 ? 64 : 32); }
static double rup(double x, double q) { return ceil(x / q) * q; }
/* src/planner.cpp:153-168 (tile_by_padding, tiles_of) */
static int tile_by_padding(int m, int n) {
  int best = 2;
  double best_eff = -1;
  for (int c = 0; c < 3; ++c) {
    const double td = tile_dim(c);
    const double eff = (double)m * n / (rup(m, td) * rup(n, td));
    if (eff >= 0.75) return c;
    if (eff > best_eff) { best_eff = eff; best = c; }
  }
  return best;
}
static double tiles_of(int m, int n, int cfg) {
  const double td = tile_dim(cfg);
  return ceil(m / td) * ceil(n / td);
}
/* src/planner.cpp:170-202 (constants and cost) */
static void cost(const oz2o_shape* p, int nm, int cfg, const oz2o_device_model* dm, double* t_emu,
                 double* t_nat) {
  static const double eff[3] = {1.0, 0.63, 0.30};
  const double m = p->m, n = p->n, k = p->k, kp = (double)kp_of(p->k), td = tile_dim(cfg);
  const double c_rw = (p->beta != 0.0) ? 2.0 : 1.0;
  const double np = nm + 1;
  const double prep = (2.0 * (m * k + k * n) * 8 + np * (m + n) * kp + 4.0 * 4 * (m + n)) / dm->mem_bw;
  const double slots = (double)dm->num_sms * 2;
  const double per_tile = 2.0 * td * td * kp / (dm->int8_ops * eff[cfg] / slots);
  const double gemm = ceil(np * tiles_of(p->m, p->n, cfg) / slots) * per_tile + np * m * n * 4 / dm->mem_bw;
  const double recon = (np * m * n * 4 + c_rw * m * n * 8) / dm->mem_bw;
  *t_emu = prep + gemm + recon;
  const double nat_c = 2.0 * m * n * k / dm->fp64_flops;
  const double nat_m = (m * k + k * n + c_rw * m * n) * 8 / dm->mem_bw;
  *t_nat = nat_c > nat_m ? nat_c : nat_m;
}
/* src/planner.cpp:204-231 (tune_tiles) */
static int tune_tiles(const oz2o_shape* probs, int num, const oz2o_device_model* dm, oz2o_plan_entry* out) {
  const double slots = (double)dm->num_sms * 2;
  int any = 0;
  for (int pass = 0; pass < 3; ++pass) {
    double W = 0;
    for (int g = 0; g < num; ++g) {
      if (out[g].route != OZ2O_ROUTE_EMU) continue;
      const double td = tile_dim(out[g].tile_cfg);
      W += (out[g].num_moduli + 1) * tiles_of(probs[g].m, probs[g].n, out[g].tile_cfg) * td * td *
           (double)kp_of(probs[g].k);
    }
    if (W <= 0) return any;
    const double per_slot = W / slots;
    int changed = 0;
    for (int g = 0; g < num; ++g) {
      if (out[g].route != OZ2O_ROUTE_EMU || out[g].tile_cfg >= 2) continue;
      const double td = tile_dim(out[g].tile_cfg);
      if (td * td * (double)kp_of(probs[g].k) > per_slot) { out[g].tile_cfg++; changed = 1; }
    }
    if (!changed) return any;
    any = 1;
  }
  return any;
}
/* src/planner.cpp:137-148 (ggemm_plan_num_moduli) */
static int plan_num_moduli(int cfg_nm, double target, int k) {
  int nm;
  if (cfg_nm > 0) {
    nm = cfg_nm;
  } else {
    nm = oz2o_choose_num_moduli(k, target > 0 ? target : 1e-15);
    if (nm < 0) return -1;
  }
  return nm < 2 ? 2 : (nm > OZ2O_MAX_MODULI ? OZ2O_MAX_MODULI : nm);
}
/* src/planner.cpp:236-263 (plan_shape) and 286-330 (ggemm_plan_ex, without the shape memo, which is
   bit-identical) */
int oz2o_plan(const oz2o_shape* probs, int num, int cfg_nm, double target, int allow_fb, int path,
              const oz2o_device_model* dm, double rho, oz2o_plan_entry* out) {
  const int autop = (path == 4);
  for (int g = 0; g < num; ++g) {
    const oz2o_shape* p = &probs[g];
    oz2o_plan_entry* e = &out[g];
    e->route = OZ2O_ROUTE_EMU; e->num_moduli = 0; e->tile_cfg = 0; e->t_emu_s = e->t_native_s = 0;
    if (p->m == 0 || p->n == 0) { e->route = OZ2O_ROUTE_EMPTY; continue; }
    if (p->k == 0) { e->route = OZ2O_ROUTE_K_ZERO; continue; }
    if (p->alpha == 0.0) { e->route = OZ2O_ROUTE_ALPHA_ZERO; continue; }
    if (p->k > OZ2O_MAX_K) {
      if (!allow_fb) return 3;
      e->route = OZ2O_ROUTE_K_TOO_LARGE;
      continue;
    }
    if (autop && allow_fb && p->k <= 16) { e->route = OZ2O_ROUTE_SMALL_K; continue; }
    if (autop && !(cfg_nm > 0)) {
      e->num_moduli = oz2o_choose_num_moduli_cw(p->k, rho);
      if (e->num_moduli >= 0) e->num_moduli = e->num_moduli < 2 ? 2 : (e->num_moduli > 20 ? 20 : e->num_moduli);
    } else {
      e->num_moduli = plan_num_moduli(cfg_nm, target, p->k);
    }
    if (e->num_moduli < 0) {
      if (!allow_fb) return 3;
      e->route = OZ2O_ROUTE_PRECISION; e->num_moduli = 0;
      continue;
    }
    if (!autop) continue;
    e->tile_cfg = tile_by_padding(p->m, p->n);
    cost(p, e->num_moduli, e->tile_cfg, dm, &e->t_emu_s, &e->t_native_s);
    if (allow_fb) {
      if ((double)p->m * p->n * p->k < dm->tiny_mnk) e->route = OZ2O_ROUTE_TINY;
      else if (e->t_emu_s > e->t_native_s) e->route = OZ2O_ROUTE_UNPROFITABLE;
    }
  }
  if (autop && tune_tiles(probs, num, dm, out)) {
    for (int g = 0; g < num; ++g) {
      oz2o_plan_entry* e = &out[g];
      if (e->route != OZ2O_ROUTE_EMU) continue;
      cost(&probs[g], e->num_moduli, e->tile_cfg, dm, &e->t_emu_s, &e->t_native_s);
      if (allow_fb && e->t_emu_s > e->t_native_s) e->route = OZ2O_ROUTE_UNPROFITABLE;
    }
  }
  return 0;
}
