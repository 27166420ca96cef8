// katgen.cpp -- regenerates the input data of the reference's numerics test and provides a
// long-double reference GEMM for error gates (TEST INFRASTRUCTURE ONLY; built into
// tests/golden/libkatgen.so by tests/golden/build_katgen.py).
//
// The reference test (tests/test_numerics_standalone.cu:57-76) draws every matrix entry from one
// process-wide std::mt19937_64 seeded 12345:  entry = (U(0,1) - 0.5) * exp(phi * Z),  with a
// fresh std::uniform_real_distribution<double>(0,1) and std::normal_distribution<double>(0,1)
// per entry, A filled column by column (m rows of each of the k columns, lda = m + pad), then B
// (k rows of n columns, ldb = k + 3), then C0 (m rows of n columns, ldc = m + 1) with phi = 0.
// Replaying the same calls in the same order through libstdc++ gives the same doubles, which the
// logged "naive FP64 dot rel_cw" values (log lines 23-327) confirm case by case.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <random>
#include <vector>

namespace {
std::mt19937_64 g_rng(12345);
int g_order = 0;  // 0: U drawn before Z, 1: Z drawn before U

double draw(double phi) {
  std::uniform_real_distribution<double> U(0.0, 1.0);
  std::normal_distribution<double> Z(0.0, 1.0);
  if (g_order == 0) {
    const double u = U(g_rng);
    const double z = Z(g_rng);
    return (u - 0.5) * std::exp(phi * z);
  }
  const double z = Z(g_rng);
  const double u = U(g_rng);
  return (u - 0.5) * std::exp(phi * z);
}
}  // namespace

extern "C" {

void katgen_seed(unsigned long long seed, int order) {
  g_rng.seed(seed);
  g_order = order;
}

// A: (m + lda_pad) x k, B: (k + 3) x n, C0: (m + 1) x n, all column-major, caller-allocated
// and zero-initialised (padding rows are never written).
void katgen_make(int m, int n, int k, int lda_pad, double phi, double* A, double* B, double* C0) {
  const size_t lda = (size_t)m + lda_pad, ldb = (size_t)k + 3, ldc = (size_t)m + 1;
  for (int c = 0; c < k; ++c)
    for (int r = 0; r < m; ++r) A[r + c * lda] = draw(phi);
  for (int c = 0; c < n; ++c)
    for (int r = 0; r < k; ++r) B[r + c * ldb] = draw(phi);
  for (int c = 0; c < n; ++c)
    for (int r = 0; r < m; ++r) C0[r + c * ldc] = draw(0.0);
}

// Long-double Neumaier reference R = alpha*A*B + beta*C0 (m x n, ld m), plus
// absAB = (|A||B|)_ij and nrm = ||A(i,:)|| ||B(:,j)|| (as double).
void katgen_reference(int m, int n, int k, const double* A, int lda, const double* B, int ldb,
                      const double* C0, int ldc, double alpha, double beta, long double* R,
                      double* absAB, double* nrm) {
  std::vector<long double> ra(m, 0.0L), cb(n, 0.0L);
  for (int i = 0; i < m; ++i)
    for (int q = 0; q < k; ++q) { long double a = A[i + (size_t)q * lda]; ra[i] += a * a; }
  for (int j = 0; j < n; ++j)
    for (int q = 0; q < k; ++q) { long double b = B[q + (size_t)j * ldb]; cb[j] += b * b; }
  for (int j = 0; j < n; ++j)
    for (int i = 0; i < m; ++i) {
      long double s = 0.0L, comp = 0.0L, sa = 0.0L;
      for (int q = 0; q < k; ++q) {
        long double t = (long double)A[i + (size_t)q * lda] * (long double)B[q + (size_t)j * ldb];
        long double u = s + t;
        comp += (fabsl(s) >= fabsl(t)) ? (s - u) + t : (t - u) + s;
        s = u;
        sa += fabsl(t);
      }
      s += comp;
      const long double c0 = beta == 0.0 ? 0.0L : (long double)C0[i + (size_t)j * ldc];
      R[i + (size_t)j * m] = (long double)alpha * s + (long double)beta * c0;
      absAB[i + (size_t)j * m] = (double)sa;
      nrm[i + (size_t)j * m] = (double)sqrtl(ra[i] * cb[j]);
    }
}

// Same reference, returned as double hi + double lo (R ~= hi + lo) for callers without
// long double (numpy on some platforms).
void katgen_reference_dd(int m, int n, int k, const double* A, int lda, const double* B, int ldb,
                         const double* C0, int ldc, double alpha, double beta, double* hi,
                         double* lo, double* absAB, double* nrm) {
  std::vector<long double> R((size_t)m * n);
  katgen_reference(m, n, k, A, lda, B, ldb, C0, ldc, alpha, beta, R.data(), absAB, nrm);
  for (size_t q = 0; q < R.size(); ++q) {
    hi[q] = (double)R[q];
    lo[q] = (double)(R[q] - (long double)hi[q]);
  }
}

// max_ij |naive_dot - R| / |R| with the naive loop s += a*b in double (no FMA), alpha=1, beta=0:
// the "naive FP64 dot rel_cw" figure the reference test prints for each sweep shape.
double katgen_naive_relcw(int m, int n, int k, const double* A, int lda, const double* B, int ldb,
                          const long double* R) {
  double worst = 0;
  for (int j = 0; j < n; ++j)
    for (int i = 0; i < m; ++i) {
      volatile double s = 0;
      for (int q = 0; q < k; ++q) {
        volatile double p = A[i + (size_t)q * lda] * B[q + (size_t)j * ldb];
        s = s + p;
      }
      long double r = R[i + (size_t)j * m];
      if (r != 0) {
        double e = (double)(fabsl((long double)s - r) / fabsl(r));
        if (e > worst) worst = e;
      }
    }
  return worst;
}

// Componentwise gate of tests/test_numerics_standalone.cu:180-206:
//   gate = max |C - R| / (gamma_n (|alpha| absAB + |beta C0|)),  n = k + [alpha != 1] + [beta != 0].
// Returns the gate value; *over counts entries with err > gamma_n den (non-finite C included).
double katgen_gate(int m, int n, int k, double alpha, double beta, const double* C, int ldc,
                   const double* C0, int ldc0, const long double* R, const double* absAB,
                   long long* over) {
  double nn = (double)k + (alpha != 1.0) + (beta != 0.0);
  if (nn < 1) nn = 1;
  const double u = std::ldexp(1.0, -53);
  const double gam = nn * u / (1.0 - nn * u);
  double gate = 0;
  long long cnt = 0;
  for (int j = 0; j < n; ++j)
    for (int i = 0; i < m; ++i) {
      const double c = C[i + (size_t)j * ldc];
      const long double r = R[i + (size_t)j * m];
      const long double err = fabsl((long double)c - r);
      const double sa = std::fabs(alpha) * absAB[i + (size_t)j * m];
      const double c0 = beta == 0.0 ? 0.0 : C0[i + (size_t)j * ldc0];
      const long double den = gam * ((long double)sa + fabsl((long double)beta * c0));
      double g;
      if (!std::isfinite(c)) g = INFINITY;
      else if (den > 0) g = (double)(err / den);
      else g = err > 0 ? INFINITY : 0.0;
      if (!(g <= 1.0)) ++cnt;
      if (!(g <= gate)) gate = g;
    }
  if (over) *over = cnt;
  return gate;
}

// The four error columns the reference test prints per problem (tests/test_numerics_standalone.cu:
// 180-206, check()): out[0] rel_cw = max |C - R| / |R| (R != 0), out[1] rel_abs and out[2] rel_nrm =
// max err_ab / (|alpha| absAB) and / (|alpha| nrm) with err_ab = max(0, |C - R| - 4u(|beta C0| + |R|)),
// out[3] gate = max |C - R| / (gamma_n (|alpha| absAB + |beta C0|)).  Running maxima use std::max,
// so a NaN candidate never replaces the maximum.  Returns 1 when the padding rows i in [m, ldc) of
// C equal those of C0 (the test's beta_ok), else 0.
int katgen_check(int m, int n, int k, double alpha, double beta, const double* C, const double* C0, int ldc,
                 const long double* R, const double* absAB, const double* nrm, double* out) {
  double nn = (double)k + (alpha != 1.0) + (beta != 0.0);
  if (nn < 1) nn = 1;
  const double u = std::ldexp(1.0, -53);
  const double gam = nn * u / (1.0 - nn * u);
  double cw = 0, ab = 0, nr = 0, gate = 0;
  int beta_ok = 1;
  for (int j = 0; j < n; ++j) {
    for (int i = 0; i < m; ++i) {
      const long double r = R[i + (size_t)j * m];
      const double c = C[i + (size_t)j * ldc];
      const double c0 = C0[i + (size_t)j * ldc];
      const long double err = fabsl((long double)c - r);
      const long double slack = 4.0L * ldexpl(1.0L, -53) * (fabsl((long double)beta * c0) + fabsl(r));
      const long double err_ab = err > slack ? err - slack : 0.0L;
      if (r != 0) cw = std::max(cw, (double)(err / fabsl(r)));
      const double sa = std::fabs(alpha) * absAB[i + (size_t)j * m];
      const double sn = std::fabs(alpha) * nrm[i + (size_t)j * m];
      if (sa > 0) ab = std::max(ab, (double)(err_ab / sa));
      if (sn > 0) nr = std::max(nr, (double)(err_ab / sn));
      else if (err_ab > 0) nr = INFINITY;
      const long double den = gam * ((long double)sa + fabsl((long double)beta * c0));
      if (den > 0) gate = std::max(gate, (double)(err / den));
      else if (err > 0) gate = INFINITY;
    }
    for (int i = m; i < ldc; ++i)
      if (C[i + (size_t)j * ldc] != C0[i + (size_t)j * ldc]) beta_ok = 0;
  }
  out[0] = cw;
  out[1] = ab;
  out[2] = nr;
  out[3] = gate;
  return beta_ok;
}

}  // extern "C"
