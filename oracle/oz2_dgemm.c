/* oz2_dgemm.c -- the CPU FP64 baseline GEMM timed beside the GPU path (TEST INFRASTRUCTURE).
 *
 * C = alpha*A*B + beta*C, column-major, no transpose (the ggemm_problem_t convention).  Blocked
 * over (column block, row block, k block) with an OpenMP loop over column blocks; the inner
 * kernel is a plain multiply-add loop the compiler vectorises (AVX2 + FMA).  beta == 0 does not
 * read C.  It is a reported baseline, not a tuned BLAS.
 */
#include <string.h>

#include "oz2_oracle.h"

void oz2o_dgemm(int m, int n, int k, double alpha, const double* A, int lda, const double* B,
                int ldb, double beta, double* C, int ldc) {
  enum { MB = 64, NB = 32, KB = 256 };
  const int nblk = (n + NB - 1) / NB;
#pragma omp parallel for schedule(dynamic, 1)
  for (int jb = 0; jb < nblk; ++jb) {
    const int j0 = jb * NB, j1 = j0 + NB < n ? j0 + NB : n;
    double acc[NB][MB];
    for (int i0 = 0; i0 < m; i0 += MB) {
      const int i1 = i0 + MB < m ? i0 + MB : m, mi = i1 - i0;
      memset(acc, 0, sizeof acc);
      for (int q0 = 0; q0 < k; q0 += KB) {
        const int q1 = q0 + KB < k ? q0 + KB : k;
        for (int j = j0; j < j1; ++j) {
          double* c = acc[j - j0];
          for (int q = q0; q < q1; ++q) {
            const double b = B[q + (size_t)j * ldb];
            const double* a = A + i0 + (size_t)q * lda;
            for (int i = 0; i < mi; ++i) c[i] += a[i] * b;
          }
        }
      }
      for (int j = j0; j < j1; ++j)
        for (int i = 0; i < mi; ++i) {
          double* cp = C + (i0 + i) + (size_t)j * ldc;
          const double ab = alpha * acc[j - j0][i];
          *cp = (beta == 0.0) ? ab : ab + beta * *cp;
        }
    }
  }
}
