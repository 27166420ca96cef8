/* oz2_oracle.h -- CPU oracle for the grouped Ozaki-II (CRT) FP64 GEMM hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference algorithm
 * (moneychen168/Coding-Basic-HW-2) used as the parity checker by tests/, by
 * __graft_entry__.smoke() and by the cpu_baseline leg of bench.py.  No product code links,
 * loads or calls it; the product path fails loudly when its HIP library is missing.
 *
 * Every function cites the reference file:line it follows.  Pinning (see tests/test_oracle.py):
 *   - CRT tables / error bound / choose N: the log2P, bound(k=1024) and choose(1e-15) KATs of
 *     results/final_590258/logs/test_numerics_standalone.log:3-17, plus exact big-integer
 *     identities (CRT inverse, M_l reconstruction, pairwise coprimality) re-derived in Python.
 *   - prep (shifts, residues, abs plane, norm bounds): the exact residue identity of
 *     tests/test_numerics_standalone.cu:210-258 (fmodl of truncl(ldexpl(a, s))), the
 *     ||A'_i|| <= T_N budget, maximality of s_i, and the per-(shape, phi, N) repair counts of
 *     the log (lines 23-340) which depend on every shift and norm bound.
 *   - int GEMM: brute-force int64 dot, plus the closed form all -128 at kp = 131040.
 *   - reconstruct / certificate: the repair-count KATs above, 899 uncertified == repaired
 *     (log:357), 6688 grouped repairs (log:343), non-finite counter 2 (log:355), and the
 *     componentwise gamma_n gate against a long-double Neumaier reference.
 *   - planner: the route table of tests/test_planner.cpp:127-186 with
 *     tests/testdata/planner/valid.json.
 */
#ifndef OZ2_ORACLE_H
#define OZ2_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OZ2O_MAX_MODULI 20
#define OZ2O_POW2_TABLE 128
#define OZ2O_S2_BITS 18
#define OZ2O_MAX_K 131040
#define OZ2O_SHIFT_NONFINITE (-2147483647 - 1)
#define OZ2O_SHIFT_ZERO (-2147483647)
#define OZ2O_REPAIR_OFF 0
#define OZ2O_REPAIR_COUNT 1
#define OZ2O_REPAIR_ON 2

/* Same quantities as src/moduli.h:43-58 (index N = 1..20 for the per-N rows). */
typedef struct {
  int32_t p[OZ2O_MAX_MODULI];
  uint32_t magic[OZ2O_MAX_MODULI];
  uint8_t pow2[OZ2O_MAX_MODULI][OZ2O_POW2_TABLE];
  uint64_t s1[OZ2O_MAX_MODULI + 1][OZ2O_MAX_MODULI];
  uint32_t s2[OZ2O_MAX_MODULI + 1][OZ2O_MAX_MODULI];
  int32_t qinv[OZ2O_MAX_MODULI + 1][OZ2O_MAX_MODULI];
  int64_t P1[OZ2O_MAX_MODULI + 1];
  double P2[OZ2O_MAX_MODULI + 1];
  double inv_Pu[OZ2O_MAX_MODULI + 1];
  int32_t log2_u1[OZ2O_MAX_MODULI + 1];
  double T[OZ2O_MAX_MODULI + 1];
  double log2P[OZ2O_MAX_MODULI + 1];
} oz2o_tables;

int oz2o_build_tables(oz2o_tables* t);            /* 0 on success */
const oz2o_tables* oz2o_tables_get(void);         /* built once */

double oz2o_error_bound(int k, int N);
int oz2o_choose_num_moduli(int k, double target_rel_err);
int oz2o_choose_num_moduli_cw(int k, double rho_budget);

/* Prep of one operand of one problem (alpha != 0).  Output planes are row-major
 * [plane][vec][kp] with plane stride vecs*kp bytes (planes 0..N-1 residues, plane N abs plane);
 * ws is [4][vecs] int32 {shift, abs shift, ||dA|| float bits, ||A'|| float bits}.
 * rows: A is m x k column-major (lda); one vector per row.   cols: B is k x n column-major (ldb). */
void oz2o_prep_rows(int m, int k, int N, const double* A, int lda, int8_t* A8, int32_t* ws,
                    long long* nonfinite);
void oz2o_prep_cols(int n, int k, int N, const double* B, int ldb, int8_t* B8, int32_t* ws,
                    long long* nonfinite);

/* C32 (m x n column-major, ld m) = A8 (m x kp row-major) * B8 (n x kp row-major)^T, exact.
 * Returns 0, or 1 if an entry does not fit int32. */
int oz2o_i8_gemm(int m, int n, int kp, const int8_t* A8, const int8_t* B8, int32_t* C32);
/* Exact int8 dot products (oz2_i8dot.c): one of length n, and one row against four rows. */
int64_t oz2o_dot_i8(const int8_t* a, const int8_t* b, int n);
void oz2o_dot4_i8(const int8_t* a, const int8_t* b0, const int8_t* b1, const int8_t* b2, const int8_t* b3, int n,
                  int64_t* out);

/* Reconstruct one problem from its N+1 int32 planes (plane stride m*n).  cnt[0..3] +=
 * {unused, uncertified, repaired, safety_fallback}. */
void oz2o_reconstruct(int m, int n, int k, int N, const double* A, int lda, const double* B, int ldb,
                      double* C, int ldc, double alpha, double beta, const int32_t* C32,
                      const int32_t* rws, const int32_t* cws, int mode, long long* cnt);

/* Full emulation of one problem (prep -> int GEMM -> reconstruct); scratch is allocated here.
 * cnt[0..3] += {nonfinite vectors, uncertified, repaired, safety}.  Returns 0 on success. */
int oz2o_emulate(int m, int n, int k, int N, const double* A, int lda, const double* B, int ldb,
                 double* C, int ldc, double alpha, double beta, int mode, long long* cnt);

double oz2o_fp64_dot(int k, const double* a, int lda, const double* b);

/* Blocked FP64 GEMM C = alpha*A*B + beta*C (column-major), OpenMP over (problem tile) when built
 * with -fopenmp: the timed CPU baseline. */
void oz2o_dgemm(int m, int n, int k, double alpha, const double* A, int lda, const double* B, int ldb,
                double beta, double* C, int ldc);

/* ---- planner (src/planner.h:7-37, src/planner.cpp) ---- */
enum {
  OZ2O_ROUTE_EMU = 0, OZ2O_ROUTE_EMPTY = 1, OZ2O_ROUTE_K_ZERO = 2, OZ2O_ROUTE_K_TOO_LARGE = 3,
  OZ2O_ROUTE_TINY = 4, OZ2O_ROUTE_UNPROFITABLE = 5, OZ2O_ROUTE_PRECISION = 6,
  OZ2O_ROUTE_SMALL_K = 7, OZ2O_ROUTE_ALPHA_ZERO = 8
};
typedef struct { int num_sms; double fp64_flops, int8_ops, mem_bw, tiny_mnk; } oz2o_device_model;
typedef struct { int route, num_moduli, tile_cfg; double t_emu_s, t_native_s; } oz2o_plan_entry;
typedef struct { int m, n, k; double alpha, beta; } oz2o_shape;

/* path: 2 EMU_LOOP, 3 EMU_GROUPED, 4 AUTO.  Returns 0 or 3 (GGEMM_ERR_UNSAFE). */
int oz2o_plan(const oz2o_shape* probs, int num, int cfg_num_moduli, double cfg_target,
              int allow_fallback, int path, const oz2o_device_model* dm, double rho_budget,
              oz2o_plan_entry* out);
int oz2o_route_is_fallback(int route);

#ifdef __cplusplus
}
#endif
#endif
