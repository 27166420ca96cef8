/* ggemm.h -- grouped FP64 GEMM on MI355X (gfx950), FP64 emulated on INT8 MFMA with the
 * Ozaki scheme II (CRT).  Column-major, no transpose:
 *     C_g = alpha_g * A_g (m_g x k_g) * B_g (k_g x n_g) + beta_g * C_g      for g = 0..G-1.
 *
 * Drop-in C ABI for the reference's include/ggemm.h:1-90.  Every type, field, enum value and
 * function below keeps the reference's name, order and meaning; the only change is the stream
 * type (hipStream_t, pointer-sized like cudaStream_t).  The GGEMM_ERR_* return codes, private in
 * the reference (src/internal.h:65-75), are part of this ABI with the same values.
 */
#ifndef GGEMM_H
#define GGEMM_H
#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* include/ggemm.h:12-18 */
typedef struct {
  int m, n, k;
  const double* A; int lda;   /* device pointers */
  const double* B; int ldb;
  double*       C; int ldc;
  double alpha, beta;
} ggemm_problem_t;

/* include/ggemm.h:20-31 */
typedef enum {
  GGEMM_PATH_NATIVE_LOOP = 0,        /* native FP64 (own FP64-MFMA DGEMM), one launch per problem */
  GGEMM_PATH_NATIVE_GROUPED = 1,     /* native FP64, one grouped launch */
  GGEMM_PATH_EMU_LOOP = 2,           /* per problem: prep, one INT8 GEMM per plane, reconstruct */
  GGEMM_PATH_EMU_GROUPED = 3,        /* fused grouped pipeline: 6 launches for the whole group
                                        (prep, INT8 GEMM, reconstruct, FP64 dot-product pass, the
                                        pass's row gather and crossings GEMM) */
  GGEMM_PATH_AUTO = 4,               /* EMU_GROUPED + planner (adaptive N, cost-based fallback) */
  GGEMM_PATH_EMU_GROUPED_REUSE = 5,  /* EMU_GROUPED + operand reuse */
  GGEMM_PATH_EMU_LOOP_BATCHED = 6    /* per problem: prep, one INT8 GEMM over its planes, reconstruct */
} ggemm_path_t;

/* include/ggemm.h:33-38 (field order is ABI: callers use positional initialisers) */
typedef struct {
  int num_moduli;         /* 0 = adaptive per problem; else fixed N in [2, GGEMM_MAX_MODULI] */
  double target_rel_err;  /* adaptive target (normwise), default 1e-15 */
  int allow_fallback;     /* 1 = route unsafe / unprofitable problems to native FP64 */
  int repair_mode;        /* GGEMM_REPAIR_*; 0 = path default */
} ggemm_config_t;

#define GGEMM_MAX_MODULI 20

/* include/ggemm.h:43-46 */
#define GGEMM_REPAIR_DEFAULT 0   /* EMU_* paths: COUNT; AUTO: ON */
#define GGEMM_REPAIR_OFF     1   /* no certificate */
#define GGEMM_REPAIR_COUNT   2   /* certificate evaluated, failures counted, emulated value kept */
#define GGEMM_REPAIR_ON      3   /* failures recomputed as FP64 dot products */

/* include/ggemm.h:48-65 */
typedef struct {
  int num_problems;
  int num_fallback;        /* problems routed to native FP64 */
  int kernel_launches;     /* launches issued by the last call */
  int moduli_min, moduli_max;
  int reuse_enabled;
  int num_unique_A;
  int num_unique_B;
  int num_promoted;
  /* Process-wide device counters, reset before / read after each call; -1 unless the environment
   * variable GGEMM_STATS_REPAIR=1 (reading them synchronises the stream).  Not per handle. */
  long long num_repaired;         /* entries recomputed in FP64 by the certificate (repair ON) */
  long long num_uncertified;      /* repair COUNT: entries failing the certificate */
  long long num_safety_fallback;  /* entries computed in FP64 because of NaN/Inf input */
} ggemm_stats_t;

/* src/internal.h:65-75 (values unchanged) */
enum {
  GGEMM_OK = 0,
  GGEMM_ERR_INVALID = 1,    /* bad args / null handle / num_problems > max_problems */
  GGEMM_ERR_WORKSPACE = 2,  /* call exceeds the workspace sized at create */
  GGEMM_ERR_UNSAFE = 3,     /* k > GGEMM_MAX_K_EXACT (or target unreachable) and allow_fallback == 0 */
  GGEMM_ERR_CUDA = 4,       /* HIP runtime error (name kept for ABI compatibility) */
  GGEMM_ERR_CUBLAS = 5,     /* native FP64 GEMM launch error (name kept for ABI compatibility) */
  GGEMM_ERR_NUMERICS = 6,   /* prep / reconstruct launch error */
  GGEMM_ERR_I8GEMM = 7,     /* INT8 GEMM schedule / launch error */
  GGEMM_ERR_ALLOC = 8       /* only from ggemm_create */
};

/* INT8 x INT8 -> INT32 exactness: 128*128*kp < 2^31  =>  kp = round_up(k, 32) <= 131040. */
#define GGEMM_MAX_K_EXACT 131040

typedef struct ggemm_handle_s* ggemm_handle_t;

/* include/ggemm.h:71-72.  All workspace is allocated here (never inside calls). */
int ggemm_create(ggemm_handle_t* h, int max_problems, size_t max_total_A_elems,
                 size_t max_total_B_elems, size_t max_total_C_elems, hipStream_t stream);
/* include/ggemm.h:78-80.  min_k = smallest k of any emulated problem the handle will see
 * (ggemm_create uses 32); residues are stored with Kp = round_up(k, 32). */
int ggemm_create_ex(ggemm_handle_t* h, int max_problems, size_t max_total_A_elems,
                    size_t max_total_B_elems, size_t max_total_C_elems, hipStream_t stream,
                    int min_k);
/* include/ggemm.h:81 */
void ggemm_destroy(ggemm_handle_t h);

/* include/ggemm.h:85-86.  problems: HOST array of descriptors (pointers inside are device
 * pointers).  Returns GGEMM_OK or a GGEMM_ERR_* code; never allocates. */
int ggemm_grouped_dgemm(ggemm_handle_t h, ggemm_path_t path, const ggemm_config_t* cfg,
                        const ggemm_problem_t* problems, int num_problems, ggemm_stats_t* stats);

/* No counterpart in the reference.  ggemm_grouped_dgemm without a handle and without allocating
 * anything (device or host memory), for callers that cannot allocate (tight serving loops, harnesses
 * that forbid hipMalloc).  Same kernels, layouts and results (bit for bit) as a call
 * through a handle created with ggemm_create(GGEMM_NOALLOC_MAX_PROBLEMS, GGEMM_NOALLOC_MAX_ELEMS x 3):
 * the workspace is a static device array of GGEMM_NOALLOC_SCRATCH_BYTES that each GPU the library
 * runs on holds until the process ends.  Paths GGEMM_PATH_EMU_GROUPED and GGEMM_PATH_AUTO only
 * (others: GGEMM_ERR_INVALID).  Limits: at most GGEMM_NOALLOC_MAX_PROBLEMS problems
 * (GGEMM_ERR_INVALID) and sum m*k, sum k*n, sum m*n each at most GGEMM_NOALLOC_MAX_ELEMS, residues
 * counted at Kp = round_up(k, 32) (GGEMM_ERR_WORKSPACE); either error prints one line on stderr.
 * Work runs on `stream`; the call synchronises the stream (it returns after its descriptor copy has
 * landed, i.e. after earlier work on the stream), so it cannot be captured: on a stream that is being
 * captured it returns GGEMM_ERR_INVALID (one stderr line) and leaves the capture intact; capture
 * ggemm_execute_plan instead.  Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * from different streams race.  Device counters and GGEMM_STATS_REPAIR as for ggemm_grouped_dgemm. */
#define GGEMM_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
#define GGEMM_NOALLOC_MAX_PROBLEMS 64
#define GGEMM_NOALLOC_MAX_ELEMS ((size_t)262144)
int ggemm_grouped_dgemm_noalloc(ggemm_path_t path, const ggemm_config_t* cfg,
                                const ggemm_problem_t* problems, int num_problems, hipStream_t stream,
                                ggemm_stats_t* stats);

#ifdef __cplusplus
}
static_assert(sizeof(ggemm_problem_t) == 80, "ggemm_problem_t layout");
static_assert(sizeof(ggemm_config_t) == 24, "ggemm_config_t layout");
static_assert(sizeof(ggemm_stats_t) == 64, "ggemm_stats_t layout");
#endif
#endif
