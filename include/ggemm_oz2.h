/* ggemm_oz2.h -- kernel-level ("whitebox") C ABI of the MI355X Ozaki-II pipeline.
 *
 * These are the reference's internal module interfaces, kept with the same names, fields and
 * semantics so that its kernel-level tests can be expressed against the new kernels:
 *   numerics  : src/ozaki2_numerics.h:23-105 (prep / reconstruct / counters / bounds)
 *   INT8 GEMM : src/int8_grouped_gemm.h:16-94 (grouped int8 x int8 -> int32)
 *   planner   : src/planner.h:7-79 (routes, N, tile config, device model)
 * Device pointers are plain pointers; streams are hipStream_t.  Layouts (per (plane, problem)):
 *   A residues : row-major m x kp (K contiguous), plane l at A8 + l * a8_mod_stride
 *   B residues : row-major n x kp (= column-major kp x n), plane l at B8 + l * b8_mod_stride
 *   C32        : column-major m x n, ld = m, plane l at C32 + l * c32_mod_stride (int32 units)
 *   kp = round_up(k, 32); columns k..kp-1 of A8/B8 are written as 0 by prep.
 * A problem with N moduli uses N + 1 planes: 0..N-1 CRT residues, N the "abs plane"
 * floor(2^sigma |A|) in [0, 127] whose product bounds (|A||B|)_ij from below.
 */
#ifndef GGEMM_OZ2_H
#define GGEMM_OZ2_H
#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>
#include "ggemm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ numerics module */
/* src/ozaki2_numerics.h:23-30 */
typedef struct {
  int m, n, k, kp, num_moduli, lda, ldb, ldc;
  const double *A, *B; double* C; double alpha, beta;
  int8_t *A8, *B8;
  size_t a8_mod_stride, b8_mod_stride;   /* bytes */
  int32_t* C32; size_t c32_mod_stride;   /* int32 elements */
  int32_t *row_shift, *col_shift;        /* 4*m and 4*n int32 */
} oz2_problem;

#define OZ2_EXTRA_PLANES 1
#define OZ2_ROW_WS_PER_ROW 4          /* {shift, abs shift, ||dA|| float bits, ||A'|| float bits} */
#define OZ2_MAX_K 131040
#define OZ2_SHIFT_NONFINITE (-2147483647 - 1)
#define OZ2_SHIFT_ZERO (-2147483647)
#define OZ2_REPAIR_OFF 0
#define OZ2_REPAIR_COUNT 1
#define OZ2_REPAIR_ON 2

/* src/ozaki2_numerics.h:39.  Uploads the CRT tables to the current device (idempotent). */
int oz2_init_constants(void);
/* src/ozaki2_numerics.h:44.  d: DEVICE array of num descriptors.  One kernel launch. */
int oz2_prep_grouped(const oz2_problem* d, int num, int max_m, int max_n, hipStream_t s);
/* src/ozaki2_numerics.h:63-64.  One kernel launch; repair_mode OZ2_REPAIR_*. */
int oz2_reconstruct_grouped(const oz2_problem* d, int num, int max_m, int max_n, hipStream_t s,
                            int repair_mode);
/* src/ozaki2_numerics.h:76, :80, :87 (host) */
int oz2_choose_num_moduli(int k, double target_rel_err);
double oz2_error_bound(int k, int num_moduli);
int oz2_choose_num_moduli_cw(int k, double rho_budget);

/* src/ozaki2_numerics.h:90-98: sticky process-wide device counters of the current device. */
typedef struct {
  unsigned long long nonfinite_vectors;  /* A rows / B columns containing NaN/Inf (prep) */
  unsigned long long uncertified;        /* COUNT mode: entries failing the certificate */
  unsigned long long repaired;           /* ON mode: entries recomputed in FP64 */
  unsigned long long safety_fallback;    /* entries computed in FP64 because of NaN/Inf input */
} oz2_counters;
/* out may be NULL (reset only).  Enqueued on s; with out != NULL the call synchronises s. */
int oz2_read_counters(oz2_counters* out, int reset, hipStream_t s);
/* src/ozaki2_numerics.h:105: force the prep K-split factor (1..64, 0 = automatic). */
void oz2_debug_force_prep_split(int S);
/* No counterpart in the reference: the FP64 matrix-core chains the dot pass's crossings rely on, for
   the tests.  Wave w (64 lanes, one workgroup each) runs steps t = 0 .. steps - 1 of
   v_mfma_f64_16x16x4f64 from a zero accumulator on A[(w steps + t) 64 + l], B[(w steps + t) 64 + l]
   (lane l holds row / column l % 16 at k = 4 t + l / 16) and stores element e of lane l at
   D[256 w + 4 l + e] (output row l / 16 + 4 e, column l % 16).  Device pointers; one launch,
   synchronous.  Returns 0, or 1 for waves < 1 or steps < 1, 3 for a launch error. */
int oz2_mfma_f64_chains(const double* A, const double* B, double* D, int waves, int steps, hipStream_t s);

/* ------------------------------------------------------------------ INT8 grouped GEMM */
/* src/int8_grouped_gemm.h:16-23.  C = A * B^T: C[i + j*m] = sum_k A[i*kp + k] * B[j*kp + k]. */
typedef struct {
  int m, n, kp;
  const int8_t* A;
  const int8_t* B;
  int32_t* C;
  int tile_cfg;   /* 0 = large, 1 = medium, 2 = small tiles; < 0 = automatic */
} i8_problem;

/* src/int8_grouped_gemm.h:57-63 */
typedef struct {
  int tiles_main;
  int tiles_splitk;
  int num_launches;
  int ws2_offset_ints;
  size_t bytes_used;     /* bytes of the schedule image to copy H2D */
} i8_sched_info;

/* src/int8_grouped_gemm.h:40 */
size_t i8_grouped_gemm_sched_ws_bytes(int max_problems, size_t max_tiles);
/* src/int8_grouped_gemm.h:78-79: host schedule image into h_ws (>= sched_ws_bytes(num, 0)). */
int i8_grouped_gemm_build_schedule(const i8_problem* h_probs, int num, void* h_ws,
                                   size_t ws_bytes, i8_sched_info* info);
/* src/int8_grouped_gemm.h:82-83: launch only (info->num_launches kernels). */
int i8_grouped_gemm_launch(const i8_problem* d_probs, int num, const void* d_sched_ws,
                           const i8_sched_info* info, hipStream_t s);
/* src/int8_grouped_gemm.h:46: sizes the schedule builder's host scratch for max_problems
 * (problem, plane) products, so that building a schedule of at most that many allocates nothing
 * (ggemm_create_ex reserves max_problems x 21).  Larger calls still work and grow it. */
void i8_grouped_gemm_reserve(int max_problems, size_t max_tiles);
/* src/int8_grouped_gemm.h:48: growths of that host scratch so far (constant after a reserve). */
long long i8_grouped_gemm_host_allocs(void);
/* src/int8_grouped_gemm.h:72-73: build schedule + H2D + launch. */
int i8_grouped_gemm_ex(const i8_problem* d_probs, int num, const i8_problem* h_probs_for_sched,
                       void* d_sched_ws, size_t sched_ws_bytes, hipStream_t s, int* num_launches);

/* ------------------------------------------------------------------ planner */
/* src/planner.h:7-17 */
typedef enum {
  GGEMM_ROUTE_EMU = 0,
  GGEMM_ROUTE_EMPTY = 1,
  GGEMM_ROUTE_K_ZERO = 2,
  GGEMM_ROUTE_K_TOO_LARGE = 3,
  GGEMM_ROUTE_TINY = 4,
  GGEMM_ROUTE_UNPROFITABLE = 5,
  GGEMM_ROUTE_PRECISION = 6,
  GGEMM_ROUTE_SMALL_K = 7,
  GGEMM_ROUTE_ALPHA_ZERO = 8
} ggemm_route_t;
#define GGEMM_AUTO_NATIVE_MAX_K 16
#define GGEMM_RHO_BUDGET_DEFAULT 16.0

/* src/planner.h:32-37 */
typedef struct {
  int route;
  int num_moduli;
  int tile_cfg;
  double t_emu_s, t_native_s;
} ggemm_plan_entry_t;

/* src/planner.h:43-49 */
typedef struct {
  int num_sms;
  double fp64_flops;
  double int8_ops;
  double mem_bw;
  double tiny_mnk;
} ggemm_device_model_t;

/* src/planner.h:55-56.  gpu_name: the device's architecture name (gcnArchName, e.g.
 * "gfx950:sramecc+:xnack-") or marketing name; MI355X nominal values are keyed on "gfx950". */
void ggemm_device_model_init(ggemm_device_model_t* dm, const char* gpu_name, int cc_major,
                             int cc_minor, int num_sms);
/* src/planner.h:60, :68-69, :75-79 */
int ggemm_plan_num_moduli(const ggemm_config_t* cfg, int k);
int ggemm_plan(const ggemm_problem_t* probs, int num, const ggemm_config_t* cfg,
               ggemm_path_t path, const ggemm_device_model_t* dm, ggemm_plan_entry_t* out);
int ggemm_plan_ex(const ggemm_problem_t* probs, int num, const ggemm_config_t* cfg,
                  ggemm_path_t path, const ggemm_device_model_t* dm, ggemm_plan_entry_t* out,
                  int* memo, size_t memo_cap);
size_t ggemm_plan_memo_cap(int num);

#ifdef __cplusplus
}
static_assert(sizeof(oz2_problem) == 136, "oz2_problem layout");
static_assert(sizeof(i8_problem) == 48, "i8_problem layout");
#endif
#endif
