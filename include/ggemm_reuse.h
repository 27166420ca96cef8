/* ggemm_reuse.h -- operand reuse for GGEMM_PATH_EMU_GROUPED_REUSE: the host pass that finds A / B
 * operands shared across a group so the Ozaki-II prep runs once per unique operand.
 *
 * C form of the reference's interface src/operand_reuse.h:28-85 (reuse_policy, reuse_plan,
 * reuse_arena::reserve, build_operand_reuse, operand_reuse_bytes); same fields and semantics:
 *   A-key(g) = (A, lda, m, k), B-key(g) = (B, ldb, n, k); problems with N_g <= 0 are ignored.
 *   Unique operands are numbered in order of first appearance; rep = first problem carrying it.
 *   REUSE_EXACT_N : N is part of the key (operands shared only between problems with equal N).
 *   REUSE_PROMOTE : shared regardless of N; every problem is promoted to the largest N of its
 *                   connected component (problems linked through a shared A or B), because the
 *                   row / column scale shifts depend on N through the norm budget T_N.
 * build_operand_reuse allocates nothing: the arena holds all storage, sized at creation.
 */
#ifndef GGEMM_REUSE_H
#define GGEMM_REUSE_H
#include "ggemm.h"

#ifdef __cplusplus
extern "C" {
#endif

enum { REUSE_EXACT_N = 0, REUSE_PROMOTE = 1 };               /* src/operand_reuse.h:40 */
enum { REUSE_OK = 0, REUSE_ERR_CAPACITY = 1, REUSE_ERR_INVALID = 2 };   /* :42-46 */

/* src/operand_reuse.h:49-63: a view into the arena, valid until its next build. */
typedef struct {
  int status;
  int num_problems;   /* G */
  int num_ua, num_ub; /* unique A / unique B */
  int num_emu;        /* problems with N_g > 0 */
  int num_promoted;   /* problems with eff_nmod > N_g (PROMOTE) */
  const int* ua_rep;  /* [num_ua] representative problem of each unique A */
  const int* ua_nmod; /* [num_ua] residues to prep for it */
  const int* ub_rep;  /* [num_ub] */
  const int* ub_nmod; /* [num_ub] */
  const int* prob_a;  /* [G] unique-A id of problem g, -1 if not emulated */
  const int* prob_b;  /* [G] unique-B id, -1 if not emulated */
  const int* eff_nmod;/* [G] moduli problem g runs with (N_g under EXACT_N), 0 if ignored */
} reuse_plan;

typedef struct reuse_arena_s* reuse_arena_t;

/* reuse_arena::reserve (src/operand_reuse.h:71-75): storage for max_problems (>= 1; more than
 * 2^30 -> REUSE_ERR_CAPACITY and an empty arena).  *out is set in both cases; destroy it. */
int reuse_arena_create(int max_problems, reuse_arena_t* out);
void reuse_arena_destroy(reuse_arena_t a);
int reuse_arena_capacity(reuse_arena_t a);

/* src/operand_reuse.h:79-81.  nmod[g] <= 0 marks problem g as not emulated. */
reuse_plan build_operand_reuse(reuse_arena_t a, const ggemm_problem_t* probs, int num, const int* nmod,
                               int policy);

/* src/operand_reuse.h:83-85: modelled prep traffic and residue workspace (bytes), per-problem
 * prep with N_g ("before") and per-unique-operand prep with ua_nmod / ub_nmod ("after"). */
typedef struct {
  double prep_read, prep_write, ws_A8, ws_B8;
} reuse_bytes;
void operand_reuse_bytes(const reuse_plan* plan, const ggemm_problem_t* probs, const int* nmod, reuse_bytes* before,
                         reuse_bytes* after);

#ifdef __cplusplus
}
#endif
#endif
