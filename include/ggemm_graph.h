/* ggemm_graph.h -- plan / execute for repeated calls with identical shapes, replayed as a
 * hipGraph.  Drop-in for the reference's src/ggemm_graph.h:26-47 (same names and semantics).
 *
 * ggemm_make_plan   : planning + descriptors + one H2D into plan-owned memory + stream capture
 *                     of the launch sequence -> instantiated hipGraph.  Allocates and
 *                     synchronises: call it outside timed regions.
 * ggemm_execute_plan: hipGraphLaunch (no host planning, no H2D, no allocation).
 * ggemm_plan_update_pointers: same shapes, new A/B/C device pointers; patches the plan's device
 *                     descriptors with one small H2D (kernels read pointers from descriptors, so
 *                     the graph is never re-captured).
 * Every execution is ordered against the handle's stream (shared residue / INT32 scratch).
 * A plan must be destroyed before its handle.  Plans are not thread-safe.
 */
#ifndef GGEMM_GRAPH_H
#define GGEMM_GRAPH_H
#include "ggemm.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ggemm_plan_s* ggemm_plan_t;

/* src/ggemm_graph.h:30-31.  path: GGEMM_PATH_EMU_GROUPED or GGEMM_PATH_AUTO (others -> NULL). */
ggemm_plan_t ggemm_make_plan(ggemm_handle_t h, ggemm_path_t path, const ggemm_config_t* cfg,
                             const ggemm_problem_t* problems, int num_problems);
/* src/ggemm_graph.h:32-33.  *err (optional) receives the GGEMM_ERR_* code. */
ggemm_plan_t ggemm_make_plan_ex(ggemm_handle_t h, ggemm_path_t path, const ggemm_config_t* cfg,
                                const ggemm_problem_t* problems, int num_problems, int* err);
/* src/ggemm_graph.h:36 */
int ggemm_execute_plan(ggemm_plan_t plan, hipStream_t stream);
/* src/ggemm_graph.h:41-42.  A/B/C: HOST arrays of num_problems device pointers, NULL = keep. */
int ggemm_plan_update_pointers(ggemm_plan_t plan, const double* const* A, const double* const* B,
                               double* const* C);
/* src/ggemm_graph.h:45 */
int ggemm_plan_get_stats(ggemm_plan_t plan, ggemm_stats_t* stats);
/* src/ggemm_graph.h:47 */
void ggemm_destroy_plan(ggemm_plan_t plan);

#ifdef __cplusplus
}
#endif
#endif
