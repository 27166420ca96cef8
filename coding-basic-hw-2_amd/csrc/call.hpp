// call.hpp -- descriptor building and launch sequencing shared by direct calls and plans.
#pragma once
#include "common.hpp"
#include "ggemm_reuse.h"

namespace ggemm {

// Descriptor blob (identical in the pinned host mirror and the device copy):
//   [oz2_problem x ne][YDesc x ne][i8_problem x n_i8][I8Epi x n_i8][F64Problem x nn]
//   [F64 schedule(s)][INT8 schedule(s)]
// every section 256-byte aligned; the INT8 schedule is last so the H2D can stop at its used size.
struct BlobLayout {
  size_t off_oz, off_yd, off_prep, off_po, off_i8, off_epi, off_f64, off_sf64, off_si8, total;
};
// nprep: prep descriptors of operand reuse (unique A, then unique B), 0 without reuse
// off_po: the prep launch's problem order, then its block offsets (2 (ne + nprep) ints; see prep_launch)
BlobLayout layout_for(size_t ne, size_t nprep, size_t n_i8, size_t nn, size_t sched_f64, size_t sched_i8);
inline size_t sched_img(int entries) { return align_up(sched_bytes(entries), kBufAlign); }

// Everything the launch sequence of one grouped call needs.
struct GroupedCall {
  int ne = 0, nn = 0;             // emulated / native problems
  size_t n_i8 = 0;                // (problem, plane) INT8 products
  int max_m = 0, max_n = 0;
  int nmax = 0;                   // largest num_moduli among the emulated problems
  int nprep = 0;                  // operand reuse: prep descriptors (0: prep runs on the ne problems)
  int pmax_m = 0, pmax_n = 0;     // prep grid over the unique operands
  BlobLayout L{};
  i8_sched_info i8info{};
  int i8_kernel = kI8General;     // INT8 GEMM kernel the schedule was built for
  int i8_hw = -1;                 // large-tile kernel: units dispatched one workgroup each (-1: all)
  bool blocked = false;           // digit and abs planes in the blocked layout
  bool packed = false;            // every problem's residue planes in the packed layout
  int packed_kp = 0;              // problems with Kp at most this (> 0) use the packed layout
  int f64_tiles = 0;              // native GEMM launch word (tile count, kF64Tile128 for 128 x 128 tiles)
  ReconGrid rgrid{};              // compact reconstruct / dot-product grids
  int dot_form = 0;               // the handle's dot-product form override (kDotForm*)
  long long prep_blocks = 0;      // workgroups of the compact prep grid (per split)
  size_t h2d_bytes = 0;           // bytes of the blob to copy
};

int validate(ggemm_handle_t h, const ggemm_problem_t* p, int num);
// Workspace sizes of a handle for the given capacity (src/ggemm.cu:228-341 rules): fills A8_bytes,
// B8_bytes, C32_bytes, row_shift_elems, col_shift_elems and desc_bytes; allocates nothing.
void size_workspace(ggemm_handle_s* h, int max_problems, size_t max_A, size_t max_B, size_t max_C, int min_k);
int repair_mode_of(ggemm_path_t path, const ggemm_config_t* cfg);   // OZ2_REPAIR_* or -1
int counters_reset(ggemm_handle_t h, hipStream_t s);
int counters_read(ggemm_handle_t h, hipStream_t s, ggemm_stats_t* st);

// Plans nothing: takes the planner output and fills descriptors + schedules into hb (capacity
// cap), and the stats fields num_fallback / moduli_* / reuse_* / num_unique_*.  emu_idx and
// nat_idx are caller scratch of >= num ints.  Returns GGEMM_OK, WORKSPACE, INVALID or I8GEMM.
// db: the device blob hb is copied to (descriptors that point into the blob address it there).
// rp: operand-reuse plan (path EMU_GROUPED_REUSE) or nullptr
int build_grouped(ggemm_handle_t h, const ggemm_problem_t* probs, int num, const ggemm_plan_entry_t* plan,
                  int* emu_idx, int* nat_idx, char* hb, const char* db, size_t cap, GroupedCall* out, ggemm_stats_t* st,
                  const reuse_plan* rp = nullptr);
// Enqueues prep -> INT8 GEMM -> reconstruct (if ne > 0) and the native FP64 GEMM (if nn > 0) on s,
// reading descriptors from the device blob db.  *launches += kernels issued.  prof_set: stage
// timing event set (-1 = none).
int enqueue_grouped(const GroupedCall& c, const char* db, hipStream_t s, int repair, int* launches,
                    int prof_set = -1);

// Native descriptor from a problem.
inline F64Problem f64_of(const ggemm_problem_t& p) {
  F64Problem f;
  f.m = p.m; f.n = p.n; f.k = p.k; f.lda = p.lda; f.ldb = p.ldb; f.ldc = p.ldc;
  f.A = p.A; f.B = p.B; f.C = p.C; f.alpha = p.alpha; f.beta = p.beta;
  return f;
}

}  // namespace ggemm
