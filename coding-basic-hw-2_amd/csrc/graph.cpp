// graph.cpp -- plan / execute: the grouped pipeline frozen into plan-owned descriptors and
// replayed as a hipGraph (semantics of the reference's src/ggemm_graph.cu:31-394).
//
// Every kernel of the pipeline (prep, INT8 GEMM, reconstruct, native FP64 GEMM) reads its A/B/C
// pointers from device descriptors inside the plan's blob; the captured kernel arguments are
// only blob addresses.  ggemm_plan_update_pointers therefore patches the pinned mirror and issues
// one small H2D on the handle's stream -- no re-capture and no graph-exec update, for any mix of
// emulated and native problems.  The graph contains kernel nodes only (no memset, no library
// calls).  Executions on a stream other than the handle's are joined with the handle's stream on
// both sides, so all users of one handle's shared scratch are totally ordered.
#include <algorithm>
#include <cstring>
#include <new>

#include "call.hpp"

using namespace ggemm;

struct ggemm_plan_s {
  ggemm_handle_t h;
  int num;
  ggemm_problem_t* probs;        // host copy (pointers patched by update_pointers)
  ggemm_plan_entry_t* entries;
  int *emu_idx, *nat_idx;
  int repair;
  GroupedCall call;
  char* h_blob;                  // pinned mirror of d_blob
  char* d_blob;
  size_t blob_bytes;
  hipStream_t cap;               // private capture stream
  hipGraph_t graph;
  hipGraphExec_t exec;           // null when the plan has no work
  hipEvent_t ev_h, ev_p, ev_upd;
  ggemm_stats_t st;
};

namespace {

#define HIPC(x) do { if ((x) != hipSuccess) return GGEMM_ERR_CUDA; } while (0)

void free_plan(ggemm_plan_t p) {
  if (!p) return;
  if (p->h) (void)hipStreamSynchronize(p->h->stream);
  if (p->exec) (void)hipGraphExecDestroy(p->exec);
  if (p->graph) (void)hipGraphDestroy(p->graph);
  if (p->cap) (void)hipStreamDestroy(p->cap);
  if (p->ev_h) (void)hipEventDestroy(p->ev_h);
  if (p->ev_p) (void)hipEventDestroy(p->ev_p);
  if (p->ev_upd) { (void)hipEventSynchronize(p->ev_upd); (void)hipEventDestroy(p->ev_upd); }
  if (p->d_blob) (void)hipFree(p->d_blob);
  if (p->h_blob) (void)hipHostFree(p->h_blob);
  delete[] p->probs;
  delete[] p->entries;
  delete[] p->emu_idx;
  delete[] p->nat_idx;
  delete p;
}

int build(ggemm_plan_t p, ggemm_path_t path, const ggemm_config_t* cfg) {
  ggemm_handle_t h = p->h;
  int r = ggemm_plan(p->probs, p->num, cfg, path, &h->dm, p->entries);
  if (r) return r;
  // size the blob exactly: count emulated planes and native problems first
  size_t ne = 0, n_i8 = 0, nn = 0;
  for (int g = 0; g < p->num; ++g) {
    const ggemm_plan_entry_t& e = p->entries[g];
    if (e.route == GGEMM_ROUTE_EMPTY) continue;
    if (e.route != GGEMM_ROUTE_EMU) { ++nn; continue; }
    ++ne;
    n_i8 += e.num_moduli + OZ2_EXTRA_PLANES;
  }
  const BlobLayout L = layout_for(ne, 0, n_i8, nn, nn ? sched_bytes((int)nn) : 0, ne ? sched_bytes((int)n_i8) : 0);
  p->blob_bytes = align_up(std::max<size_t>(L.total, 1), kBufAlign);
  HIPC(hipMalloc(&p->d_blob, p->blob_bytes));
  HIPC(hipHostMalloc(&p->h_blob, p->blob_bytes, hipHostMallocDefault));
  std::memset(p->h_blob, 0, p->blob_bytes);
  ggemm_stats_t& st = p->st;
  st.num_problems = p->num;
  r = build_grouped(h, p->probs, p->num, p->entries, p->emu_idx, p->nat_idx, p->h_blob,
                    static_cast<const char*>(p->d_blob), p->blob_bytes, &p->call, &st);
  if (r) return r;
  st.num_repaired = st.num_uncertified = st.num_safety_fallback = -1;   // filled per execute
  HIPC(hipMemcpyAsync(p->d_blob, p->h_blob, p->call.h2d_bytes ? p->call.h2d_bytes : 1, hipMemcpyHostToDevice,
                      h->stream));
  HIPC(hipEventRecord(p->ev_upd, h->stream));
  HIPC(hipStreamSynchronize(h->stream));
  if (p->call.ne == 0 && p->call.nn == 0) return GGEMM_OK;   // nothing to run
  int launches = 0;
  HIPC(hipStreamBeginCapture(p->cap, hipStreamCaptureModeRelaxed));
  r = enqueue_grouped(p->call, p->d_blob, p->cap, p->repair, &launches);
  hipGraph_t g = nullptr;
  const hipError_t ce = hipStreamEndCapture(p->cap, &g);
  if (!r && ce != hipSuccess) r = GGEMM_ERR_CUDA;
  if (r) {
    if (g) (void)hipGraphDestroy(g);
    return r;
  }
  p->graph = g;
  st.kernel_launches = launches;
  HIPC(hipGraphInstantiate(&p->exec, p->graph, nullptr, nullptr, 0));
  HIPC(hipGraphUpload(p->exec, h->stream));
  HIPC(hipStreamSynchronize(h->stream));
  return GGEMM_OK;
}

}  // namespace

extern "C" ggemm_plan_t ggemm_make_plan_ex(ggemm_handle_t h, ggemm_path_t path, const ggemm_config_t* cfg,
                                           const ggemm_problem_t* problems, int num, int* err) {
  int dummy;
  int& e = err ? *err : dummy;
  e = GGEMM_ERR_INVALID;
  if (!h || (path != GGEMM_PATH_EMU_GROUPED && path != GGEMM_PATH_AUTO)) return nullptr;
  if ((e = validate(h, problems, num))) return nullptr;
  static const ggemm_config_t kDefault = {0, 1e-15, 1, 0};
  if (!cfg) cfg = &kDefault;
  if (cfg->num_moduli < 0 || cfg->num_moduli == 1 || cfg->num_moduli > GGEMM_MAX_MODULI ||
      repair_mode_of(path, cfg) < 0) {
    e = GGEMM_ERR_INVALID;
    return nullptr;
  }
  ggemm_plan_t p = new (std::nothrow) ggemm_plan_s();
  if (!p) { e = GGEMM_ERR_ALLOC; return nullptr; }
  p->h = h;
  p->num = num;
  p->repair = repair_mode_of(path, cfg);
  const size_t P = (size_t)std::max(num, 1);
  p->probs = new (std::nothrow) ggemm_problem_t[P];
  p->entries = new (std::nothrow) ggemm_plan_entry_t[P];
  p->emu_idx = new (std::nothrow) int[P];
  p->nat_idx = new (std::nothrow) int[P];
  if (!p->probs || !p->entries || !p->emu_idx || !p->nat_idx) {
    free_plan(p);
    e = GGEMM_ERR_ALLOC;
    return nullptr;
  }
  if (num > 0) std::memcpy(p->probs, problems, sizeof(ggemm_problem_t) * num);
  if (hipStreamCreateWithFlags(&p->cap, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreateWithFlags(&p->ev_h, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&p->ev_p, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&p->ev_upd, hipEventDisableTiming) != hipSuccess) {
    free_plan(p);
    e = GGEMM_ERR_CUDA;
    return nullptr;
  }
  if ((e = build(p, path, cfg))) {
    free_plan(p);
    return nullptr;
  }
  return p;
}

extern "C" ggemm_plan_t ggemm_make_plan(ggemm_handle_t h, ggemm_path_t path, const ggemm_config_t* cfg,
                                        const ggemm_problem_t* problems, int num) {
  return ggemm_make_plan_ex(h, path, cfg, problems, num, nullptr);
}

extern "C" int ggemm_execute_plan(ggemm_plan_t p, hipStream_t stream) {
  if (!p) return GGEMM_ERR_INVALID;
  if (!p->exec) return GGEMM_OK;
  const hipStream_t hs = p->h->stream;
  const bool counters = p->h->stats_repair && p->call.ne > 0;
  int r;
  if (stream == hs) {
    if (counters && (r = counters_reset(p->h, stream))) return r;
    HIPC(hipGraphLaunch(p->exec, stream));
  } else {
    HIPC(hipEventRecord(p->ev_h, hs));
    HIPC(hipStreamWaitEvent(stream, p->ev_h, 0));
    if (counters && (r = counters_reset(p->h, stream))) return r;
    HIPC(hipGraphLaunch(p->exec, stream));
    HIPC(hipEventRecord(p->ev_p, stream));
    HIPC(hipStreamWaitEvent(hs, p->ev_p, 0));
  }
  if (counters) return counters_read(p->h, stream, &p->st);
  return GGEMM_OK;
}

extern "C" int ggemm_plan_update_pointers(ggemm_plan_t p, const double* const* A, const double* const* B,
                                          double* const* C) {
  if (!p) return GGEMM_ERR_INVALID;
  for (int g = 0; g < p->num; ++g) {   // validate first: a bad call leaves the plan untouched
    const ggemm_problem_t& q = p->probs[g];
    if (q.m == 0 || q.n == 0) continue;
    if (C && !C[g]) return GGEMM_ERR_INVALID;
    if (q.k > 0 && ((A && !A[g]) || (B && !B[g]))) return GGEMM_ERR_INVALID;
  }
  for (int g = 0; g < p->num; ++g) {
    if (A) p->probs[g].A = A[g];
    if (B) p->probs[g].B = B[g];
    if (C) p->probs[g].C = C[g];
  }
  ggemm_handle_t h = p->h;
  HIPC(hipEventSynchronize(p->ev_upd));   // the previous patch H2D has read the mirror
  const GroupedCall& c = p->call;
  oz2_problem* hoz = reinterpret_cast<oz2_problem*>(p->h_blob + c.L.off_oz);
  for (int j = 0; j < c.ne; ++j) {
    const ggemm_problem_t& q = p->probs[p->emu_idx[j]];
    hoz[j].A = q.A;
    hoz[j].B = q.B;
    hoz[j].C = q.C;
  }
  F64Problem* hf = reinterpret_cast<F64Problem*>(p->h_blob + c.L.off_f64);
  for (int i = 0; i < c.nn; ++i) {
    const ggemm_problem_t& q = p->probs[p->nat_idx[i]];
    hf[i].A = q.A;
    hf[i].B = q.B;
    hf[i].C = q.C;
  }
  if (c.ne > 0)
    HIPC(hipMemcpyAsync(p->d_blob + c.L.off_oz, p->h_blob + c.L.off_oz, (size_t)c.ne * sizeof(oz2_problem),
                        hipMemcpyHostToDevice, h->stream));
  if (c.nn > 0)
    HIPC(hipMemcpyAsync(p->d_blob + c.L.off_f64, p->h_blob + c.L.off_f64, (size_t)c.nn * sizeof(F64Problem),
                        hipMemcpyHostToDevice, h->stream));
  HIPC(hipEventRecord(p->ev_upd, h->stream));
  return GGEMM_OK;
}

extern "C" int ggemm_plan_get_stats(ggemm_plan_t p, ggemm_stats_t* st) {
  if (!p || !st) return GGEMM_ERR_INVALID;
  *st = p->st;
  return GGEMM_OK;
}

extern "C" void ggemm_destroy_plan(ggemm_plan_t p) { free_plan(p); }
