// noalloc.hip -- ggemm_grouped_dgemm_noalloc: the grouped emulated DGEMM without a handle and without
// any allocation, for callers that cannot allocate device memory (tight serving loops, harnesses
// that forbid hipMalloc).  It has no counterpart in the reference.  It is not capturable: the call
// waits for its descriptor copy (a stream synchronisation), so on a stream that is being captured
// it returns GGEMM_ERR_INVALID before any HIP call that would invalidate the capture.
//
// Every device buffer the pipeline needs beyond the caller's A, B and C -- residue planes, CRT digit
// and abs-plane products, row / column shift words, the descriptor blob and tile schedules -- lives
// in `scratch`, a file-scope device array of GGEMM_NOALLOC_SCRATCH_BYTES that each GPU holds for
// the life of the process.  It is carved exactly like the workspace of a handle created with
// ggemm_create(GGEMM_NOALLOC_MAX_PROBLEMS, GGEMM_NOALLOC_MAX_ELEMS x 3): the same kernels run on the
// same layouts, so the bits equal ggemm_grouped_dgemm's.  Host-side scratch (plan entries, index
// lists, the descriptor image, the INT8 and FP64 tile-schedule builders' work arrays) is static or
// sized once at set-up, so a call allocates no host memory either.
//
// Set-up, once per device on the first call with that device current: hipGetSymbolAddress of
// `scratch` (its device address on this GPU; the array's name in host code is only a host-side
// stand-in), the device model and the resident CRT tables (device globals, filled by a copy).
// Every call on a GPU shares that GPU's scratch and it keeps the last call's contents; nothing in
// it needs to start at zero: every byte whose value reaches an output the call has written first
// (the digit and residue padding included).  The residue planes of rows / columns that hold a NaN
// or an Inf are not written; the INT8 GEMM may read whatever bytes an earlier call left there, but
// only entries that take the safety fallback (which reads neither digits nor products) consume
// those sums.  Calls are serialised on the host by a mutex; the
// descriptor image is copied from static host memory and the call waits for that copy (and so for
// earlier work on the stream) before it enqueues its kernels.  Calls that overlap on one GPU from
// different streams race on the scratch.
#include <cstdio>
#include <cstring>
#include <mutex>

#include "call.hpp"

namespace ggemm {
namespace {

constexpr size_t kScratchBytes = GGEMM_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxProblems = GGEMM_NOALLOC_MAX_PROBLEMS;
constexpr size_t kMaxElems = GGEMM_NOALLOC_MAX_ELEMS;
constexpr int kMaxDevices = 64;
constexpr size_t kHostBlobBytes = 1u << 20;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_mu;
ggemm_handle_s g_dev[kMaxDevices];   // per device: the carved workspace (zero-initialised: not set up)
bool g_ready[kMaxDevices];
// host scratch shared by all devices (calls are serialised by g_mu)
ggemm_plan_entry_t g_plan[kMaxProblems];
int g_memo[2 * kMaxProblems];
int g_emu_idx[kMaxProblems], g_nat_idx[kMaxProblems];
alignas(256) char g_blob[kHostBlobBytes];
bool g_limit_reported = false;
bool g_capture_reported = false;

// Carves this device's scratch into the handle-shaped workspace (returns a GGEMM_ERR_* code).
int setup(int dev) {
  ggemm_handle_s* h = &g_dev[dev];
  void* base = nullptr;
  if (hipGetSymbolAddress(&base, HIP_SYMBOL(scratch)) != hipSuccess || !base) return GGEMM_ERR_CUDA;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return GGEMM_ERR_CUDA;
  if (oz2_init_constants() != 0) return GGEMM_ERR_NUMERICS;
  std::memset(h, 0, sizeof *h);
  h->device = dev;
  h->num_cus = prop.multiProcessorCount;
  ggemm_device_model_init(&h->dm, prop.gcnArchName, prop.major, prop.minor, h->num_cus);
  h->max_problems = kMaxProblems;
  h->max_A_elems = h->max_B_elems = h->max_C_elems = kMaxElems;
  h->min_k = kKpAlign;
  h->packed_max_kp = kPackedMaxKp;
  h->compact = 1;
  size_workspace(h, kMaxProblems, kMaxElems, kMaxElems, kMaxElems, kKpAlign);
  // the carve: A8 | B8 | C32 | row shifts | column shifts | descriptor blob, 256-byte aligned
  char* p = static_cast<char*>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* q = p + off;
    off = align_up(off + bytes, kBufAlign);
    return q;
  };
  h->A8 = reinterpret_cast<int8_t*>(take(h->A8_bytes));
  h->B8 = reinterpret_cast<int8_t*>(take(h->B8_bytes));
  h->C32 = reinterpret_cast<int32_t*>(take(h->C32_bytes));
  h->row_shift = reinterpret_cast<int32_t*>(take(h->row_shift_elems * sizeof(int32_t)));
  h->col_shift = reinterpret_cast<int32_t*>(take(h->col_shift_elems * sizeof(int32_t)));
  h->d_desc = take(h->desc_bytes);
  if (off > kScratchBytes || h->desc_bytes > kHostBlobBytes) return GGEMM_ERR_WORKSPACE;
  h->h_desc = g_blob;
  h->plan = g_plan;
  h->plan_memo = g_memo;
  h->plan_memo_cap = sizeof g_memo / sizeof g_memo[0];
  h->emu_idx = g_emu_idx;
  h->nat_idx = g_nat_idx;
  i8_reserve_host((size_t)kMaxProblems * kMaxPlanes);   // schedule builder's host scratch, once
  const char* e = std::getenv("GGEMM_STATS_REPAIR");
  h->stats_repair = (e && std::atoi(e) == 1) ? 1 : 0;
  return GGEMM_OK;
}

void report_limits(const char* what) {
  if (g_limit_reported) return;
  g_limit_reported = true;
  std::fprintf(stderr,
               "[ggemm] ggemm_grouped_dgemm_noalloc: %s (limits: %d problems, sum m*k, sum k*n and sum m*n "
               "each <= %zu elements, k >= %d per emulated problem; use a handle for larger calls)\n",
               what, kMaxProblems, kMaxElems, kKpAlign);
}

}  // namespace
}  // namespace ggemm

using namespace ggemm;

extern "C" int ggemm_grouped_dgemm_noalloc(ggemm_path_t path, const ggemm_config_t* cfg,
                                           const ggemm_problem_t* problems, int num_problems, hipStream_t stream,
                                           ggemm_stats_t* stats) {
  ggemm_stats_t local;
  ggemm_stats_t* st = stats ? stats : &local;
  std::memset(st, 0, sizeof(*st));
  st->num_problems = num_problems;
  st->num_repaired = st->num_uncertified = st->num_safety_fallback = -1;
  if (path != GGEMM_PATH_EMU_GROUPED && path != GGEMM_PATH_AUTO) return GGEMM_ERR_INVALID;
  static const ggemm_config_t kDefault = {0, 1e-15, 1, 0};
  if (!cfg) cfg = &kDefault;
  if (cfg->num_moduli < 0 || cfg->num_moduli == 1 || cfg->num_moduli > GGEMM_MAX_MODULI) return GGEMM_ERR_INVALID;
  const int repair = repair_mode_of(path, cfg);
  if (repair < 0) return GGEMM_ERR_INVALID;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return GGEMM_ERR_CUDA;
  // the call synchronises its stream (descriptor copy, counters): refuse a capturing stream before
  // any call that a capture forbids, so the caller's capture stays intact
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess) return GGEMM_ERR_CUDA;
  std::lock_guard<std::mutex> lk(g_mu);
  if (cap != hipStreamCaptureStatusNone) {
    if (!g_capture_reported) {
      g_capture_reported = true;
      std::fprintf(stderr, "[ggemm] ggemm_grouped_dgemm_noalloc: the stream is being captured; this entry point "
                           "synchronises its stream and cannot be captured (use ggemm_make_plan)\n");
    }
    return GGEMM_ERR_INVALID;
  }
  if (!g_ready[dev]) {
    const int r = setup(dev);
    if (r) return r;
    g_ready[dev] = true;
  }
  ggemm_handle_s* h = &g_dev[dev];
  h->stream = stream;
  int r = validate(h, problems, num_problems);
  if (r) {
    if (r == GGEMM_ERR_WORKSPACE) report_limits("call exceeds the static workspace");
    if (r == GGEMM_ERR_INVALID && num_problems > kMaxProblems) report_limits("too many problems");
    return r;
  }
  if ((r = counters_reset(h, stream))) return r;
  r = ggemm_plan_ex(problems, num_problems, cfg, path, &h->dm, h->plan, h->plan_memo, h->plan_memo_cap);
  if (r) return r;
  GroupedCall c;
  char* db = static_cast<char*>(h->d_desc);   // this device's scratch address
  r = build_grouped(h, problems, num_problems, h->plan, h->emu_idx, h->nat_idx, g_blob, db, h->desc_bytes, &c, st);
  if (r) {
    if (r == GGEMM_ERR_WORKSPACE) report_limits("call exceeds the static workspace");
    return r;
  }
  if (c.h2d_bytes) {
    // the source is static host memory that the next call rewrites: wait for the copy to land
    if (hipMemcpyAsync(db, g_blob, c.h2d_bytes, hipMemcpyHostToDevice, stream) != hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess)
      return GGEMM_ERR_CUDA;
  }
  r = enqueue_grouped(c, db, stream, repair, &st->kernel_launches);
  if (!r) r = counters_read(h, stream, st);
  return r;
}
