// count_allocs.cpp -- counts the heap allocations the library makes inside its calls.
//
// The reference's planner test (tests/test_planner.cpp:33-50, 429-464) replaces the global
// operator new and requires zero calls inside ggemm_plan after the first call, and its INT8 test
// requires no growth of the schedule builder's host scratch after a reserve
// (tests/test_i8_grouped.cu:348-352).  This program interposes both operator new and the C
// allocator (malloc / calloc / realloc / aligned forms, forwarded to glibc's own entry points) for
// the whole process.
//
// Without arguments (host only, no GPU): plans a 65535-problem group on the AUTO and EMU_GROUPED
// paths and prints one line per path:
//   path=<p> first=<allocations in the first call> steady=<allocations in 5 later calls>
// With the argument "gpu" (needs a GPU): runs a small mixed group (emulated problems, k = 0,
// alpha = 0 and k <= 16 problems that take native routes) through ggemm_grouped_dgemm on every
// path, ggemm_execute_plan, ggemm_plan_update_pointers + ggemm_execute_plan, and
// ggemm_grouped_dgemm_noalloc, and prints one line per call kind:
//   call=<name> first=<n> steady=<n> first_all=<n> steady_all=<n>
// where first / steady count the allocations whose caller lies in the library's own code (the HIP
// runtime allocates command objects of its own inside every launch or copy; those are only in the
// *_all figures), first for the first call of the kind and steady for 5 later calls.
// Built and run by tests/test_planner_log.py (host) and tests/test_gpu_host_alloc.py (GPU);
// TEST INFRASTRUCTURE ONLY.
#include <link.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "ggemm.h"
#include "ggemm_graph.h"
#include "ggemm_oz2.h"

extern "C" void* __libc_malloc(size_t);
extern "C" void* __libc_calloc(size_t, size_t);
extern "C" void* __libc_realloc(void*, size_t);
extern "C" void* __libc_memalign(size_t, size_t);
extern "C" void __libc_free(void*);

static std::atomic<long> g_allocs{0};       // every allocation while counting
static std::atomic<long> g_lib_allocs{0};   // those called from the library's code
static std::atomic<bool> g_counting{false};
static uintptr_t g_lib_lo = 0, g_lib_hi = 0;   // address range of libggemm's loaded segments

static inline void note(void* ra) {
  if (!g_counting.load(std::memory_order_relaxed)) return;
  g_allocs.fetch_add(1, std::memory_order_relaxed);
  const uintptr_t a = reinterpret_cast<uintptr_t>(ra);
  if (a >= g_lib_lo && a < g_lib_hi) g_lib_allocs.fetch_add(1, std::memory_order_relaxed);
}
#define RA __builtin_return_address(0)

extern "C" void* malloc(size_t n) { note(RA); return __libc_malloc(n); }
extern "C" void* calloc(size_t a, size_t b) { note(RA); return __libc_calloc(a, b); }
extern "C" void* realloc(void* p, size_t n) { note(RA); return __libc_realloc(p, n); }
extern "C" void* memalign(size_t a, size_t n) { note(RA); return __libc_memalign(a, n); }
extern "C" void* aligned_alloc(size_t a, size_t n) { note(RA); return __libc_memalign(a, n); }
extern "C" int posix_memalign(void** out, size_t a, size_t n) {
  note(RA);
  void* p = __libc_memalign(a, n);
  if (!p) return 12;
  *out = p;
  return 0;
}
extern "C" void free(void* p) { __libc_free(p); }

static void* new_impl(size_t n, void* ra) {
  note(ra);
  if (void* p = __libc_malloc(n ? n : 1)) return p;
  throw std::bad_alloc();
}
static void* new_nothrow_impl(size_t n, void* ra) noexcept {
  note(ra);
  return __libc_malloc(n ? n : 1);
}
void* operator new(size_t n) { return new_impl(n, RA); }
void* operator new[](size_t n) { return new_impl(n, RA); }
void* operator new(size_t n, const std::nothrow_t&) noexcept { return new_nothrow_impl(n, RA); }
void* operator new[](size_t n, const std::nothrow_t&) noexcept { return new_nothrow_impl(n, RA); }
void operator delete(void* p) noexcept { __libc_free(p); }
void operator delete[](void* p) noexcept { __libc_free(p); }
void operator delete(void* p, size_t) noexcept { __libc_free(p); }
void operator delete[](void* p, size_t) noexcept { __libc_free(p); }

static int find_lib(struct dl_phdr_info* info, size_t, void*) {
  if (!info->dlpi_name || !std::strstr(info->dlpi_name, "libggemm_mi355x.so")) return 0;
  uintptr_t lo = UINTPTR_MAX, hi = 0;
  for (int i = 0; i < info->dlpi_phnum; ++i) {
    const ElfW(Phdr)& ph = info->dlpi_phdr[i];
    if (ph.p_type != PT_LOAD) continue;
    const uintptr_t a = info->dlpi_addr + ph.p_vaddr;
    lo = a < lo ? a : lo;
    hi = a + ph.p_memsz > hi ? a + ph.p_memsz : hi;
  }
  g_lib_lo = lo;
  g_lib_hi = hi;
  return 1;
}

// tests/test_planner.cpp:371-386: the LCG group with EMPTY / K_ZERO / K_TOO_LARGE / SMALL_K and
// alpha = 0 problems mixed in
static std::vector<ggemm_problem_t> make_group(int G, unsigned seed) {
  std::vector<ggemm_problem_t> ps(G);
  unsigned s = seed;
  auto next = [&s](int lo, int hi) {
    s = s * 1664525u + 1013904223u;
    return lo + (int)((s >> 8) % (unsigned)(hi - lo + 1));
  };
  for (int g = 0; g < G; ++g) {
    const int r = next(0, 99);
    int m = next(1, 2048);
    const int n = next(1, 2048);
    int k = next(1, 8192);
    if (r < 3) k = 0;
    else if (r < 5) m = 0;
    else if (r < 7) k = GGEMM_MAX_K_EXACT + next(1, 1000);
    else if (r < 12) k = next(1, 16);
    ggemm_problem_t& p = ps[g];
    std::memset(&p, 0, sizeof p);
    p.m = m; p.n = n; p.k = k;
    p.lda = m > 0 ? m : 1; p.ldb = k > 0 ? k : 1; p.ldc = m > 0 ? m : 1;
    p.alpha = r == 50 ? 0.0 : 1.0;
    p.beta = (r & 1) ? 1.0 : 0.0;
  }
  return ps;
}

static int host_planner() {
  ggemm_device_model_t dm;
  ggemm_device_model_init(&dm, "gfx950", 9, 5, 256);
  const int G = 65535;
  std::vector<ggemm_problem_t> ps = make_group(G, 777u);
  std::vector<ggemm_plan_entry_t> e(G);
  ggemm_config_t cfg;
  std::memset(&cfg, 0, sizeof cfg);
  cfg.target_rel_err = 1e-15;
  cfg.allow_fallback = 1;
  int bad = 0;
  for (int path : {GGEMM_PATH_AUTO, GGEMM_PATH_EMU_GROUPED}) {
    g_allocs = 0;
    g_counting = true;
    bad |= ggemm_plan(ps.data(), G, &cfg, (ggemm_path_t)path, &dm, e.data());
    g_counting = false;
    const long first = g_allocs.load();
    g_allocs = 0;
    for (int r = 0; r < 5; ++r) {
      g_counting = true;
      bad |= ggemm_plan(ps.data(), G, &cfg, (ggemm_path_t)path, &dm, e.data());
      g_counting = false;
    }
    std::printf("path=%d first=%ld steady=%ld\n", path, first, g_allocs.load());
  }
  return bad ? 1 : 0;
}

#define CK(x)                                                              \
  do {                                                                     \
    if ((x) != hipSuccess) {                                               \
      std::fprintf(stderr, "HIP error at %s:%d: %s\n", __FILE__, __LINE__, #x); \
      return 1;                                                            \
    }                                                                      \
  } while (0)

// one kind of call: the first call, then 5 more, each followed by a stream synchronisation;
// f returns a GGEMM_ERR_* code
template <class F>
static int measure(const char* name, hipStream_t s, F f) {
  long counts[4];
  for (int phase = 0; phase < 2; ++phase) {
    g_allocs = 0;
    g_lib_allocs = 0;
    for (int r = 0; r < (phase ? 5 : 1); ++r) {
      g_counting = true;
      const int rc = f();
      g_counting = false;
      if (rc) {
        std::fprintf(stderr, "%s returned %d\n", name, rc);
        return 1;
      }
      if (hipStreamSynchronize(s) != hipSuccess) return 1;
    }
    counts[phase] = g_lib_allocs.load();
    counts[2 + phase] = g_allocs.load();
  }
  std::printf("call=%s first=%ld steady=%ld first_all=%ld steady_all=%ld\n", name, counts[0], counts[1], counts[2],
              counts[3]);
  std::fflush(stdout);
  return 0;
}

static int gpu_calls() {
  dl_iterate_phdr(find_lib, nullptr);
  if (!g_lib_hi) {
    std::fprintf(stderr, "libggemm_mi355x.so not found among the loaded objects\n");
    return 1;
  }
  // (m, n, k, alpha, beta): emulated problems, then K_ZERO, ALPHA_ZERO and SMALL_K (native routes)
  struct Shape { int m, n, k; double alpha, beta; };
  const Shape shapes[] = {{200, 150, 500, 1.0, 0.0}, {96, 80, 160, -1.5, 0.5}, {64, 64, 33, 1.0, 1.0},
                          {50, 40, 0, 1.0, 0.5},     {60, 70, 100, 0.0, 0.25}, {48, 40, 8, 2.0, 0.0}};
  const int G = sizeof shapes / sizeof shapes[0];
  hipStream_t s;
  CK(hipStreamCreate(&s));
  std::vector<ggemm_problem_t> ps(G);
  std::vector<double*> dA(G), dB(G), dC(G), dC2(G);
  size_t sa = 0, sb = 0, sc = 0;
  unsigned seed = 12345u;
  auto rnd = [&seed] {
    seed = seed * 1664525u + 1013904223u;
    return ((seed >> 8) & 0xffff) / 65536.0 - 0.5;
  };
  for (int g = 0; g < G; ++g) {
    const Shape& q = shapes[g];
    const size_t na = (size_t)q.m * q.k, nb = (size_t)q.k * q.n, nc = (size_t)q.m * q.n;
    std::vector<double> h(std::max({na, nb, nc, (size_t)1}));
    CK(hipMalloc(&dA[g], sizeof(double) * std::max(na, (size_t)1)));
    CK(hipMalloc(&dB[g], sizeof(double) * std::max(nb, (size_t)1)));
    CK(hipMalloc(&dC[g], sizeof(double) * nc));
    CK(hipMalloc(&dC2[g], sizeof(double) * nc));
    for (size_t i = 0; i < na; ++i) h[i] = rnd();
    CK(hipMemcpy(dA[g], h.data(), sizeof(double) * na, hipMemcpyHostToDevice));
    for (size_t i = 0; i < nb; ++i) h[i] = rnd();
    CK(hipMemcpy(dB[g], h.data(), sizeof(double) * nb, hipMemcpyHostToDevice));
    for (size_t i = 0; i < nc; ++i) h[i] = rnd();
    CK(hipMemcpy(dC[g], h.data(), sizeof(double) * nc, hipMemcpyHostToDevice));
    CK(hipMemcpy(dC2[g], h.data(), sizeof(double) * nc, hipMemcpyHostToDevice));
    ggemm_problem_t& p = ps[g];
    std::memset(&p, 0, sizeof p);
    p.m = q.m; p.n = q.n; p.k = q.k;
    p.A = dA[g]; p.lda = q.m;
    p.B = dB[g]; p.ldb = q.k > 0 ? q.k : 1;
    p.C = dC[g]; p.ldc = q.m;
    p.alpha = q.alpha; p.beta = q.beta;
    sa += na; sb += nb; sc += nc;
  }
  ggemm_handle_t h = nullptr;
  if (ggemm_create_ex(&h, 16, sa, sb, sc, s, 1) != GGEMM_OK) {
    std::fprintf(stderr, "ggemm_create_ex failed\n");
    return 1;
  }
  ggemm_config_t cfg;
  std::memset(&cfg, 0, sizeof cfg);
  cfg.target_rel_err = 1e-15;
  cfg.allow_fallback = 1;
  cfg.repair_mode = GGEMM_REPAIR_ON;
  ggemm_stats_t st;
  static const char* names[] = {"native_loop", "native_grouped", "emu_loop", "emu_grouped", "auto",
                                "emu_grouped_reuse", "emu_loop_batched"};
  for (int path = 0; path <= 6; ++path)
    if (measure(names[path], s, [&] { return ggemm_grouped_dgemm(h, (ggemm_path_t)path, &cfg, ps.data(), G, &st); }))
      return 1;
  int err = 0;
  ggemm_plan_t plan = ggemm_make_plan_ex(h, GGEMM_PATH_AUTO, &cfg, ps.data(), G, &err);
  if (!plan) {
    std::fprintf(stderr, "ggemm_make_plan_ex failed: %d\n", err);
    return 1;
  }
  if (measure("execute_plan", s, [&] { return ggemm_execute_plan(plan, s); })) return 1;
  int flip = 0;
  if (measure("update_pointers_execute", s, [&] {
        flip ^= 1;
        const int r = ggemm_plan_update_pointers(plan, nullptr, nullptr, flip ? dC2.data() : dC.data());
        return r ? r : ggemm_execute_plan(plan, s);
      }))
    return 1;
  if (measure("plan_get_stats", s, [&] { return ggemm_plan_get_stats(plan, &st); })) return 1;
  ggemm_destroy_plan(plan);
  if (measure("noalloc", s, [&] { return ggemm_grouped_dgemm_noalloc(GGEMM_PATH_AUTO, &cfg, ps.data(), G, s, &st); }))
    return 1;
  ggemm_destroy(h);
  for (int g = 0; g < G; ++g) {
    CK(hipFree(dA[g]));
    CK(hipFree(dB[g]));
    CK(hipFree(dC[g]));
    CK(hipFree(dC2[g]));
  }
  CK(hipStreamDestroy(s));
  return 0;
}

int main(int argc, char** argv) {
  if (argc > 1 && !std::strcmp(argv[1], "gpu")) return gpu_calls();
  return host_planner();
}
