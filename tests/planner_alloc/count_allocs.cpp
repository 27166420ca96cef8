// count_allocs.cpp -- counts the heap allocations made inside ggemm_plan (host only, no GPU).
//
// The reference's planner test (tests/test_planner.cpp:33-50, 429-464) replaces the global
// operator new and requires zero calls inside ggemm_plan after the first call.  This program
// interposes both operator new and the C allocator (malloc / calloc / realloc / aligned forms,
// forwarded to glibc's own entry points) for the whole process, plans a 65535-problem group on the
// AUTO and EMU_GROUPED paths, and prints one line per path:
//   path=<p> first=<allocations in the first call> steady=<allocations in 5 later calls>
// Built and run by tests/test_planner_log.py against the library; TEST INFRASTRUCTURE ONLY.
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

#include "ggemm.h"
#include "ggemm_oz2.h"

extern "C" void* __libc_malloc(size_t);
extern "C" void* __libc_calloc(size_t, size_t);
extern "C" void* __libc_realloc(void*, size_t);
extern "C" void* __libc_memalign(size_t, size_t);
extern "C" void __libc_free(void*);

static std::atomic<long> g_allocs{0};
static std::atomic<bool> g_counting{false};
static inline void note() {
  if (g_counting.load(std::memory_order_relaxed)) g_allocs.fetch_add(1, std::memory_order_relaxed);
}

extern "C" void* malloc(size_t n) { note(); return __libc_malloc(n); }
extern "C" void* calloc(size_t a, size_t b) { note(); return __libc_calloc(a, b); }
extern "C" void* realloc(void* p, size_t n) { note(); return __libc_realloc(p, n); }
extern "C" void* memalign(size_t a, size_t n) { note(); return __libc_memalign(a, n); }
extern "C" void* aligned_alloc(size_t a, size_t n) { note(); return __libc_memalign(a, n); }
extern "C" int posix_memalign(void** out, size_t a, size_t n) {
  note();
  void* p = __libc_memalign(a, n);
  if (!p) return 12;
  *out = p;
  return 0;
}
extern "C" void free(void* p) { __libc_free(p); }

void* operator new(size_t n) {
  note();
  if (void* p = __libc_malloc(n ? n : 1)) return p;
  throw std::bad_alloc();
}
void* operator new[](size_t n) { return operator new(n); }
void* operator new(size_t n, const std::nothrow_t&) noexcept { note(); return __libc_malloc(n ? n : 1); }
void* operator new[](size_t n, const std::nothrow_t&) noexcept { note(); return __libc_malloc(n ? n : 1); }
void operator delete(void* p) noexcept { __libc_free(p); }
void operator delete[](void* p) noexcept { __libc_free(p); }
void operator delete(void* p, size_t) noexcept { __libc_free(p); }
void operator delete[](void* p, size_t) noexcept { __libc_free(p); }

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

int main() {
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
