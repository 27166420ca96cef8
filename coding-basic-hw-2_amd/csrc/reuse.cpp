// reuse.cpp -- operand reuse host pass (include/ggemm_reuse.h), semantics of
// src/operand_reuse.cpp:47-141.
//
// One linear sweep over the problems assigns unique-A / unique-B ids in order of first appearance
// through two open-addressing tables (keys hashed, collisions resolved by comparing the key
// fields of the representative problem).  Table slots carry a generation number, so a build
// starts with an empty table without clearing it.  PROMOTE then joins, for every emulated
// problem, its unique A and unique B in a disjoint-set forest and gives every member of a
// component the component's largest N.  No allocation after the arena is created.
#include <algorithm>
#include <cstdint>
#include <new>
#include <vector>

#include "ggemm_reuse.h"

struct reuse_arena_s {
  int cap = 0;
  uint32_t mask = 0;
  uint32_t gen = 0;
  std::vector<uint32_t> a_gen, b_gen;   // table slot generations
  std::vector<int> a_slot, b_slot;      // unique id stored in a slot
  std::vector<int> ua_rep, ua_nmod, ub_rep, ub_nmod, prob_a, prob_b, eff_nmod;
  std::vector<int> parent, best;        // disjoint sets over [0, cap) unique A, [cap, 2 cap) unique B
};

namespace {

uint64_t fmix(uint64_t x) {   // 64-bit finaliser (MurmurHash3's fmix64)
  x ^= x >> 33;
  x *= 0xff51afd7ed558ccdULL;
  x ^= x >> 33;
  x *= 0xc4ceb9fe1a85ec53ULL;
  x ^= x >> 33;
  return x;
}
uint32_t slot_of(const void* ptr, int ld, int rows, int k, int extra, uint32_t mask) {
  uint64_t h = fmix(reinterpret_cast<uintptr_t>(ptr));
  h = fmix(h ^ (((uint64_t)(uint32_t)ld << 32) | (uint32_t)rows));
  h = fmix(h ^ (((uint64_t)(uint32_t)k << 32) | (uint32_t)extra));
  return (uint32_t)h & mask;
}
int root(int* parent, int x) {
  while (parent[x] != x) {
    parent[x] = parent[parent[x]];
    x = parent[x];
  }
  return x;
}

// The unique operand of problem g on one side (A: is_a), or -1 - slot of the free table slot
// where it is to be inserted.
int lookup(reuse_arena_s& w, const ggemm_problem_t* probs, int g, bool is_a, int N, bool exact) {
  const ggemm_problem_t& p = probs[g];
  const void* ptr = is_a ? (const void*)p.A : (const void*)p.B;
  const int ld = is_a ? p.lda : p.ldb, rows = is_a ? p.m : p.n;
  const std::vector<uint32_t>& gens = is_a ? w.a_gen : w.b_gen;
  const std::vector<int>& slots = is_a ? w.a_slot : w.b_slot;
  const std::vector<int>& rep = is_a ? w.ua_rep : w.ub_rep;
  const std::vector<int>& nmod = is_a ? w.ua_nmod : w.ub_nmod;
  for (uint32_t s = slot_of(ptr, ld, rows, p.k, (exact ? N : 0) ^ (is_a ? 0 : 0x2545F491), w.mask);;
       s = (s + 1) & w.mask) {
    if (gens[s] != w.gen) return -1 - (int)s;   // free slot: caller inserts
    const int id = slots[s];
    const ggemm_problem_t& q = probs[rep[id]];
    const bool same = is_a ? (q.A == p.A && q.lda == p.lda && q.m == p.m && q.k == p.k)
                           : (q.B == p.B && q.ldb == p.ldb && q.n == p.n && q.k == p.k);
    if (same && (!exact || nmod[id] == N)) return id;
  }
}

}  // namespace

extern "C" int reuse_arena_create(int max_problems, reuse_arena_t* out) {
  if (!out) return REUSE_ERR_INVALID;
  reuse_arena_s* w = new (std::nothrow) reuse_arena_s();
  *out = w;
  if (!w) return REUSE_ERR_INVALID;
  if (max_problems < 1) max_problems = 1;
  if (max_problems > (1 << 30)) return REUSE_ERR_CAPACITY;   // table of 2 cap slots must fit 32 bits
  uint32_t size = 2;
  while (size < 2u * (uint32_t)max_problems) size <<= 1;
  try {
    w->a_gen.assign(size, 0u);
    w->b_gen.assign(size, 0u);
    w->a_slot.assign(size, -1);
    w->b_slot.assign(size, -1);
    for (auto* v : {&w->ua_rep, &w->ua_nmod, &w->ub_rep, &w->ub_nmod, &w->prob_a, &w->prob_b, &w->eff_nmod})
      v->assign(max_problems, 0);
    w->parent.assign(2 * (size_t)max_problems, 0);
    w->best.assign(2 * (size_t)max_problems, 0);
  } catch (...) {
    *w = reuse_arena_s();
    return REUSE_ERR_CAPACITY;
  }
  w->cap = max_problems;
  w->mask = size - 1;
  return REUSE_OK;
}

extern "C" void reuse_arena_destroy(reuse_arena_t a) { delete a; }

extern "C" int reuse_arena_capacity(reuse_arena_t a) { return a ? a->cap : 0; }

extern "C" reuse_plan build_operand_reuse(reuse_arena_t a, const ggemm_problem_t* probs, int num, const int* nmod,
                                          int policy) {
  reuse_plan r{};
  r.num_problems = num;
  if (!a || num < 0 || (num > 0 && (!probs || !nmod)) || (policy != REUSE_EXACT_N && policy != REUSE_PROMOTE)) {
    r.status = REUSE_ERR_INVALID;
    return r;
  }
  reuse_arena_s& w = *a;
  if (num > w.cap) {
    r.status = REUSE_ERR_CAPACITY;
    return r;
  }
  if (++w.gen == 0) {   // generation wrap: clear the tables once
    std::fill(w.a_gen.begin(), w.a_gen.end(), 0u);
    std::fill(w.b_gen.begin(), w.b_gen.end(), 0u);
    w.gen = 1;
  }
  const bool exact = policy == REUSE_EXACT_N;
  int nua = 0, nub = 0, nemu = 0;
  for (int g = 0; g < num; ++g) {
    const int N = nmod[g];
    if (N <= 0) {
      w.prob_a[g] = w.prob_b[g] = -1;
      w.eff_nmod[g] = 0;
      continue;
    }
    ++nemu;
    for (int side = 0; side < 2; ++side) {
      const bool is_a = side == 0;
      int id = lookup(w, probs, g, is_a, N, exact);
      std::vector<int>& rep = is_a ? w.ua_rep : w.ub_rep;
      std::vector<int>& nm = is_a ? w.ua_nmod : w.ub_nmod;
      if (id < 0) {   // new unique operand in the free slot
        const uint32_t s = (uint32_t)(-1 - id);
        id = is_a ? nua++ : nub++;
        (is_a ? w.a_gen : w.b_gen)[s] = w.gen;
        (is_a ? w.a_slot : w.b_slot)[s] = id;
        rep[id] = g;
        nm[id] = N;
      } else {
        nm[id] = std::max(nm[id], N);
      }
      (is_a ? w.prob_a : w.prob_b)[g] = id;
    }
    w.eff_nmod[g] = N;
  }
  int promoted = 0;
  if (!exact && nemu > 0) {
    int* parent = w.parent.data();
    int* best = w.best.data();
    const int ob = w.cap;
    for (int u = 0; u < nua; ++u) { parent[u] = u; best[u] = w.ua_nmod[u]; }
    for (int u = 0; u < nub; ++u) { parent[ob + u] = ob + u; best[ob + u] = w.ub_nmod[u]; }
    for (int g = 0; g < num; ++g) {
      if (w.prob_a[g] < 0) continue;
      const int x = root(parent, w.prob_a[g]), y = root(parent, ob + w.prob_b[g]);
      if (x == y) continue;
      const int lo = std::min(x, y), hi = std::max(x, y);
      parent[hi] = lo;
      best[lo] = std::max(best[lo], best[hi]);
    }
    for (int u = 0; u < nua; ++u) w.ua_nmod[u] = best[root(parent, u)];
    for (int u = 0; u < nub; ++u) w.ub_nmod[u] = best[root(parent, ob + u)];
    for (int g = 0; g < num; ++g) {
      if (w.prob_a[g] < 0) continue;
      const int N = w.ua_nmod[w.prob_a[g]];
      promoted += N > w.eff_nmod[g];
      w.eff_nmod[g] = N;
    }
  }
  r.status = REUSE_OK;
  r.num_ua = nua;
  r.num_ub = nub;
  r.num_emu = nemu;
  r.num_promoted = promoted;
  r.ua_rep = w.ua_rep.data();
  r.ua_nmod = w.ua_nmod.data();
  r.ub_rep = w.ub_rep.data();
  r.ub_nmod = w.ub_nmod.data();
  r.prob_a = w.prob_a.data();
  r.prob_b = w.prob_b.data();
  r.eff_nmod = w.eff_nmod.data();
  return r;
}

namespace {
double kp_d(int k) { return (double)(((size_t)k + 31) / 32 * 32); }
double align256(double x) { return (double)(((size_t)x + 255) / 256 * 256); }
}  // namespace

// src/operand_reuse.cpp:143-186 (the modelled-bytes formulas of src/operand_reuse.h:76-82)
extern "C" void operand_reuse_bytes(const reuse_plan* plan, const ggemm_problem_t* probs, const int* nmod,
                                    reuse_bytes* before, reuse_bytes* after) {
  reuse_bytes b{}, t{};
  if (!plan || plan->status != REUSE_OK || (plan->num_problems > 0 && (!probs || !nmod))) {
    if (before) *before = b;
    if (after) *after = t;
    return;
  }
  int nb = 0;
  double sa = 0, sb = 0;
  for (int g = 0; g < plan->num_problems; ++g) {
    if (nmod[g] <= 0) continue;
    const ggemm_problem_t& p = probs[g];
    const double kp = kp_d(p.k), m = p.m, n = p.n, k = p.k;
    b.prep_read += 16.0 * (m * k + k * n);
    b.prep_write += nmod[g] * kp * (m + n) + 4.0 * (m + n);
    sa += align256(m * kp);
    sb += align256(n * kp);
    nb = std::max(nb, nmod[g]);
  }
  b.ws_A8 = nb * sa;
  b.ws_B8 = nb * sb;
  int na = 0;
  sa = sb = 0;
  for (int u = 0; u < plan->num_ua; ++u) {
    const ggemm_problem_t& p = probs[plan->ua_rep[u]];
    const double kp = kp_d(p.k), m = p.m, k = p.k;
    t.prep_read += 16.0 * m * k;
    t.prep_write += plan->ua_nmod[u] * kp * m + 4.0 * m;
    sa += align256(m * kp);
    na = std::max(na, plan->ua_nmod[u]);
  }
  for (int u = 0; u < plan->num_ub; ++u) {
    const ggemm_problem_t& p = probs[plan->ub_rep[u]];
    const double kp = kp_d(p.k), n = p.n, k = p.k;
    t.prep_read += 16.0 * k * n;
    t.prep_write += plan->ub_nmod[u] * kp * n + 4.0 * n;
    sb += align256(n * kp);
    na = std::max(na, plan->ub_nmod[u]);
  }
  t.ws_A8 = na * sa;
  t.ws_B8 = na * sb;
  if (before) *before = b;
  if (after) *after = t;
}
