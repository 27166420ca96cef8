// i8gemm.hip -- grouped INT8 x INT8 -> INT32 GEMM on gfx950 MFMA (exact accumulation).
//
// Problem (src/int8_grouped_gemm.h:4-10 layout): A m x kp and B n x kp row-major (K contiguous),
// C = A B^T column-major m x n (ld m), kp % 32 == 0, |C| <= 128^2 kp < 2^31 (kp <= 131040).
//
// One launch covers every (problem, plane) of the group.  The host builds a tile table in
// longest-processing-time order (heaviest tiles first, src/int8_grouped_gemm.cu:602-675 semantics);
// workgroup b takes tile b, finds its entry by binary search over the prefix table, and rasters
// the entry's tiles m-fastest so that neighbouring workgroups share the B panel.
// Tile configurations (256 threads = 4 waves in a 2 x 2 arrangement):
//   cfg 0: 128 x 128, BK 128   wave tile 64 x 64 = 4 x 4 MFMA blocks
//   cfg 1:  64 x  64, BK 128   wave tile 32 x 32 = 2 x 2
//   cfg 2:  32 x  32, BK 256   wave tile 16 x 16 = 1 x 1
// Each 64-deep k step is one v_mfma_i32_16x16x64_i8 per 16 x 16 block.  Operands go
// HBM -> VGPR -> LDS with 128-bit accesses, double-buffered (one barrier per BK step); LDS rows
// hold BK bytes with the 16-byte chunk index XOR-swizzled by the row so that the 16-lane groups of
// a ds_read_b128 fragment load hit distinct banks.  Rows >= m / n and k >= kp are zero-filled
// (kp % 32 == 0, so every 16-byte chunk is wholly inside or outside), k steps wholly beyond kp
// are skipped, and the epilogue store is predicated.
#include <algorithm>
#include <cstring>
#include <mutex>
#include <vector>

#include "common.hpp"

namespace ggemm {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;

template <int BM_, int BN_, int BK_>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_;
  static constexpr int WM = BM / 2, WN = BN / 2;     // wave tile
  static constexpr int FM = WM / 16, FN = WN / 16;   // 16 x 16 MFMA blocks per wave
  static constexpr int CPR = BK / 16;                // 16-byte chunks per LDS row
  static constexpr int LA = BM * CPR / kThreads;     // chunks per thread per stage
  static constexpr int LB = BN * CPR / kThreads;
  static constexpr int STAGE = (BM + BN) * BK;
  static_assert(BM * CPR % kThreads == 0 && BN * CPR % kThreads == 0, "chunk split");
  static_assert(FM >= 1 && FN >= 1, "wave tile");
};
using Cfg0 = Cfg<128, 128, 128>;
using Cfg1 = Cfg<64, 64, 128>;
using Cfg2 = Cfg<32, 32, 256>;
constexpr int kSmem = 2 * Cfg0::STAGE;   // 64 KB: the largest double-buffered stage pair
static_assert(2 * Cfg1::STAGE <= kSmem && 2 * Cfg2::STAGE <= kSmem, "smem");

template <int CPR>
__device__ __forceinline__ int swz(int row, int ch) {
  return ch ^ (row & (CPR - 1) & 7);
}

template <class C>
__device__ __forceinline__ void load_global(uint4 (&ra)[C::LA], uint4 (&rb)[C::LB], const int8_t* A, const int8_t* B,
                                            int m_rem, int n_rem, int kp, int k0, int tid) {
#pragma unroll
  for (int q = 0; q < C::LA; ++q) {
    const int c = tid + q * kThreads, row = c / C::CPR, ch = c % C::CPR;
    const int kk = k0 + ch * 16;
    ra[q] = (row < m_rem && kk < kp) ? *reinterpret_cast<const uint4*>(A + (size_t)row * kp + kk)
                                     : make_uint4(0u, 0u, 0u, 0u);
  }
#pragma unroll
  for (int q = 0; q < C::LB; ++q) {
    const int c = tid + q * kThreads, row = c / C::CPR, ch = c % C::CPR;
    const int kk = k0 + ch * 16;
    rb[q] = (row < n_rem && kk < kp) ? *reinterpret_cast<const uint4*>(B + (size_t)row * kp + kk)
                                     : make_uint4(0u, 0u, 0u, 0u);
  }
}

template <class C>
__device__ __forceinline__ void store_lds(int8_t* st, const uint4 (&ra)[C::LA], const uint4 (&rb)[C::LB], int tid) {
  int8_t* sA = st;
  int8_t* sB = st + C::BM * C::BK;
#pragma unroll
  for (int q = 0; q < C::LA; ++q) {
    const int c = tid + q * kThreads, row = c / C::CPR, ch = c % C::CPR;
    *reinterpret_cast<uint4*>(sA + row * C::BK + swz<C::CPR>(row, ch) * 16) = ra[q];
  }
#pragma unroll
  for (int q = 0; q < C::LB; ++q) {
    const int c = tid + q * kThreads, row = c / C::CPR, ch = c % C::CPR;
    *reinterpret_cast<uint4*>(sB + row * C::BK + swz<C::CPR>(row, ch) * 16) = rb[q];
  }
}

template <class C>
__device__ __forceinline__ void run_tile(int8_t* smem, const i8_problem& P, int tm, int tn) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int row0 = tm * C::BM, col0 = tn * C::BN;
  const int m_rem = P.m - row0, n_rem = P.n - col0;
  const int kp = P.kp;
  const int8_t* A = P.A + (size_t)row0 * kp;
  const int8_t* B = P.B + (size_t)col0 * kp;
  const int nk = (kp + C::BK - 1) / C::BK;

  v4i acc[C::FM][C::FN];
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  uint4 ra[C::LA], rb[C::LB];
  load_global<C>(ra, rb, A, B, m_rem, n_rem, kp, 0, tid);
  store_lds<C>(smem, ra, rb, tid);
  __syncthreads();

  const int frow = lane & 15, fch = lane >> 4;   // fragment row within a block, chunk within a k step
  for (int kt = 0; kt < nk; ++kt) {
    const int k0 = kt * C::BK;
    if (kt + 1 < nk) load_global<C>(ra, rb, A, B, m_rem, n_rem, kp, k0 + C::BK, tid);
    const int8_t* sA = smem + (kt & 1) * C::STAGE;
    const int8_t* sB = sA + C::BM * C::BK;
#pragma unroll
    for (int ks = 0; ks < C::BK / 64; ++ks) {
      if (k0 + ks * 64 >= kp) break;   // block-uniform
      const int ch = ks * 4 + fch;
      v4i a[C::FM], b[C::FN];
#pragma unroll
      for (int i = 0; i < C::FM; ++i) {
        const int row = wm * C::WM + i * 16 + frow;
        a[i] = *reinterpret_cast<const v4i*>(sA + row * C::BK + swz<C::CPR>(row, ch) * 16);
      }
#pragma unroll
      for (int j = 0; j < C::FN; ++j) {
        const int row = wn * C::WN + j * 16 + frow;
        b[j] = *reinterpret_cast<const v4i*>(sB + row * C::BK + swz<C::CPR>(row, ch) * 16);
      }
#pragma unroll
      for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store_lds<C>(smem + ((kt + 1) & 1) * C::STAGE, ra, rb, tid);
    __syncthreads();
  }

  // D block layout: lane l, register r -> row 4 (l / 16) + r, column l % 16
  int32_t* Cout = P.C;
  const size_t ldc = (size_t)P.m;
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
      const int col = col0 + wn * C::WN + j * 16 + (lane & 15);
      const int rb0 = row0 + wm * C::WM + i * 16 + 4 * (lane >> 4);
      if (col < P.n) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (rb0 + r < P.m) Cout[(size_t)(rb0 + r) + (size_t)col * ldc] = acc[i][j][r];
      }
    }
}

__global__ void __launch_bounds__(kThreads) i8_grouped_kernel(const i8_problem* __restrict__ probs,
                                                              const int* __restrict__ sched) {
  extern __shared__ __align__(16) int8_t smem[];
  const int tile = blockIdx.x;
  const int ne = sched[1];
  const int* prefix = sched + kSchedHdr;
  const int* entry = prefix + ne + 1;
  int lo = 0, hi = ne - 1;   // largest e with prefix[e] <= tile
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (prefix[mid] <= tile) lo = mid; else hi = mid - 1;
  }
  const int e = entry[lo];
  const int cfg = e & 3;
  const int local = tile - prefix[lo];
  const i8_problem P = probs[e >> 2];
  const int edge = cfg == 0 ? 128 : (cfg == 1 ? 64 : 32);
  const int tiles_m = (P.m + edge - 1) / edge;
  const int tm = local % tiles_m, tn = local / tiles_m;
  switch (cfg) {
    case 0: run_tile<Cfg0>(smem, P, tm, tn); break;
    case 1: run_tile<Cfg1>(smem, P, tm, tn); break;
    default: run_tile<Cfg2>(smem, P, tm, tn); break;
  }
}

// ----------------------------------------------------------------------------- host side
struct Ent {
  double cost;
  int tiles, prob, cfg;
};
std::mutex g_mu;
std::vector<Ent> g_ents;

bool valid_problem(const i8_problem& p) {
  if (p.m < 0 || p.n < 0 || p.kp < 0 || (p.kp % 32) != 0 || p.kp > OZ2_MAX_K) return false;
  if (p.m == 0 || p.n == 0 || p.kp == 0) return true;
  if (!p.A || !p.B || !p.C) return false;
  if ((reinterpret_cast<uintptr_t>(p.A) & 15) || (reinterpret_cast<uintptr_t>(p.B) & 15)) return false;
  return (reinterpret_cast<uintptr_t>(p.C) & 3) == 0;
}
int tiles_of(int cfg, int m, int n) {
  const int e = i8_tile_edge(cfg);
  return ((m + e - 1) / e) * ((n + e - 1) / e);
}
// Automatic tile: least padded work per unit efficiency (relative efficiencies 1, 0.63, 0.30).
int auto_cfg(int m, int n) {
  static const double eff[3] = {1.0, 0.63, 0.30};
  int best = 0;
  double best_cost = 1e300;
  for (int c = 0; c < kI8NumCfg; ++c) {
    const double b = i8_tile_edge(c);
    const double cost = tiles_of(c, m, n) * b * b / eff[c];
    if (cost < best_cost) { best_cost = cost; best = c; }
  }
  return best;
}

}  // namespace

int i8_build_schedule(const i8_problem* h, int num, void* h_ws, size_t ws_bytes, i8_sched_info* info, int num_cus) {
  if (num < 0 || (num > 0 && !h) || !h_ws || !info) return 1;
  if (ws_bytes < sched_bytes(num)) return 2;
  std::lock_guard<std::mutex> lk(g_mu);
  std::vector<Ent>& ents = g_ents;
  ents.clear();
  for (int i = 0; i < num; ++i) {
    if (!valid_problem(h[i])) return 3;
    if (h[i].m == 0 || h[i].n == 0 || h[i].kp == 0) continue;
    int c = h[i].tile_cfg;
    if (c < 0) c = auto_cfg(h[i].m, h[i].n);
    if (c >= kI8NumCfg) c = kI8NumCfg - 1;
    const double b = i8_tile_edge(c);
    ents.push_back({b * b * (double)(h[i].kp + 128), tiles_of(c, h[i].m, h[i].n), i, c});
  }
  // group-level fill: fewer tiles than CUs -> automatic 128-edge problems drop to 64
  long long t = 0;
  for (auto& e : ents) t += e.tiles;
  if (t < num_cus)
    for (auto& e : ents)
      if (e.cfg == 0 && h[e.prob].tile_cfg < 0) {
        e.cfg = 1;
        e.tiles = tiles_of(1, h[e.prob].m, h[e.prob].n);
        e.cost = 64.0 * 64.0 * (double)(h[e.prob].kp + 128);
      }
  std::stable_sort(ents.begin(), ents.end(), [](const Ent& a, const Ent& b) {
    if (a.cost != b.cost) return a.cost > b.cost;
    return a.tiles > b.tiles;
  });
  int* img = static_cast<int*>(h_ws);
  const size_t ne = ents.size();
  int* prefix = img + kSchedHdr;
  int* entry = prefix + ne + 1;
  long long tot = 0;
  for (size_t j = 0; j < ne; ++j) {
    prefix[j] = (int)tot;
    tot += ents[j].tiles;
    entry[j] = (ents[j].prob << 2) | ents[j].cfg;
  }
  prefix[ne] = (int)tot;
  if (tot > 0x7fffffffLL - 1000000) return 5;
  std::memset(img, 0, sizeof(int) * kSchedHdr);
  img[0] = (int)tot;
  img[1] = (int)ne;
  info->tiles_main = (int)tot;
  info->tiles_splitk = 0;
  info->num_launches = tot > 0 ? 1 : 0;
  info->ws2_offset_ints = 0;
  info->bytes_used = sizeof(int) * (kSchedHdr + 2 * ne + 1);
  return 0;
}

int i8_launch(const i8_problem* d_probs, const void* d_sched, const i8_sched_info* info, hipStream_t s) {
  if (!info) return 1;
  if (info->num_launches == 0 || info->tiles_main == 0) return 0;
  if (!d_probs || !d_sched) return 1;
  hipLaunchKernelGGL(i8_grouped_kernel, dim3((unsigned)info->tiles_main), dim3(kThreads), kSmem, s, d_probs,
                     static_cast<const int*>(d_sched));
  return hipGetLastError() == hipSuccess ? 0 : 6;
}

}  // namespace ggemm

using namespace ggemm;

extern "C" size_t i8_grouped_gemm_sched_ws_bytes(int max_problems, size_t) {
  return sched_bytes(max_problems < 0 ? 0 : max_problems);
}

extern "C" int i8_grouped_gemm_build_schedule(const i8_problem* h_probs, int num, void* h_ws, size_t ws_bytes,
                                              i8_sched_info* info) {
  DevCtx* c = dev_ctx();
  return i8_build_schedule(h_probs, num, h_ws, ws_bytes, info, c ? c->num_cus : 256);
}

extern "C" int i8_grouped_gemm_launch(const i8_problem* d_probs, int, const void* d_sched_ws,
                                      const i8_sched_info* info, hipStream_t s) {
  return i8_launch(d_probs, d_sched_ws, info, s);
}

extern "C" int i8_grouped_gemm_ex(const i8_problem* d_probs, int num, const i8_problem* h_probs, void* d_sched_ws,
                                  size_t sched_ws_bytes, hipStream_t s, int* num_launches) {
  if (num_launches) *num_launches = 0;
  if (num == 0) return 0;
  if (!d_sched_ws) return 1;
  const size_t need = sched_bytes(num);
  if (need > sched_ws_bytes) return 2;
  std::vector<int> img(need / sizeof(int) + 1);
  i8_sched_info info;
  int rc = i8_grouped_gemm_build_schedule(h_probs, num, img.data(), need, &info);
  if (rc) return rc;
  if (info.num_launches == 0) return 0;
  if (hipMemcpyAsync(d_sched_ws, img.data(), info.bytes_used, hipMemcpyHostToDevice, s) != hipSuccess) return 7;
  // the pageable source must stay valid until the copy has consumed it
  if (hipStreamSynchronize(s) != hipSuccess) return 7;
  rc = i8_launch(d_probs, d_sched_ws, &info, s);
  if (!rc && num_launches) *num_launches = info.num_launches;
  return rc;
}
