// i8gemm.hip -- grouped INT8 x INT8 -> INT32 GEMM on gfx950 MFMA (exact accumulation).
//
// Problem (src/int8_grouped_gemm.h:4-10 layout): A m x kp and B n x kp row-major (K contiguous),
// C = A B^T column-major m x n (ld m), kp % 32 == 0, |C| <= 128^2 kp < 2^31 (kp <= 131040).
//
// One launch covers every (problem, plane) of a group.  The host builds a tile table in
// longest-processing-time order (heaviest tiles first, the reference's scheduling contract,
// src/int8_grouped_gemm.cu:602-675).  Workgroup b takes one tile:
//   * XCD-aware dispatch: MI355X deals workgroups round-robin to its 8 XCDs (b mod 8), each with
//     its own L2.  Workgroup b is mapped to tile chunk (b mod 8) + 8 (b / (8 C)) of C = 32
//     consecutive table tiles, so one XCD works through contiguous runs of the table;
//   * inside an entry tiles are rastered in groups of 8 tile-rows (8 x 4 blocks of 32 tiles),
//     so the 32 compute units of an XCD share 8 A panels and 4 B panels.
// Tile configurations, 512 threads = 8 waves in a 2 (M) x 4 (N) arrangement:
//   cfg 0: 256 x 256, BK  64   wave tile 128 x 64 = 8 x 4 blocks of v_mfma_i32_16x16x64_i8
//   cfg 1: 128 x 128, BK 128   wave tile  64 x 32 = 4 x 2 blocks
//   cfg 2:  64 x  64, BK 256   wave tile  32 x 16 = 2 x 1 blocks
// Every stage moves 32 KB (2 x 16 B per thread per operand).  Operands go HBM -> VGPR -> LDS;
// the VGPR staging is double-buffered so global loads are issued two k-stages ahead of their use,
// LDS is double-buffered (one barrier per stage).  LDS rows hold BK bytes with the 16-byte chunk
// index XOR-swizzled by the row, so the 16-lane groups of each ds_read_b128 fragment load hit
// distinct banks.  Rows >= m / n and k >= kp are zero-filled (kp % 32 == 0: every 16-byte chunk
// is wholly inside or outside), k steps wholly beyond kp are skipped.
// Epilogue, per problem: int32 C (the reference contract, used by the kernel-level API and the
// abs plane), or -- in the production pipeline -- the CRT residue byte
// y = ((C mod p) q) mod p of the plane's modulus p and CRT inverse q, which is all the
// reconstruction needs from a residue plane; this cuts the plane write from 4 to 1 byte.
#include <algorithm>
#include <cstring>
#include <mutex>
#include <vector>

#include "common.hpp"

namespace ggemm {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kThreads = 512;
constexpr int kChunk = 32;   // tiles per XCD chunk
constexpr int kXcds = 8;
constexpr int kGroupM = 8;   // tile-rows per raster group

template <int BM_, int BN_, int BK_>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_;
  static constexpr int WM = BM / 2, WN = BN / 4;     // wave tile (2 x 4 waves)
  static constexpr int FM = WM / 16, FN = WN / 16;   // 16 x 16 MFMA blocks per wave
  static constexpr int CPR = BK / 16;                // 16-byte chunks per LDS row
  static constexpr int LA = BM * CPR / kThreads;     // chunks per thread per stage
  static constexpr int LB = BN * CPR / kThreads;
  static constexpr int STAGE = (BM + BN) * BK;
  static_assert(BM * CPR % kThreads == 0 && BN * CPR % kThreads == 0, "chunk split");
  static_assert(FM >= 1 && FN >= 1, "wave tile");
};
using Cfg0 = Cfg<256, 256, 64>;
using Cfg1 = Cfg<128, 128, 128>;
using Cfg2 = Cfg<64, 64, 256>;
constexpr int kSmem = 2 * Cfg0::STAGE;   // 64 KB
static_assert(2 * Cfg1::STAGE <= kSmem && 2 * Cfg2::STAGE <= kSmem, "smem");

template <int CPR>
__device__ __forceinline__ int swz(int row, int ch) {
  if constexpr (CPR == 4) return ch ^ ((row >> 1) & 3);
  else return ch ^ (row & 7);
}

template <class C>
struct Stage {
  uint4 a[C::LA], b[C::LB];
};

template <class C>
__device__ __forceinline__ void load_global(Stage<C>& s, const int8_t* A, const int8_t* B, int m_rem, int n_rem,
                                            int kp, int k0, int tid) {
#pragma unroll
  for (int q = 0; q < C::LA; ++q) {
    const int c = tid + q * kThreads, row = c / C::CPR, ch = c % C::CPR;
    const int kk = k0 + ch * 16;
    s.a[q] = (row < m_rem && kk < kp) ? *reinterpret_cast<const uint4*>(A + (size_t)row * kp + kk)
                                      : make_uint4(0u, 0u, 0u, 0u);
  }
#pragma unroll
  for (int q = 0; q < C::LB; ++q) {
    const int c = tid + q * kThreads, row = c / C::CPR, ch = c % C::CPR;
    const int kk = k0 + ch * 16;
    s.b[q] = (row < n_rem && kk < kp) ? *reinterpret_cast<const uint4*>(B + (size_t)row * kp + kk)
                                      : make_uint4(0u, 0u, 0u, 0u);
  }
}

template <class C>
__device__ __forceinline__ void store_lds(int8_t* st, const Stage<C>& s, int tid) {
  int8_t* sA = st;
  int8_t* sB = st + C::BM * C::BK;
#pragma unroll
  for (int q = 0; q < C::LA; ++q) {
    const int c = tid + q * kThreads, row = c / C::CPR, ch = c % C::CPR;
    *reinterpret_cast<uint4*>(sA + row * C::BK + swz<C::CPR>(row, ch) * 16) = s.a[q];
  }
#pragma unroll
  for (int q = 0; q < C::LB; ++q) {
    const int c = tid + q * kThreads, row = c / C::CPR, ch = c % C::CPR;
    *reinterpret_cast<uint4*>(sB + row * C::BK + swz<C::CPR>(row, ch) * 16) = s.b[q];
  }
}

template <class C>
__device__ __forceinline__ void mma_stage(const int8_t* st, int k0, int kp, int wm, int wn, int lane,
                                          v4i (&acc)[C::FM][C::FN]) {
  const int8_t* sA = st;
  const int8_t* sB = st + C::BM * C::BK;
  const int frow = lane & 15, fch = lane >> 4;
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
}

__device__ __forceinline__ uint32_t mod_small(uint32_t u, uint32_t p, uint32_t magic) {
  uint32_t r = u - __umulhi(u, magic) * p;   // magic = floor(2^32/p): quotient low by at most 1
  r = r >= p ? r - p : r;
  return r >= p ? r - p : r;
}
__device__ __forceinline__ uint32_t crt_digit(int32_t c, const I8Epi& e) {
  const uint32_t uc = c < 0 ? 0u - (uint32_t)c : (uint32_t)c;
  uint32_t r = mod_small(uc, e.p, e.magic);
  if (c < 0 && r) r = e.p - r;
  return mod_small(r * e.q, e.p, e.magic);
}

template <class C>
__device__ __forceinline__ void run_tile(int8_t* smem, const i8_problem& P, const I8Epi& epi, int tm, int tn) {
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

  Stage<C> s0, s1;
  load_global<C>(s0, A, B, m_rem, n_rem, kp, 0, tid);
  if (nk > 1) load_global<C>(s1, A, B, m_rem, n_rem, kp, C::BK, tid);
  store_lds<C>(smem, s0, tid);
  __syncthreads();
  // two k-stages per trip so that the staging set index is static: stage kt lives in LDS buffer
  // kt & 1; its successor kt + 1 is in staging set (kt + 1) & 1; loads for kt + 2 reuse set kt & 1.
  for (int kt = 0; kt < nk; kt += 2) {
    if (kt + 2 < nk) load_global<C>(s0, A, B, m_rem, n_rem, kp, (kt + 2) * C::BK, tid);
    mma_stage<C>(smem, kt * C::BK, kp, wm, wn, lane, acc);
    if (kt + 1 < nk) store_lds<C>(smem + C::STAGE, s1, tid);
    __syncthreads();
    if (kt + 1 >= nk) break;
    if (kt + 3 < nk) load_global<C>(s1, A, B, m_rem, n_rem, kp, (kt + 3) * C::BK, tid);
    mma_stage<C>(smem + C::STAGE, (kt + 1) * C::BK, kp, wm, wn, lane, acc);
    if (kt + 2 < nk) store_lds<C>(smem, s0, tid);
    __syncthreads();
  }

  // D block layout: lane l, register r -> row 4 (l / 16) + r, column l % 16; a lane's 4 values
  // are 4 consecutive rows of one column, i.e. contiguous in the column-major output.
  const size_t ldc = (size_t)P.m;
  const bool vec = (P.m % 4 == 0) && ((reinterpret_cast<uintptr_t>(P.C) & (epi.mode ? 3 : 15)) == 0);
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
      const int col = col0 + wn * C::WN + j * 16 + (lane & 15);
      const int r0 = row0 + wm * C::WM + i * 16 + 4 * (lane >> 4);
      if (col >= P.n || r0 >= P.m) continue;
      const v4i v = acc[i][j];
      if (epi.mode == 0) {
        int32_t* out = reinterpret_cast<int32_t*>(P.C) + (size_t)r0 + (size_t)col * ldc;
        if (vec && r0 + 3 < P.m) {
          *reinterpret_cast<v4i*>(out) = v;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (r0 + r < P.m) out[r] = v[r];
        }
      } else {
        uint8_t* out = reinterpret_cast<uint8_t*>(P.C) + (size_t)r0 + (size_t)col * ldc;
        uint32_t y[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] = crt_digit(v[r], epi);
        if (vec && r0 + 3 < P.m) {
          *reinterpret_cast<uint32_t*>(out) = y[0] | (y[1] << 8) | (y[2] << 16) | (y[3] << 24);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (r0 + r < P.m) out[r] = (uint8_t)y[r];
        }
      }
    }
}

__global__ void __launch_bounds__(kThreads) i8_grouped_kernel(const i8_problem* __restrict__ probs,
                                                              const I8Epi* __restrict__ epis,
                                                              const int* __restrict__ sched) {
  extern __shared__ __align__(16) int8_t smem[];
  const int total = sched[0];
  const int ne = sched[1];
  // XCD-aware remap of the dispatch index (a permutation of [0, total))
  const int b = blockIdx.x;
  const int span = kXcds * kChunk;
  const int full = total / span * span;
  int tile = b;
  if (b < full) {
    const int x = b % kXcds, q = b / kXcds;
    tile = (q / kChunk) * span + x * kChunk + (q % kChunk);
  }
  const int* prefix = sched + kSchedHdr;
  const int* entry = prefix + ne + 1;
  int lo = 0, hi = ne - 1;   // largest e with prefix[e] <= tile
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (prefix[mid] <= tile) lo = mid; else hi = mid - 1;
  }
  const int e = entry[lo];
  const int cfg = e & 3, pi = e >> 2;
  const int local = tile - prefix[lo];
  const i8_problem P = probs[pi];
  I8Epi epi{0u, 1u, 0u, 0u};
  if (epis) epi = epis[pi];
  const int edge = cfg == 0 ? 256 : (cfg == 1 ? 128 : 64);
  const int tiles_m = (P.m + edge - 1) / edge, tiles_n = (P.n + edge - 1) / edge;
  // grouped raster: blocks of kGroupM tile-rows, m fastest inside a block
  const int per_group = kGroupM * tiles_n;
  const int g = local / per_group, first_m = g * kGroupM;
  const int gsz = min(kGroupM, tiles_m - first_m);
  const int r = local - g * per_group;
  const int tm = first_m + r % gsz, tn = r / gsz;
  switch (cfg) {
    case 0: run_tile<Cfg0>(smem, P, epi, tm, tn); break;
    case 1: run_tile<Cfg1>(smem, P, epi, tm, tn); break;
    default: run_tile<Cfg2>(smem, P, epi, tm, tn); break;
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
// Automatic tile: least padded work per unit efficiency (relative efficiencies 1, 0.7, 0.35).
int auto_cfg(int m, int n) {
  static const double eff[3] = {1.0, 0.7, 0.35};
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
  // group-level fill: fewer tiles than compute units -> shrink automatic tiles one step
  for (int pass = 0; pass < 2; ++pass) {
    long long t = 0;
    for (auto& e : ents) t += e.tiles;
    if (t >= num_cus) break;
    for (auto& e : ents)
      if (e.cfg < kI8NumCfg - 1 && h[e.prob].tile_cfg < 0) {
        ++e.cfg;
        const double b = i8_tile_edge(e.cfg);
        e.tiles = tiles_of(e.cfg, h[e.prob].m, h[e.prob].n);
        e.cost = b * b * (double)(h[e.prob].kp + 128);
      }
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

int i8_launch(const i8_problem* d_probs, const I8Epi* d_epi, const void* d_sched, const i8_sched_info* info,
              hipStream_t s) {
  if (!info) return 1;
  if (info->num_launches == 0 || info->tiles_main == 0) return 0;
  if (!d_probs || !d_sched) return 1;
  hipLaunchKernelGGL(i8_grouped_kernel, dim3((unsigned)info->tiles_main), dim3(kThreads), kSmem, s, d_probs, d_epi,
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
  return i8_launch(d_probs, nullptr, d_sched_ws, info, s);
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
  rc = i8_launch(d_probs, nullptr, d_sched_ws, &info, s);
  if (!rc && num_launches) *num_launches = info.num_launches;
  return rc;
}
