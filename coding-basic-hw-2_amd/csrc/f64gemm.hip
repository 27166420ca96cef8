// f64gemm.hip -- grouped native FP64 GEMM on gfx950 MFMA: C = alpha A B + beta C, column-major,
// no transpose.  Replaces the reference's cuBLAS calls for its native routes (K_ZERO, ALPHA_ZERO,
// K_TOO_LARGE, SMALL_K, TINY, UNPROFITABLE, PRECISION) and the two native paths
// (src/ggemm.cu:102-184, src/ggemm_graph.cu:88-102).
//
// One launch per group: 64 x 64 output tiles of all problems in one table (same prefix/entry
// format as the INT8 GEMM), workgroup b takes tile b.  256 threads = 4 waves (2 x 2), wave tile
// 32 x 32 = 2 x 2 blocks of v_mfma_f64_16x16x4_f64; K staged 16 deep through LDS (double buffer,
// 32 KB: five workgroups per compute unit, 4 % faster than four with padded rows), A read as
// 512-byte column segments, B as 128-byte row segments.  Descriptors live in device
// memory, so a captured graph replays with new pointers after one small H2D.
// BLAS semantics: alpha == 0 or k == 0 never reads A or B; beta == 0 never reads C.
#include <algorithm>
#include <cstring>
#include <vector>

#include "common.hpp"

namespace ggemm {
namespace {

typedef double v4d __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kTile = 64;
constexpr int kBK = 16;

// LDS column of element (k, c): 16-column blocks XOR-swizzled by k mod 4, so the four k rows a
// fragment read touches sit in different banks without padding
__device__ __forceinline__ int swc(int k, int c) { return c ^ ((k & 3) << 4); }

__global__ void __launch_bounds__(kThreads, 5) f64_grouped_kernel(const F64Problem* __restrict__ probs,
                                                                  const int* __restrict__ sched) {
  __shared__ double sA[2][kBK][kTile];
  __shared__ double sB[2][kBK][kTile];
  const int tile = blockIdx.x;
  const int ne = sched[1];
  const int* prefix = sched + kSchedHdr;
  const int* entry = prefix + ne + 1;
  int lo = 0, hi = ne - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (prefix[mid] <= tile) lo = mid; else hi = mid - 1;
  }
  const F64Problem P = probs[entry[lo] >> 2];
  const int local = tile - prefix[lo];
  const int tiles_m = (P.m + kTile - 1) / kTile;
  const int row0 = (local % tiles_m) * kTile, col0 = (local / tiles_m) * kTile;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;

  v4d acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v4d{0.0, 0.0, 0.0, 0.0};

  const bool compute = P.alpha != 0.0 && P.k > 0;
  if (compute) {
    // loaders: A element (ar, ak + 4q), B element (bk + q, bc)
    const int ar = tid & 63, ak = tid >> 6;
    const int bc = tid >> 2, bk = (tid & 3) * 4;
    const size_t lda = (size_t)P.lda, ldb = (size_t)P.ldb;
    const bool arow = row0 + ar < P.m, bcol = col0 + bc < P.n;
    double ra[4], rb[4];
    auto gload = [&](int k0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int k = k0 + ak + 4 * q;
        ra[q] = (arow && k < P.k) ? P.A[(size_t)(row0 + ar) + (size_t)k * lda] : 0.0;
        const int kb = k0 + bk + q;
        rb[q] = (bcol && kb < P.k) ? P.B[(size_t)kb + (size_t)(col0 + bc) * ldb] : 0.0;
      }
    };
    auto sstore = [&](int st) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        sA[st][ak + 4 * q][swc(ak + 4 * q, ar)] = ra[q];
        sB[st][bk + q][swc(bk + q, bc)] = rb[q];
      }
    };
    const int nk = (P.k + kBK - 1) / kBK;
    gload(0);
    sstore(0);
    __syncthreads();
    const int fr = lane & 15, fk = lane >> 4;
    for (int kt = 0; kt < nk; ++kt) {
      if (kt + 1 < nk) gload((kt + 1) * kBK);
      const int st = kt & 1;
#pragma unroll
      for (int s = 0; s < kBK / 4; ++s) {
        double a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) a[i] = sA[st][4 * s + fk][swc(fk, wm * 32 + i * 16 + fr)];
#pragma unroll
        for (int j = 0; j < 2; ++j) b[j] = sB[st][4 * s + fk][swc(fk, wn * 32 + j * 16 + fr)];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[i], b[j], acc[i][j], 0, 0, 0);
      }
      if (kt + 1 < nk) sstore((kt + 1) & 1);
      __syncthreads();
    }
  }
  // D block layout of v_mfma_f64_16x16x4f64: lane l, register r -> row 4 r + l / 16, column l % 16
  // (four single-row groups; the INT8 / F32 16 x 16 instructions use four consecutive rows instead)
  const size_t ldc = (size_t)P.ldc;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = col0 + wn * 32 + j * 16 + (lane & 15);
      const int rbase = row0 + wm * 32 + i * 16 + (lane >> 4);
      if (col >= P.n) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = rbase + 4 * r;
        if (row >= P.m) continue;
        double* cp = P.C + (size_t)row + (size_t)col * ldc;
        const double ab = compute ? P.alpha * acc[i][j][r] : 0.0;
        *cp = (P.beta == 0.0) ? ab : (compute ? ab + P.beta * *cp : P.beta * *cp);
      }
    }
}

}  // namespace

int f64_build_schedule(const F64Problem* h, int num, void* h_ws, size_t ws_bytes, int* total_tiles,
                       size_t* bytes_used) {
  if (num < 0 || (num > 0 && !h) || !h_ws || !total_tiles) return 1;
  if (ws_bytes < sched_bytes(num)) return 2;
  int* img = static_cast<int*>(h_ws);
  std::vector<std::pair<double, int>> order;
  order.reserve(num);
  for (int i = 0; i < num; ++i)
    if (h[i].m > 0 && h[i].n > 0) order.push_back({(double)std::max(h[i].k, 1), i});
  std::stable_sort(order.begin(), order.end(), [](auto& a, auto& b) { return a.first > b.first; });
  const size_t ne = order.size();
  int* prefix = img + kSchedHdr;
  int* entry = prefix + ne + 1;
  long long tot = 0;
  for (size_t j = 0; j < ne; ++j) {
    const F64Problem& p = h[order[j].second];
    prefix[j] = (int)tot;
    tot += (long long)((p.m + kTile - 1) / kTile) * ((p.n + kTile - 1) / kTile);
    entry[j] = order[j].second << 2;
  }
  prefix[ne] = (int)tot;
  if (tot > 0x7fffffffLL - 1000000) return 5;
  std::memset(img, 0, sizeof(int) * kSchedHdr);
  img[0] = (int)tot;
  img[1] = (int)ne;
  *total_tiles = (int)tot;
  if (bytes_used) *bytes_used = sizeof(int) * (kSchedHdr + 2 * ne + 1);
  return 0;
}

int f64_launch(const F64Problem* d_probs, const void* d_sched, int total_tiles, hipStream_t s) {
  if (total_tiles <= 0) return 0;
  hipLaunchKernelGGL(f64_grouped_kernel, dim3((unsigned)total_tiles), dim3(kThreads), 0, s, d_probs,
                     static_cast<const int*>(d_sched));
  return hipGetLastError() == hipSuccess ? 0 : 1;
}

}  // namespace ggemm
