// f64gemm.hip -- grouped native FP64 GEMM on gfx950 MFMA: C = alpha A B + beta C, column-major,
// no transpose.  Replaces the reference's cuBLAS calls for its native routes (K_ZERO, ALPHA_ZERO,
// K_TOO_LARGE, SMALL_K, TINY, UNPROFITABLE, PRECISION) and the two native paths
// (src/ggemm.cu:102-184, src/ggemm_graph.cu:88-102).
//
// One launch per group: T x T output tiles of all problems in one table (same prefix/entry format
// as the INT8 GEMM), workgroup b takes tile b.  256 threads = 4 waves (2 x 2), wave tile
// T/2 x T/2 of 16 x 16 blocks of v_mfma_f64_16x16x4f64; K staged 16 deep through LDS (double
// buffer, XOR-swizzled rows).  Two tile sizes, one per group:
//   T = 64: 2 x 2 blocks per wave, 32 KB of LDS, five workgroups per compute unit (4 % faster than
//           four with padded rows) -- small and ragged groups;
//   T = 128: 4 x 4 blocks per wave, 64 KB of LDS, two workgroups per compute unit: half the
//           operand traffic per flop and four times the MFMA work per fragment read -- groups
//           with enough large tiles to fill the GPU twice.
// Every output entry takes the same k-ordered chain of MFMAs (zero-padded beyond k) at either
// size, so both give bit-identical results.  Descriptors live in device memory, so a captured
// graph replays with new pointers after one small H2D.
// BLAS semantics: alpha == 0 or k == 0 never reads A or B; beta == 0 never reads C.
#include <algorithm>
#include <cstring>
#include <vector>

#include "common.hpp"

namespace ggemm {
namespace {

typedef double v4d __attribute__((ext_vector_type(4)));
// global address space: the descriptor pointers would otherwise compile to flat loads, which also
// count in lgkmcnt, so every LDS fragment wait would wait for the next stage's prefetch as well
#define GLOBAL __attribute__((address_space(1)))
constexpr int kThreads = 256;
constexpr int kBK = 16;

// LDS column of element (k, c): 16-column blocks XOR-swizzled by k mod 4, so the four k rows a
// fragment read touches sit in different banks without padding (bits 4-5 only: c stays in [0, T))
__device__ __forceinline__ int swc(int k, int c) { return c ^ ((k & 3) << 4); }

template <int T>
__global__ void __launch_bounds__(kThreads, T == 64 ? 5 : 2) f64_grouped_kernel(const F64Problem* __restrict__ probs,
                                                                              const int* __restrict__ sched) {
  constexpr int FB = T / 32;            // 16 x 16 blocks per wave and dimension
  constexpr int KS = kThreads / T;      // A loader: k rows per pass over the tile's rows
  constexpr int NA = kBK / KS;          // A elements per thread
  constexpr int NB = kBK / KS;          // B elements per thread (consecutive k of one column)
  __shared__ double sA[2][kBK][T];
  __shared__ double sB[2][kBK][T];
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
  const int tiles_m = (P.m + T - 1) / T;
  const int row0 = (local % tiles_m) * T, col0 = (local / tiles_m) * T;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;

  v4d acc[FB][FB];
#pragma unroll
  for (int i = 0; i < FB; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j) acc[i][j] = v4d{0.0, 0.0, 0.0, 0.0};

  const bool compute = P.alpha != 0.0 && P.k > 0;
  if (compute) {
    // loaders: A element (ar, ak + KS q), B element (bk + q, bc)
    const int ar = tid % T, ak = tid / T;
    const int bc = tid / KS, bk = (tid % KS) * NB;
    const size_t lda = (size_t)P.lda, ldb = (size_t)P.ldb;
    const bool arow = row0 + ar < P.m, bcol = col0 + bc < P.n;
    const GLOBAL double* Ag = (const GLOBAL double*)P.A;
    const GLOBAL double* Bg = (const GLOBAL double*)P.B;
    double ra[NA], rb[NB];
    // full tiles (every row and column inside, k a multiple of the stage) load without bounds
    // tests from two per-stage base pointers; the values are the same either way
    const bool full = row0 + T <= P.m && col0 + T <= P.n && P.k % kBK == 0;
    auto gload = [&](int k0) {
      if (full) {
        const GLOBAL double* pa = Ag + (size_t)(row0 + ar) + (size_t)(k0 + ak) * lda;
        const GLOBAL double* pb = Bg + (size_t)(col0 + bc) * ldb + (size_t)(k0 + bk);
#pragma unroll
        for (int q = 0; q < NA; ++q) ra[q] = pa[(size_t)(KS * q) * lda];
#pragma unroll
        for (int q = 0; q < NB; ++q) rb[q] = pb[q];
        return;
      }
#pragma unroll
      for (int q = 0; q < NA; ++q) {
        const int k = k0 + ak + KS * q;
        ra[q] = (arow && k < P.k) ? Ag[(size_t)(row0 + ar) + (size_t)k * lda] : 0.0;
      }
#pragma unroll
      for (int q = 0; q < NB; ++q) {
        const int kb = k0 + bk + q;
        rb[q] = (bcol && kb < P.k) ? Bg[(size_t)kb + (size_t)(col0 + bc) * ldb] : 0.0;
      }
    };
    auto sstore = [&](int st) {
#pragma unroll
      for (int q = 0; q < NA; ++q) sA[st][ak + KS * q][swc(ak + KS * q, ar)] = ra[q];
#pragma unroll
      for (int q = 0; q < NB; ++q) sB[st][bk + q][swc(bk + q, bc)] = rb[q];
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
        double a[FB], b[FB];
#pragma unroll
        for (int i = 0; i < FB; ++i) a[i] = sA[st][4 * s + fk][swc(fk, wm * (T / 2) + i * 16 + fr)];
#pragma unroll
        for (int j = 0; j < FB; ++j) b[j] = sB[st][4 * s + fk][swc(fk, wn * (T / 2) + j * 16 + fr)];
#pragma unroll
        for (int i = 0; i < FB; ++i)
#pragma unroll
          for (int j = 0; j < FB; ++j) acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[i], b[j], acc[i][j], 0, 0, 0);
      }
      if (kt + 1 < nk) sstore((kt + 1) & 1);
      __syncthreads();
    }
  }
  // D block layout of v_mfma_f64_16x16x4f64: lane l, register r -> row 4 r + l / 16, column l % 16
  // (four single-row groups; the INT8 / F32 16 x 16 instructions use four consecutive rows instead).
  // With beta != 0 the C0 values of a batch of blocks are all loaded before the batch's stores:
  // entry by entry, each C0 load waited for its data before the store (the stores might alias
  // the next loads), one memory round trip per entry.
  const size_t ldc = (size_t)P.ldc;
  GLOBAL double* const Cg = (GLOBAL double*)P.C;
  const bool rd = P.beta != 0.0;
  constexpr int NBLK = FB * FB, BATCH = NBLK < 8 ? NBLK : 8;
#pragma unroll
  for (int b0 = 0; b0 < NBLK; b0 += BATCH) {
    double c0[BATCH][4];
#pragma unroll
    for (int q = 0; q < BATCH; ++q) {
      const int i = (b0 + q) / FB, j = (b0 + q) % FB;
      const int col = col0 + wn * (T / 2) + j * 16 + (lane & 15);
      const int rbase = row0 + wm * (T / 2) + i * 16 + (lane >> 4);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = rbase + 4 * r;
        c0[q][r] = (rd && col < P.n && row < P.m) ? Cg[(size_t)row + (size_t)col * ldc] : 0.0;
      }
    }
#pragma unroll
    for (int q = 0; q < BATCH; ++q) {
      const int i = (b0 + q) / FB, j = (b0 + q) % FB;
      const int col = col0 + wn * (T / 2) + j * 16 + (lane & 15);
      const int rbase = row0 + wm * (T / 2) + i * 16 + (lane >> 4);
      if (col >= P.n) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = rbase + 4 * r;
        if (row >= P.m) continue;
        const double ab = compute ? P.alpha * acc[i][j][r] : 0.0;
        Cg[(size_t)row + (size_t)col * ldc] = !rd ? ab : (compute ? ab + P.beta * c0[q][r] : P.beta * c0[q][r]);
      }
    }
  }
}

}  // namespace

namespace {
long long tiles_of(const F64Problem& p, int t) { return (long long)((p.m + t - 1) / t) * ((p.n + t - 1) / t); }
}  // namespace

int f64_build_schedule(const F64Problem* h, int num, void* h_ws, size_t ws_bytes, int* launch, size_t* bytes_used,
                       int tile_mode) {
  if (num < 0 || (num > 0 && !h) || !h_ws || !launch) return 1;
  if (ws_bytes < sched_bytes(num)) return 2;
  // tile edge: 128 when the 128 x 128 tiles fill two workgroups on each of 256 compute units at
  // least twice and pad the outputs by at most 1/8 more than 64 x 64 tiles do, else 64
  int tile = tile_mode == 64 || tile_mode == 128 ? tile_mode : 64;
  if (tile_mode == 0) {
    long long t128 = 0, a64 = 0;
    for (int i = 0; i < num; ++i)
      if (h[i].m > 0 && h[i].n > 0) {
        t128 += tiles_of(h[i], 128);
        a64 += tiles_of(h[i], 64);
      }
    if (t128 >= 1024 && 4 * t128 * 8 <= a64 * 9) tile = 128;
  }
  // problems with outputs, longest k first (ties by index: the order a stable sort keeps), sorted
  // in place in the image's entry array -- no host scratch
  int* img = static_cast<int*>(h_ws);
  size_t ne = 0;
  for (int i = 0; i < num; ++i) ne += h[i].m > 0 && h[i].n > 0;
  int* prefix = img + kSchedHdr;
  int* entry = prefix + ne + 1;
  for (int i = 0, j = 0; i < num; ++i)
    if (h[i].m > 0 && h[i].n > 0) entry[j++] = i;
  std::sort(entry, entry + ne, [h](int a, int b) {
    const int ka = std::max(h[a].k, 1), kb = std::max(h[b].k, 1);
    return ka != kb ? ka > kb : a < b;
  });
  long long tot = 0;
  for (size_t j = 0; j < ne; ++j) {
    const F64Problem& p = h[entry[j]];
    prefix[j] = (int)tot;
    tot += tiles_of(p, tile);
    entry[j] <<= 2;
  }
  prefix[ne] = (int)tot;
  if (tot >= kF64Tile128) return 5;
  std::memset(img, 0, sizeof(int) * kSchedHdr);
  img[0] = (int)tot;
  img[1] = (int)ne;
  *launch = tot == 0 ? 0 : (int)tot | (tile == 128 ? kF64Tile128 : 0);
  if (bytes_used) *bytes_used = sizeof(int) * (kSchedHdr + 2 * ne + 1);
  return 0;
}

int f64_launch(const F64Problem* d_probs, const void* d_sched, int launch, hipStream_t s) {
  if (launch <= 0) return 0;
  const unsigned tiles = (unsigned)(launch & (kF64Tile128 - 1));
  if (launch & kF64Tile128)
    hipLaunchKernelGGL(f64_grouped_kernel<128>, dim3(tiles), dim3(kThreads), 0, s, d_probs, static_cast<const int*>(d_sched));
  else
    hipLaunchKernelGGL(f64_grouped_kernel<64>, dim3(tiles), dim3(kThreads), 0, s, d_probs, static_cast<const int*>(d_sched));
  return hipGetLastError() == hipSuccess ? 0 : 1;
}

}  // namespace ggemm
