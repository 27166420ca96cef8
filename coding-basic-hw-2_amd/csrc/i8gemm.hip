// i8gemm.hip -- grouped INT8 x INT8 -> INT32 GEMM on gfx950 MFMA (exact accumulation).
//
// Problem (src/int8_grouped_gemm.h:4-10 layout): A m x kp and B n x kp row-major (K contiguous),
// C = A B^T column-major m x n (ld m), kp % 32 == 0, |C| <= 128^2 kp < 2^31 (kp <= 131040).
//
// One launch covers every (problem, plane) of a group.  The host builds a tile table in
// longest-processing-time order (heaviest tiles first, the reference's scheduling contract,
// src/int8_grouped_gemm.cu:602-675).  Workgroup b takes one tile:
//   * XCD-aware dispatch: MI355X deals workgroups round-robin to its 8 XCDs (b mod 8), each with
//     its own L2.  Workgroup b is mapped to tile chunk (b mod 8) + 8 (b / (8 C)) of C
//     consecutive table tiles, so one XCD works through contiguous runs of the table;
//   * inside an entry tiles are rastered in groups of G tile-rows, m fastest, so the compute
//     units of an XCD share A and B panels in L2.
//   General kernel C = 32, G = 8: a 1024^2 product's 32 tiles share one L2 and each plane is read
//   from HBM once (C = 16 reads them 1.5 times at equal speed).  Large-tile kernel C = 16, G = 4:
//   on 8192^2 x 16384 products 1-3 % faster than 32 / 8 in two of three same-box comparisons,
//   equal in the third (G = 16: 10 % slower).
// General kernel: workgroups of 512 threads = 8 waves in a 4 x 2 arrangement, two workgroups per
// compute unit (one's epilogue and barrier waits overlap the other's MFMA work):
//   cfg 0: 256 x 128 tile, wave tile 64 x 64 = 4 x 4 blocks of v_mfma_i32_16x16x64_i8
//   cfg 1: 128 x 128 tile, wave tile 32 x 64 = 2 x 4 blocks
//   cfg 2:  64 x  64 tile, wave tile 16 x 32 = 1 x 2 blocks
// Large-tile kernel: one workgroup of 16 waves (4 x 4) per compute unit, 256 x 256 tiles.
// K advances in stages of 64.  Operands go HBM -> LDS directly (global_load_lds_dwordx4, no VGPR
// round trip) into a ring of 3 LDS stages, two stages ahead of the MFMA work; one barrier per
// stage.  An LDS row holds the 64 k-bytes of one A / B row as 4 chunks of 16 bytes, chunk index
// XOR-swizzled by (row / 2) mod 4 so that the 16-lane groups of each 128-bit fragment read hit
// distinct banks.  A DMA instruction fills 1 KB (16 rows): lane l writes chunk l mod 4 of row
// l / 4 and so loads the global chunk that the swizzle puts there.
// Fragment reads are issued as inline ds_read_b128 with a single lgkmcnt wait: the compiler would
// otherwise place a vmcnt(0) before every LDS read that may alias an LDS DMA in flight, which
// drains the prefetch ring.  The ring's own waits are explicit (s_waitcnt vmcnt(n) + s_barrier).
// Bounds: rows >= m / n load (clamped) row m-1 / n-1 and only feed outputs that are not stored;
// with kp % 64 == 32 the last stage's A chunks k >= kp are overwritten with zeros before use.
// Operands: row-major residues (the kernel-level API) or, in the production pipeline, the packed
// layout, where a stage's 64 k-bytes of 16 consecutive rows are one contiguous kilobyte.
// Epilogue, per problem: int32 C (the reference contract, used by the kernel-level API and the
// abs plane), or -- in the production pipeline -- one residue byte C mod p per entry (I8Epi),
// which with q-folded A residues is the CRT digit; this cuts the plane write from 4 to 1 byte.
// The production pipeline also stores in the blocked layout: each 16 x 16 MFMA result block is one
// contiguous 256-byte (digits) or 1 KB (int32) store instead of 16 column pieces.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <type_traits>
#include <vector>

#include "common.hpp"

#define GGEMM_LDS(p) ((__attribute__((address_space(3))) void*)(p))
// output stores through global-address-space pointers (flat stores would also count in lgkmcnt)
#define GLOBAL __attribute__((address_space(1)))

namespace ggemm {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kBK = 64;
// XCD chunk (tiles) and raster group (tile-rows) of the two kernels
constexpr int kChunk = 32, kGroupM = 8;     // general kernel
constexpr int kChunkL = 16, kGroupML = 4;   // large-tile kernel
constexpr int kXcds = 8;

// Tile BM x BN computed by WGM x WGN waves through an NST-stage LDS ring.
template <int BM_, int BN_, int WGM_, int WGN_, int NST_>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_, NST = NST_;
  static constexpr int NW = WGM * WGN, NT = 64 * NW;
  static constexpr int WM = BM / WGM, WN = BN / WGN;   // wave tile
  static constexpr int FM = WM / 16, FN = WN / 16;     // 16 x 16 MFMA blocks per wave
  static constexpr int SA = BM * kBK, SB = BN * kBK, STAGE = SA + SB;
  static constexpr int PA = SA / 1024, PB = SB / 1024; // 1 KB DMA pieces per operand and stage
  // a stage's A pieces then B pieces, dealt to the waves round-robin: piece g = wave + NW q
  static constexpr int VM = (PA + PB) / NW;            // DMA instructions per wave and stage
  static constexpr int SMEM = NST * STAGE;
  // k loop with the stage barrier between the two halves of a stage's MFMAs (below): pays for
  // the large-tile kernels (one workgroup per compute unit), not for the general kernel's two
  // workgroups
  static constexpr bool kSplit = NW >= 16;
  static_assert((PA + PB) % NW == 0 && FM >= 1 && FN >= 1, "tile split");
};
// general kernel: 512 threads = 8 waves of (BM / 4) x (BN / 2), two workgroups per compute unit
// (72 KB of LDS each, four waves per SIMD); against 4 waves of (BM / 2) x (BN / 2) the 256 x 128
// tiles of 1024^3 products run 1.4-3 % faster (more waves hide the DMA and LDS waits)
using Cfg0 = Cfg<256, 128, 4, 2, 3>;
using Cfg1 = Cfg<128, 128, 4, 2, 3>;
using Cfg2 = Cfg<64, 64, 4, 2, 3>;
constexpr int kThreads = 512;
constexpr int kSmem = Cfg0::SMEM;
static_assert(Cfg1::SMEM <= kSmem && Cfg2::SMEM <= kSmem, "smem");
// large-tile kernel: 1024 threads = 16 waves of 64 x 64 (4 per SIMD, so one wave's LDS reads and
// barrier waits overlap the others' MFMAs), one workgroup per compute unit, 128 KB ring
using CfgL = Cfg<256, 256, 4, 4, 4>;
constexpr int kThreadsL = CfgL::NT;
constexpr int kSmemL = CfgL::SMEM;

__device__ __forceinline__ int swz(int row, int ch) { return ch ^ ((row >> 1) & 3); }

// f(integral_constant<int, I>) for I = B .. E - 1: indices of accumulator arrays stay compile-time
// constants (a loop the unroller declines to flatten would put the accumulators in memory)
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// ds_read_b128 at LDS byte address addr + OFF
template <int OFF>
__device__ __forceinline__ v4i lds_read(uint32_t addr) {
  v4i r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
template <int F, int OFF0, int I = 0>
__device__ __forceinline__ void read_frags(v4i* f, uint32_t addr) {
  if constexpr (I < F) {
    f[I] = lds_read<OFF0 + I * 1024>(addr);
    read_frags<F, OFF0, I + 1>(f, addr);
  }
}
// at most VM of this wave's LDS DMA instructions outstanding, LDS ops done, then the barrier
template <int VM>
__device__ __forceinline__ void wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(VM) : "memory");
}

// Wait for this wave's LDS reads with every fragment register an operand of the wait, so that no
// compiler-generated copy of a fragment can be placed before its data has arrived.
template <int FM, int FN>
__device__ __forceinline__ void lds_wait_frags(v4i (&a)[FM], v4i (&b)[FN]) {
  if constexpr (FM == 4 && FN == 4) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]));
  } else if constexpr (FM == 2 && FN == 4) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a[0]), "+v"(a[1]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]));
  } else {
    static_assert(FM == 1 && FN == 2, "fragment counts");
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a[0]), "+v"(b[0]), "+v"(b[1]));
  }
}

// One k-stage of an operand: the address of its tile's first row, the byte stride between rows and
// the valid bytes per row (chunks at or past it load chunk 0 instead; A's are zeroed in LDS).
struct StageSrc {
  const int8_t* base;
  int stride, lim;
};
// row-major residues (rows x kp, the kernel-level API) or the packed layout (production)
__device__ __forceinline__ StageSrc stage_src(const int8_t* plane, int rows, int row0, int kp, int k0, bool packed) {
  if (packed) {
    const int b = k0 >> 6, rb = b == (kp >> 6) ? 32 : 64;
    return StageSrc{plane + (size_t)b * rows * 64 + (size_t)row0 * rb, rb, rb};
  }
  return StageSrc{plane + (size_t)row0 * kp + k0, kp, kp - k0};
}

// This wave's DMA pieces of a stage (wave-uniform): fa(A piece) and fb(B piece), C::VM in all.
template <class C, class FA, class FB>
__device__ __forceinline__ void for_pieces(int wave, FA&& fa, FB&& fb) {
  if constexpr (C::PA % C::NW == 0) {   // the A / B split is a multiple of the wave count
#pragma unroll
    for (int q = 0; q < C::PA / C::NW; ++q) fa(wave + C::NW * q);
#pragma unroll
    for (int q = 0; q < C::PB / C::NW; ++q) fb(wave + C::NW * q);
  } else {
#pragma unroll
    for (int q = 0; q < C::VM; ++q) {
      const int g = wave + C::NW * q;
      if (g < C::PA) fa(g); else fb(g - C::PA);
    }
  }
}

template <class C>
__device__ __forceinline__ void dma_stage(const StageSrc& a, const StageSrc& b, int m_rem, int n_rem, uint8_t* st,
                                          int wave, int lane) {
  const int r_in = lane >> 2, pc = lane & 3;
  auto piece_of = [&](const StageSrc& o, int rem, int piece, uint8_t* dst) {
    const int row = piece * 16 + r_in;
    const int kk = 16 * swz(row, pc);
    const int rr = row < rem ? row : rem - 1;
    __builtin_amdgcn_global_load_lds((const void*)(o.base + (size_t)rr * o.stride + (kk < o.lim ? kk : 0)),
                                     GGEMM_LDS(dst + piece * 1024), 16, 0, 0);
  };
  for_pieces<C>(wave, [&](int piece) { piece_of(a, m_rem, piece, st); },
                [&](int piece) { piece_of(b, n_rem, piece, st + C::SA); });
}

// The same stage when every row of the tile exists and every chunk is inside the row (the common
// case): piece offsets are wave-uniform and the per-lane offset r_in stride + 16 swz(r_in, pc) is
// fixed for the tile (the swizzle of row 16 piece + r_in depends on r_in only), so each DMA is a
// scalar base plus one per-lane offset.
template <class C>
__device__ __forceinline__ void dma_stage_full(const int8_t* a, const int8_t* b, int a_stride, int b_stride,
                                               uint32_t a_lane, uint32_t b_lane, uint8_t* st, int wave) {
  for_pieces<C>(
      wave,
      [&](int piece) {
        __builtin_amdgcn_global_load_lds((const void*)(a + (size_t)piece * 16 * a_stride + a_lane),
                                         GGEMM_LDS(st + piece * 1024), 16, 0, 0);
      },
      [&](int piece) {
        __builtin_amdgcn_global_load_lds((const void*)(b + (size_t)piece * 16 * b_stride + b_lane),
                                         GGEMM_LDS(st + C::SA + piece * 1024), 16, 0, 0);
      });
}

// C mod p in [0, p) from u = C + bias >= 0: q = umulhi(u, mc) with mc = ceil(2^32 / p) is floor(u / p)
// or one more (u (mc - 2^32/p) < 2^32), so r = u - q p is in [-p, p), and min(r, r + p) as unsigned
// is r mod p.  kAcc: u is the accumulator (it started at the bias), u < 2^30 + p and q < 2^23, so
// r is one 24-bit multiply-add.
template <bool kAcc>
__device__ __forceinline__ uint32_t residue_byte(int32_t c, const I8Epi& e) {
  const uint32_t u = kAcc ? (uint32_t)c : (uint32_t)c + e.bias;
  const uint32_t q = __umulhi(u, e.mc);
  const int r = kAcc ? __mul24((int)q, -(int)e.p) + (int)u : (int)(u - q * e.p);
  return min((uint32_t)r, (uint32_t)(r + (int)e.p));
}

// Blocked epilogue: kind 0 int32 blocks (16 bytes per lane), 1 residue bytes from biased
// accumulators, 2 residue bytes with the bias added here (4 bytes per lane, packed with v_perm).
// The block offsets are wave-uniform; a lane writes at 4 lane entries into each block.
template <class C>
__device__ __forceinline__ void store_blocked(const v4i (&acc)[C::FM][C::FN], const i8_problem& P, const I8Epi& epi,
                                              int kind, int bi0, int bj0, int mb, int lane) {
  GLOBAL uint8_t* const y8 = ((GLOBAL uint8_t*)P.C) + 4 * lane;
  GLOBAL int32_t* const y32 = ((GLOBAL int32_t*)P.C) + 4 * lane;
  static_for<0, C::FN * C::FM>([&](auto ij) {
    constexpr int j = decltype(ij)::value / C::FM, i = decltype(ij)::value % C::FM;
    const int bi = bi0 + i, bj = bj0 + j;
    if (bi * 16 < P.m && bj * 16 < P.n) {   // wave-uniform
      const size_t e0 = ((size_t)bj * mb + bi) * 256;
      const v4i v = acc[i][j];
      if (kind == 0) {
        *reinterpret_cast<GLOBAL v4i*>(y32 + e0) = v;
      } else {
        uint32_t y[4];
        if (kind == 1) {
#pragma unroll
          for (int r = 0; r < 4; ++r) y[r] = residue_byte<true>(v[r], epi);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) y[r] = residue_byte<false>(v[r], epi);
        }
        const uint32_t lo = __builtin_amdgcn_perm(y[1], y[0], 0x0c0c0400u);
        const uint32_t hi = __builtin_amdgcn_perm(y[3], y[2], 0x0c0c0400u);
        *reinterpret_cast<GLOBAL uint32_t*>(y8 + e0) = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
      }
    }
  });
}

// Epilogue of a tile: the accumulators of the wave (wm, wn) = (wave % WGM, wave / WGM) stored as int32
// or residue bytes, blocked or column-major (I8Epi).
template <class C>
__device__ __forceinline__ void tile_epilogue(const v4i (&acc)[C::FM][C::FN], const i8_problem& P, const I8Epi& epi,
                                              int row0, int col0, int wave, int lane) {
  constexpr int FM = C::FM, FN = C::FN;
  const int wm = wave % C::WGM, wn = wave / C::WGM;
  // D block layout: lane l, register r -> row 4 (l / 16) + r, column l % 16; a lane's 4 values
  // are 4 consecutive rows of one column, i.e. contiguous in the column-major output, and the
  // 64 lanes' values are one 16 x 16 block of the blocked output layout.
  const bool residue = (epi.mode & kEpiResidue) != 0;
  if (epi.mode & kEpiBlocked) {   // every existing block is stored whole (padding included)
    // block (bi, bj) of the wave: uniform offset (bj MB + bi) 256 entries, lane l at entries 4 l
    const int mb = (P.m + 15) / 16;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int bi0 = (row0 + (wv % C::WGM) * C::WM) / 16, bj0 = (col0 + (wv / C::WGM) * C::WN) / 16;
    const int kind = !residue ? 0 : (epi.mode & kEpiAccBias) ? 1 : 2;
    store_blocked<C>(acc, P, epi, kind, bi0, bj0, mb, lane);
    return;
  }
  const size_t ldc = (size_t)P.m;
  const bool vec = (P.m % 4 == 0) && ((reinterpret_cast<uintptr_t>(P.C) & (residue ? 3 : 15)) == 0);
  static_for<0, FM * FN>([&](auto ij) {
    constexpr int i = decltype(ij)::value / FN, j = decltype(ij)::value % FN;
    const int col = col0 + wn * C::WN + j * 16 + (lane & 15);
    const int r0 = row0 + wm * C::WM + i * 16 + 4 * (lane >> 4);
    if (col < P.n && r0 < P.m) {
      const v4i v = acc[i][j];
      if (!residue) {
        GLOBAL int32_t* out = ((GLOBAL int32_t*)P.C) + (size_t)r0 + (size_t)col * ldc;
        if (vec && r0 + 3 < P.m) {
          *reinterpret_cast<GLOBAL v4i*>(out) = v;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (r0 + r < P.m) out[r] = v[r];
        }
      } else {
        GLOBAL uint8_t* out = ((GLOBAL uint8_t*)P.C) + (size_t)r0 + (size_t)col * ldc;
        uint32_t y[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] = (epi.mode & kEpiAccBias) ? residue_byte<true>(v[r], epi) : residue_byte<false>(v[r], epi);
        if (vec && r0 + 3 < P.m) {
          *reinterpret_cast<GLOBAL uint32_t*>(out) = y[0] | (y[1] << 8) | (y[2] << 16) | (y[3] << 24);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (r0 + r < P.m) out[r] = (uint8_t)y[r];
        }
      }
    }
  });
}

template <class C, bool kPacked>
__device__ __forceinline__ void run_tile(uint8_t* lds, const i8_problem& P, const I8Epi& epi, int tm, int tn) {
  constexpr int FM = C::FM, FN = C::FN, NST = C::NST;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % C::WGM, wn = wave / C::WGM;
  const int row0 = tm * C::BM, col0 = tn * C::BN;
  const int m_rem = P.m - row0, n_rem = P.n - col0;
  const int kp = P.kp;
  const int nk = (kp + kBK - 1) / kBK;
  // full stages: all tile rows exist and the stage has 64 bytes per row (packed: every k-block but
  // a final half block; row-major: every stage but a final half stage)
  const bool full_rows = m_rem >= C::BM && n_rem >= C::BN;
  const int fstride = kPacked ? 64 : kp;
  const int r_in = lane >> 2;
  const uint32_t lane_off = (uint32_t)(r_in * fstride + 16 * swz(r_in, lane & 3));
  auto load = [&](int kt, uint8_t* st) {
    const int k0 = kt * kBK;
    if (full_rows && k0 + kBK <= kp) {
      const int8_t* a = kPacked ? P.A + (size_t)(k0 >> 6) * P.m * 64 + (size_t)row0 * 64 : P.A + (size_t)row0 * kp + k0;
      const int8_t* b = kPacked ? P.B + (size_t)(k0 >> 6) * P.n * 64 + (size_t)col0 * 64 : P.B + (size_t)col0 * kp + k0;
      dma_stage_full<C>(a, b, fstride, fstride, lane_off, lane_off, st, wave);
    } else {
      dma_stage<C>(stage_src(P.A, P.m, row0, kp, k0, kPacked), stage_src(P.B, P.n, col0, kp, k0, kPacked), m_rem,
                   n_rem, st, wave, lane);
    }
  };

  // fragment addresses: rows wm WM + 16 i + lane % 16 (A), wn WN + 16 j + lane % 16 (B), chunk lane / 16;
  // the swizzle depends on row / 2 mod 4 only, so blocks i, j sit at fixed 1 KB immediates
  const int fr = lane & 15, fc = lane >> 4;
  const uint32_t lbase = (uint32_t)(uintptr_t)GGEMM_LDS(lds);
  const int ra = wm * C::WM + fr, rb = wn * C::WN + fr;
  const uint32_t a_addr = lbase + ra * kBK + swz(ra, fc) * 16;
  const uint32_t b_addr = lbase + rb * kBK + swz(rb, fc) * 16;

  const int a0 = (epi.mode & kEpiAccBias) ? (int)epi.bias : 0;   // accumulator start
  v4i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4i{a0, a0, a0, a0};

  // a final half stage (k in [kp, kp + 32)): zero A's chunks 2, 3 (B's duplicate chunk 0)
  auto zero_half = [&](uint8_t* st) {
    for (int c = tid; c < C::BM * 2; c += C::NT) {
      const int row = c >> 1, ch = 2 + (c & 1);
      *reinterpret_cast<uint4*>(st + row * kBK + swz(row, ch) * 16) = make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto mfmas = [&](const v4i* a, const v4i (&b)[FN], int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
  };
  if constexpr (C::kSplit) {
    // Stage s in ring slot s mod NST.  Iteration kt holds stage kt's fragments in registers: it
    // issues the MFMAs of the first half of the A blocks, then (those queued on the matrix core)
    // waits for stage kt + 1 and passes the barrier, refills slot kt (every wave holds its
    // fragments) with stage kt + NST, reads stage kt + 1's first-half A fragments into the
    // registers just consumed, issues the second half and reads the rest of stage kt + 1.  The
    // barrier and the LDS latency overlap queued MFMA work (16-wave kernel: 2.4 % at k = 16384).
    constexpr int H = FM / 2;
#pragma unroll
    for (int q = 0; q < NST; ++q)
      if (q < nk) load(q, lds + q * C::STAGE);
    if (nk <= 0) return;      // never scheduled: problems with kp == 0 get no tiles
    __builtin_assume(nk > 0);  // one path into the epilogue (no zero-trip copy of the accumulators)
    // stage 0 landed (stages 1 .. NST - 1 may still be in flight)
    if (NST - 1 < nk) wait_barrier<(NST - 1) * C::VM>(); else wait_barrier<0>();
    if (nk == 1 && (kp & 63)) {
      zero_half(lds);
      wait_barrier<0>();
    }
    v4i a[FM], b[FN];
    read_frags<FN, C::SA>(b, b_addr);
    read_frags<FM, 0>(a, a_addr);
    int buf = 0;
    for (int kt = 0; kt < nk; ++kt) {
      lds_wait_frags<FM, FN>(a, b);   // stage kt's fragments are valid after this wait
      mfmas(a, b, 0, H);
      const bool more = kt + 1 < nk;
      const int nb = buf + 1 == NST ? 0 : buf + 1;
      const uint32_t so = (uint32_t)(nb * C::STAGE);
      if (more) {
        // stage kt + 1 landed (the NST - 2 stages after it may still be in flight; near the end
        // fewer were issued, so wait for everything)
        if (kt + NST - 1 < nk) wait_barrier<(NST - 2) * C::VM>(); else wait_barrier<0>();
        if (kt + NST < nk) load(kt + NST, lds + buf * C::STAGE);
        if (kt + 2 == nk && (kp & 63)) {
          zero_half(lds + nb * C::STAGE);
          wait_barrier<0>();
        }
        read_frags<H, 0>(a, a_addr + so);
      }
      mfmas(a, b, H, FM);
      if (more) {
        read_frags<FM - H, H * 1024>(a + H, a_addr + so);
        read_frags<FN, C::SA>(b, b_addr + so);
      }
      buf = nb;
    }
    // the last iteration issues no reads: an explicit wait keeps every path into the epilogue
    // free of pending LDS loads (also for the assembly dataflow check)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  } else {
    // Stage kt waits, passes the barrier (every wave is done with stage kt - 1), refills slot
    // kt - 1 with stage kt + NST - 1, reads all its fragments and issues every MFMA.  With two
    // workgroups per compute unit the other workgroup's MFMAs cover this one's waits.
#pragma unroll
    for (int q = 0; q < NST - 1; ++q)
      if (q < nk) load(q, lds + q * C::STAGE);
    int buf = 0;
    if (nk <= 0) return;      // never scheduled: problems with kp == 0 get no tiles
    __builtin_assume(nk > 0);  // one path into the epilogue (no zero-trip copy of the accumulators)
    for (int kt = 0; kt < nk; ++kt) {
      // stage kt landed (the NST - 2 stages after it may still be in flight; near the end fewer
      // were issued, so wait for everything) and every wave is done with stage kt - 1
      if (kt + NST - 2 < nk) wait_barrier<(NST - 2) * C::VM>(); else wait_barrier<0>();
      if (kt + NST - 1 < nk) {
        int b2 = buf + NST - 1;   // the ring slot of stage kt - 1
        if (b2 >= NST) b2 -= NST;
        load(kt + NST - 1, lds + b2 * C::STAGE);
      }
      if (kt == nk - 1 && (kp & 63)) {
        zero_half(lds + buf * C::STAGE);
        wait_barrier<0>();
      }
      const uint32_t so = (uint32_t)(buf * C::STAGE);
      v4i a[FM], b[FN];
      read_frags<FN, C::SA>(b, b_addr + so);
      read_frags<FM, 0>(a, a_addr + so);
      lds_wait_frags<FM, FN>(a, b);   // the fragments are valid after this wait
      // raised wave priority while the stage's MFMAs issue, ahead of the other waves' DMA, LDS
      // reads and epilogue (0.4-1.1 % faster on 1024^3 products in two same-box comparisons; the
      // 16-wave kernel measured 1 % slower with it)
      __builtin_amdgcn_s_setprio(1);
      mfmas(a, b, 0, FM);
      __builtin_amdgcn_s_setprio(0);
      buf = buf + 1 == NST ? 0 : buf + 1;
    }
  }

  tile_epilogue<C>(acc, P, epi, row0, col0, wave, lane);
}

// Tile of workgroup blockIdx.x: XCD-aware remap of the dispatch index (a permutation of
// [0, total)) and entry lookup in the prefix table; `local` is the tile index inside the entry.
struct TileRef {
  int pi, cfg, local;
};
template <int CH>
__device__ __forceinline__ TileRef find_tile(const int* __restrict__ sched) {
  const int total = sched[0];
  const int ne = sched[1];
  const int b = blockIdx.x;
  const int span = kXcds * CH;
  const int full = total / span * span;
  int tile = b;
  if (b < full) {
    const int x = b % kXcds, q = b / kXcds;
    tile = (q / CH) * span + x * CH + (q % CH);
  }
  const int* prefix = sched + kSchedHdr;
  const int* entry = prefix + ne + 1;
  const int per = sched[2];   // tiles of every entry when they are all equal (no search), else 0
  int lo;
  if (per > 0) {
    lo = tile / per;
  } else {
    lo = 0;                   // largest e with prefix[e] <= tile
    int hi = ne - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (prefix[mid] <= tile) lo = mid; else hi = mid - 1;
    }
  }
  const int e = entry[lo];
  return TileRef{e >> 2, e & 3, tile - (per > 0 ? lo * per : prefix[lo])};
}
// grouped raster inside a product: blocks of GM tile-rows, m fastest inside a block
template <int GM>
__device__ __forceinline__ void raster(int local, int m, int n, int bm, int bn, int& tm, int& tn) {
  const int tiles_m = (m + bm - 1) / bm, tiles_n = (n + bn - 1) / bn;
  const int per_group = GM * tiles_n;
  const int g = local / per_group, first_m = g * GM;
  const int gsz = min(GM, tiles_m - first_m);
  const int r = local - g * per_group;
  tm = first_m + r % gsz;
  tn = r / gsz;
}

__global__ void __launch_bounds__(kThreads, 2) i8_grouped_kernel(const i8_problem* __restrict__ probs,
                                                                 const I8Epi* __restrict__ epis,
                                                                 const int* __restrict__ sched) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  const TileRef t = find_tile<kChunk>(sched);
  const i8_problem P = probs[t.pi];
  I8Epi epi{0u, 1u, 0u, 0u};
  if (epis) epi = epis[t.pi];
  int tm, tn;
  raster<kGroupM>(t.local, P.m, P.n, i8_tile_m(t.cfg), i8_tile_n(t.cfg), tm, tn);
  switch (t.cfg) {
    case 0: (epi.mode & kEpiPacked) ? run_tile<Cfg0, true>(lds, P, epi, tm, tn) : run_tile<Cfg0, false>(lds, P, epi, tm, tn); break;
    case 1: (epi.mode & kEpiPacked) ? run_tile<Cfg1, true>(lds, P, epi, tm, tn) : run_tile<Cfg1, false>(lds, P, epi, tm, tn); break;
    default: (epi.mode & kEpiPacked) ? run_tile<Cfg2, true>(lds, P, epi, tm, tn) : run_tile<Cfg2, false>(lds, P, epi, tm, tn); break;
  }
}

// every tile of the schedule is a 256 x 256 tile
__global__ void __launch_bounds__(kThreadsL, 1) i8_large_kernel(const i8_problem* __restrict__ probs,
                                                                const I8Epi* __restrict__ epis,
                                                                const int* __restrict__ sched) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  const TileRef t = find_tile<kChunkL>(sched);
  const i8_problem P = probs[t.pi];
  I8Epi epi{0u, 1u, 0u, 0u};
  if (epis) epi = epis[t.pi];
  int tm, tn;
  raster<kGroupML>(t.local, P.m, P.n, CfgL::BM, CfgL::BN, tm, tn);
  if (epi.mode & kEpiPacked) run_tile<CfgL, true>(lds, P, epi, tm, tn);
  else run_tile<CfgL, false>(lds, P, epi, tm, tn);
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
  const int bm = i8_tile_m(cfg), bn = i8_tile_n(cfg);
  return ((m + bm - 1) / bm) * ((n + bn - 1) / bn);
}
// Automatic tile: least padded work per unit efficiency (relative efficiencies 1, 0.7, 0.35).
int auto_cfg(int m, int n) {
  static const double eff[3] = {1.0, 0.7, 0.35};
  int best = 0;
  double best_cost = 1e300;
  for (int c = 0; c < kI8NumCfg; ++c) {
    const double cost = tiles_of(c, m, n) * (double)i8_tile_m(c) * i8_tile_n(c) / eff[c];
    if (cost < best_cost) { best_cost = cost; best = c; }
  }
  return best;
}

}  // namespace

int i8_build_schedule(const i8_problem* h, int num, void* h_ws, size_t ws_bytes, i8_sched_info* info, int num_cus,
                      int large, int* kernel) {
  if (num < 0 || (num > 0 && !h) || !h_ws || !info) return 1;
  if (ws_bytes < sched_bytes(num)) return 2;
  if (kernel) *kernel = kI8General;
  std::lock_guard<std::mutex> lk(g_mu);
  std::vector<Ent>& ents = g_ents;
  ents.clear();
  for (int i = 0; i < num; ++i) {
    if (!valid_problem(h[i])) return 3;
    if (h[i].m == 0 || h[i].n == 0 || h[i].kp == 0) continue;
    int c = h[i].tile_cfg;
    if (c < 0) c = auto_cfg(h[i].m, h[i].n);
    if (c >= kI8NumCfg) c = kI8NumCfg - 1;
    ents.push_back({(double)i8_tile_m(c) * i8_tile_n(c) * (double)(h[i].kp + 128), tiles_of(c, h[i].m, h[i].n), i, c});
  }
  bool all_auto = !ents.empty();
  for (auto& e : ents) all_auto = all_auto && h[e.prob].tile_cfg < 0;
  const bool force_large = large == kLargeForce && all_auto;
  // group-level fill: fewer tiles than workgroup slots (2 per compute unit) -> shrink automatic
  // tiles one step
  for (int pass = 0; pass < 2 && !force_large; ++pass) {
    long long t = 0;
    for (auto& e : ents) t += e.tiles;
    if (t >= 2LL * num_cus) break;
    for (auto& e : ents)
      if (e.cfg < kI8NumCfg - 1 && h[e.prob].tile_cfg < 0) {
        ++e.cfg;
        e.tiles = tiles_of(e.cfg, h[e.prob].m, h[e.prob].n);
        e.cost = (double)i8_tile_m(e.cfg) * i8_tile_n(e.cfg) * (double)(h[e.prob].kp + 128);
      }
  }
  // large-tile kernel: every product on automatic large tiles, and enough 256 x 256 tiles to give
  // every compute unit one
  if (large != kLargeNever && !ents.empty()) {
    bool all = true;
    long long t = 0;
    for (auto& e : ents) {
      all = all && e.cfg == 0 && h[e.prob].tile_cfg < 0;
      t += (long long)((h[e.prob].m + 255) / 256) * ((h[e.prob].n + 255) / 256);
    }
    if (force_large || (all && t >= num_cus)) {
      for (auto& e : ents) {
        e.tiles = ((h[e.prob].m + 255) / 256) * ((h[e.prob].n + 255) / 256);
        e.cost = 256.0 * 256.0 * (double)(h[e.prob].kp + 128);
      }
      if (kernel) *kernel = kI8Large;
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
  bool same = ne > 0;
  for (size_t j = 1; j < ne && same; ++j) same = ents[j].tiles == ents[0].tiles;
  img[2] = same ? ents[0].tiles : 0;
  info->tiles_main = (int)tot;
  info->tiles_splitk = 0;
  info->num_launches = tot > 0 ? 1 : 0;
  info->ws2_offset_ints = 0;
  info->bytes_used = sizeof(int) * (kSchedHdr + 2 * ne + 1);
  return 0;
}

I8Epi i8_epi_residue(uint32_t p, int kp) {
  const uint32_t mc = (uint32_t)((4294967296ull + p - 1) / p);
  if (kp <= kAccBiasMaxKp) return I8Epi{kEpiResidue | kEpiAccBias, p, mc, p * (((1u << 29) + p - 1) / p)};
  return I8Epi{kEpiResidue, p, mc, p * (uint32_t)((2147483648ull + p - 1) / p)};
}

namespace {
// the kernels' dynamic LDS exceeds the default limit: raise it once per device
bool lds_attrs_set() {
  static std::mutex mu;
  static std::vector<int> done;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  std::lock_guard<std::mutex> lk(mu);
  if ((int)done.size() <= dev) done.resize(dev + 1, 0);
  if (!done[dev]) {
    if (hipFuncSetAttribute((const void*)i8_grouped_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kSmem) !=
            hipSuccess ||
        hipFuncSetAttribute((const void*)i8_large_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kSmemL) !=
            hipSuccess)
      return false;
    done[dev] = 1;
  }
  return true;
}
}  // namespace

int i8_launch(const i8_problem* d_probs, const I8Epi* d_epi, const void* d_sched, const i8_sched_info* info,
              hipStream_t s, int kernel) {
  if (!info) return 1;
  if (info->num_launches == 0 || info->tiles_main == 0) return 0;
  if (!d_probs || !d_sched) return 1;
  if (!lds_attrs_set()) return 6;
  if (kernel == kI8Large)
    hipLaunchKernelGGL(i8_large_kernel, dim3((unsigned)info->tiles_main), dim3(kThreadsL), kSmemL, s, d_probs, d_epi,
                       static_cast<const int*>(d_sched));

  else
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
