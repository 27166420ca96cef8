// i8gemm.hip -- grouped INT8 x INT8 -> INT32 GEMM on gfx950 MFMA (exact accumulation).
//
// Problem (src/int8_grouped_gemm.h:4-10 layout): A m x kp and B n x kp row-major (K contiguous),
// C = A B^T column-major m x n (ld m), kp % 32 == 0, |C| <= 128^2 kp < 2^31 (kp <= 131040).
//
// One launch covers every (problem, plane) of a group, with persistent workgroups and a
// work-stealing tile scheduler (the reference's contract, src/int8_grouped_gemm.cu:360-407 and
// :602-675).  The host builds a tile table in longest-processing-time order (heaviest tiles
// first) and deals its entries -- whole (problem, plane) products -- to eight queues, one per XCD
// (MI355X deals workgroups round-robin to its 8 XCDs, b mod 8, each with its own L2): a product's
// residue panels are then read from HBM by one XCD only and shared through its L2 (on 8192^2 x
// 16384 products, spreading each product over all XCDs read 6.3 times the planes' bytes from HBM).
// A workgroup takes tiles from its own XCD's queue by an atomic counter, fetched one tile ahead,
// and once that queue is exhausted steals from the others in turn; the last workgroup to finish
// resets the counters.  Inside a product tiles are rastered in groups of G tile-rows, m fastest,
// so the compute units of an XCD share A and B panels in L2 (general kernel G = 8, large-tile
// kernel G = 4).  When a tile's last k-stage is in registers, the workgroup issues the next tile's
// first stages into the free LDS ring before its epilogue, so the operand stream does not drain
// between tiles.
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
#include <atomic>
#include <cmath>
#include <cstdlib>
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
// raster group (tile-rows) of the two kernels
constexpr int kGroupM = 8;    // general kernel
constexpr int kGroupML = 4;   // large-tile kernel

// Tile BM x BN computed by WGM x WGN waves through an NST-stage LDS ring of BK-byte k-stages.
template <int ID_, int BM_, int BN_, int WGM_, int WGN_, int NST_, int BK_ = kBK>
struct Cfg {
  static constexpr int ID = ID_;   // tile configuration number in the schedule's entries
  static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_, NST = NST_;
  static constexpr int BK = BK_;                       // k-bytes of a stage (64 or 128)
  static constexpr int CH = BK / 16, RP = 1024 / BK;   // 16-byte chunks per LDS row, rows per DMA piece
  static constexpr int NW = WGM * WGN, NT = 64 * NW;
  static constexpr int WM = BM / WGM, WN = BN / WGN;   // wave tile
  static constexpr int FM = WM / 16, FN = WN / 16;     // 16 x 16 MFMA blocks per wave
  static constexpr int SA = BM * BK, SB = BN * BK, STAGE = SA + SB;
  static constexpr int PA = SA / 1024, PB = SB / 1024; // 1 KB DMA pieces per operand and stage
  // a stage's A pieces then B pieces, dealt to the waves round-robin: piece g = wave + NW q
  static constexpr int VM = (PA + PB) / NW;            // DMA instructions per wave and stage
  static constexpr int SMEM = NST * STAGE;
  // k loop with the stage barrier between the two halves of a stage's MFMAs (below): pays for
  // the large-tile kernels (one workgroup per compute unit), not for the general kernel's two
  // workgroups
  static constexpr bool kSplit = BM * BN >= 256 * 256;
  static_assert((PA + PB) % NW == 0 && FM >= 1 && FN >= 1, "tile split");
  static_assert(BK == 64 || (BK == 128 && kSplit && NST == 2 && NW % 2 == 0 && PA % NW == 0), "128-byte stages");
};
// general kernel: 512 threads = 8 waves of (BM / 4) x (BN / 2), two workgroups per compute unit
// (72 KB of LDS each, four waves per SIMD); against 4 waves of (BM / 2) x (BN / 2) the 256 x 128
// tiles of 1024^3 products run 1.4-3 % faster (more waves hide the DMA and LDS waits)
using Cfg0 = Cfg<0, 256, 128, 4, 2, 3>;
using Cfg1 = Cfg<1, 128, 128, 4, 2, 3>;
using Cfg2 = Cfg<2, 64, 64, 4, 2, 3>;
constexpr int kThreads = 512;
// after a configuration's ring: the tile's row shifts (256 int) then its column shifts (256 int),
// for the non-finite check
constexpr int kTileCheckBytes = 2048;
constexpr int kSmem = Cfg0::SMEM + kTileCheckBytes;
static_assert(Cfg1::SMEM <= kSmem && Cfg2::SMEM <= kSmem, "smem");
// large-tile kernel: 1024 threads = 16 waves of 64 x 64 (4 per SIMD, so one wave's LDS reads and
// barrier waits overlap the others' MFMAs; 8 waves of 128 x 64, a quarter fewer LDS fragment
// bytes, measured 6 % slower), one workgroup per compute unit, 128 KB ring
constexpr int kLargeWGM = 4, kLargeWGN = 4;   // waves of the large-tile kernel
using CfgL = Cfg<0, 256, 256, kLargeWGM, kLargeWGN, 4>;
// the same tiles on row-major residues with 128-byte stages through a 2-stage ring of 64 KB: a
// stage's row is one whole 128-byte line, one L1 -> L2 request where 64-byte stages take two (the
// second, a stage later, an L2 hit); the per-CU request stream is what bounds this kernel, and
// 8192^2 x 16384 products run 5 % faster (119.0 -> 113.7 ms per launch, same box)
using CfgL128 = Cfg<0, 256, 256, kLargeWGM, kLargeWGN, 2, 128>;
constexpr int kThreadsL = CfgL::NT;
static_assert(CfgL128::NT == kThreadsL, "large-tile configurations");
constexpr int kSmemL = (CfgL::SMEM > CfgL128::SMEM ? CfgL::SMEM : CfgL128::SMEM) + kTileCheckBytes;

// LDS position of 16-byte chunk ch of a row of CH chunks: XOR with (row / 2) mod CH, so that the
// 16 lanes of a 128-bit fragment read (16 consecutive rows, one chunk) hit distinct banks
template <int CH>
__device__ __forceinline__ int swz(int row, int ch) { return ch ^ ((row >> 1) & (CH - 1)); }

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
// F fragments of consecutive 16-row blocks (BS bytes apart: 16 rows of the stage)
template <int F, int OFF0, int BS = 1024, int I = 0>
__device__ __forceinline__ void read_frags(v4i* f, uint32_t addr) {
  if constexpr (I < F) {
    f[I] = lds_read<OFF0 + I * BS>(addr);
    read_frags<F, OFF0, BS, I + 1>(f, addr);
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
  const int r_in = lane / C::CH, pc = lane % C::CH;
  auto piece_of = [&](const StageSrc& o, int rem, int piece, uint8_t* dst) {
    const int row = piece * C::RP + r_in;
    const int kk = 16 * swz<C::CH>(row, pc);
    const int rr = row < rem ? row : rem - 1;
    __builtin_amdgcn_global_load_lds((const void*)(o.base + (size_t)rr * o.stride + (kk < o.lim ? kk : 0)),
                                     GGEMM_LDS(dst + piece * 1024), 16, 0, 0);
  };
  for_pieces<C>(wave, [&](int piece) { piece_of(a, m_rem, piece, st); },
                [&](int piece) { piece_of(b, n_rem, piece, st + C::SA); });
}

// The same stage when every row of the tile exists and every chunk is inside the row (the common
// case): piece offsets are wave-uniform and the per-lane offset r_in stride + 16 swz(row, pc) is
// fixed for the tile (64-byte stages: the swizzle of row 16 piece + r_in depends on r_in only;
// 128-byte stages: on r_in and the parity of the piece, which is the wave's parity for every piece
// of the wave), so each DMA is a scalar base plus one per-lane offset.
template <class C>
__device__ __forceinline__ void dma_stage_full(const int8_t* a, const int8_t* b, int a_stride, int b_stride,
                                               uint32_t a_lane, uint32_t b_lane, uint8_t* st, int wave) {
  for_pieces<C>(
      wave,
      [&](int piece) {
        __builtin_amdgcn_global_load_lds((const void*)(a + (size_t)piece * C::RP * a_stride + a_lane),
                                         GGEMM_LDS(st + piece * 1024), 16, 0, 0);
      },
      [&](int piece) {
        __builtin_amdgcn_global_load_lds((const void*)(b + (size_t)piece * C::RP * b_stride + b_lane),
                                         GGEMM_LDS(st + C::SA + piece * 1024), 16, 0, 0);
      });
}

// A stage of a compacted tile: the tile's rows are entries row0 .. of the product's finite-row list
// and its columns entries col0 .. of its finite-column list (rm / cm: the tile's window of the lists
// in LDS, nr / nc entries from row0 / col0 on; rows past a list repeat its last, and their results
// are not stored), so each lane's row of each of its pieces is gathered; VM DMA instructions per
// wave, selects rather than branches between them.
template <class C, bool kPacked>
__device__ __forceinline__ void dma_stage_mapped(const int8_t* A, const int8_t* B, int m, int n, int kp, int k0,
                                                 const int* rm, const int* cm, int nr, int nc, uint8_t* st,
                                                 int wave, int lane) {
  const int r_in = lane / C::CH, pc = lane % C::CH;
#pragma unroll
  for (int q = 0; q < C::VM; ++q) {
    const int g = wave + C::NW * q;
    const bool isa = g < C::PA;
    const int piece = isa ? g : g - C::PA;
    const int row = piece * C::RP + r_in;
    const int kk = 16 * swz<C::CH>(row, pc);
    const int8_t* const plane = isa ? A : B;
    const int rows = isa ? m : n, lr = isa ? nr : nc;
    const int orow = (isa ? rm : cm)[row < lr ? row : lr - 1];
    size_t off;
    int lim;
    if (kPacked) {
      const int b = k0 >> 6, rb = b == (kp >> 6) ? 32 : 64;
      off = (size_t)b * rows * 64 + (size_t)orow * rb;
      lim = rb;
    } else {
      off = (size_t)orow * kp + k0;
      lim = kp - k0;
    }
    __builtin_amdgcn_global_load_lds((const void*)(plane + off + (kk < lim ? kk : 0)),
                                     GGEMM_LDS(st + (isa ? 0 : C::SA) + piece * 1024), 16, 0, 0);
  }
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
// or residue bytes, blocked or column-major (I8Epi).  Compacted tile (rmap != nullptr, blocked only):
// tile row r is product row rmap[r] (r < nr), tile column c product column cmap[c] (c < nc), each
// entry stored at its own place in the blocked layout.
template <class C>
__device__ __forceinline__ void tile_epilogue(const v4i (&acc)[C::FM][C::FN], const i8_problem& P, const I8Epi& epi,
                                              int row0, int col0, int wave, int lane, const int* rmap = nullptr,
                                              const int* cmap = nullptr, int nr = 0, int nc = 0) {
  constexpr int FM = C::FM, FN = C::FN;
  const int wm = wave % C::WGM, wn = wave / C::WGM;
  if (rmap) {
    const bool res = (epi.mode & kEpiResidue) != 0, accb = (epi.mode & kEpiAccBias) != 0;
    const int mb = (P.m + 15) / 16;
    GLOBAL uint8_t* const y8 = (GLOBAL uint8_t*)P.C;
    GLOBAL int32_t* const y32 = (GLOBAL int32_t*)P.C;
    static_for<0, FM * FN>([&](auto ij) {
      constexpr int i = decltype(ij)::value / FN, j = decltype(ij)::value % FN;
      const int cl = wn * C::WN + j * 16 + (lane & 15);
      if (cl < nc) {
        const int oc = cmap[cl];
        const v4i v = acc[i][j];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int rl = wm * C::WM + i * 16 + 4 * (lane >> 4) + r;
          if (rl < nr) {
            const int orr = rmap[rl];
            const size_t e = blocked_word(orr & ~3, oc, mb) + (size_t)(orr & 3);
            if (!res) y32[e] = v[r];
            else y8[e] = (uint8_t)(accb ? residue_byte<true>(v[r], epi) : residue_byte<false>(v[r], epi));
          }
        }
      }
    });
    return;
  }
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

// threadIdx.x, opaque to the optimizer: per-lane values derived from it are computed per tile
// instead of being hoisted out of the persistent loop (one set per tile configuration, live
// throughout, took the kernels past their register budget)
__device__ __forceinline__ int tile_tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// Operand stream of one tile: the DMA of its k-stage kt into an LDS ring slot.
template <class C, bool kPacked>
struct TileSrc {
  const int8_t* A;
  const int8_t* B;
  int m, n, kp, row0, col0, m_rem, n_rem;
  bool full_rows;
  uint32_t lane_off;
  int wave, lane;
  // compacted tile (rm != nullptr): rows tm BM .. of the finite-row list (rm: the tile's window of
  // it in LDS, nr = m_rem >= 1 entries from there on), columns tn BN .. of the finite-column list
  const int* rm = nullptr;
  const int* cm = nullptr;
  __device__ __forceinline__ TileSrc(const i8_problem& P, int tm, int tn, const int* rmap, const int* cmap, int nr,
                                     int nc)
      : A(P.A), B(P.B), m(P.m), n(P.n), kp(P.kp), row0(tm * C::BM), col0(tn * C::BN), m_rem(nr), n_rem(nc) {
    const int tid = tile_tid();
    lane = tid & 63;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    full_rows = false;
    lane_off = 0;
    rm = rmap;
    cm = cmap;
  }
  __device__ __forceinline__ TileSrc(const i8_problem& P, int tm, int tn)
      : A(P.A), B(P.B), m(P.m), n(P.n), kp(P.kp), row0(tm * C::BM), col0(tn * C::BN), m_rem(P.m - tm * C::BM),
        n_rem(P.n - tn * C::BN) {
    const int tid = tile_tid();
    lane = tid & 63;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // full stages: all tile rows exist and the stage has 64 bytes per row (packed: every k-block but
    // a final half block; row-major: every stage but a final half stage)
    full_rows = m_rem >= C::BM && n_rem >= C::BN;
    static_assert(!kPacked || C::BK == 64, "packed residues are 64-byte k-blocks");
    const int fstride = kPacked ? 64 : kp;
    const int r_in = lane / C::CH;
    lane_off = (uint32_t)(r_in * fstride + 16 * swz<C::CH>(wave * C::RP + r_in, lane % C::CH));
  }
  __device__ __forceinline__ void load(int kt, uint8_t* st) const {
    const int k0 = kt * C::BK;
    if (rm) {
      dma_stage_mapped<C, kPacked>(A, B, m, n, kp, k0, rm, cm, m_rem, n_rem, st, wave, lane);
      return;
    }
    if (full_rows && k0 + C::BK <= kp) {
      const int8_t* a = kPacked ? A + (size_t)(k0 >> 6) * m * 64 + (size_t)row0 * 64 : A + (size_t)row0 * kp + k0;
      const int8_t* b = kPacked ? B + (size_t)(k0 >> 6) * n * 64 + (size_t)col0 * 64 : B + (size_t)col0 * kp + k0;
      dma_stage_full<C>(a, b, kPacked ? 64 : kp, kPacked ? 64 : kp, lane_off, lane_off, st, wave);
    } else {
      dma_stage<C>(stage_src(A, m, row0, kp, k0, kPacked), stage_src(B, n, col0, kp, k0, kPacked), m_rem, n_rem, st,
                   wave, lane);
    }
  }
  // stage kt by the general form only: VM DMA instructions per wave with no branch between them
  // and the ones of the next stage (the count the tile check's wait relies on)
  __device__ __forceinline__ void load_general(int kt, uint8_t* st) const {
    const int k0 = kt * C::BK;
    dma_stage<C>(stage_src(A, m, row0, kp, k0, kPacked), stage_src(B, n, col0, kp, k0, kPacked), m_rem, n_rem, st,
                 wave, lane);
  }
  // the stages a tile's k loop expects in flight when it starts (ring slots 0, 1, ...): NST with the
  // split loop, NST - 1 otherwise
  __device__ __forceinline__ void prologue(uint8_t* lds) const {
    constexpr int PRE = C::kSplit ? C::NST : C::NST - 1;
    const int nk = (kp + C::BK - 1) / C::BK;
#pragma unroll
    for (int q = 0; q < PRE; ++q)
      if (q < nk) load(q, lds + q * C::STAGE);
  }
};

__device__ __forceinline__ I8Epi epi_of(const I8Epi* __restrict__ epis, int pi) {
  return epis ? epis[pi] : I8Epi{0u, 1u, 0u, 0u, nullptr, nullptr, nullptr};
}

// A unit of the persistent schedule, decoded: one tile (tm, tn) of product pi (< 0: none).
struct Unit {
  int pi, cfg, tm, tn;
};

// One tile: the k loop over its stages and the epilogue.  The tile's prologue stages (TileSrc::
// prologue) are in flight when it starts.  kFresh: they are this workgroup's only memory operations
// in flight (a workgroup that runs one tile), so the first wait lets the later prologue stages
// stay in flight; otherwise (persistent workgroups) the previous tile's epilogue stores may be
// in flight too, and the first wait is a full one.
// claim(): called by every thread once, after the tile's last stage has landed (no operand load of
// this tile is in flight any more); it starts the fetch of the workgroup's next unit.  next():
// called by every thread once, after the last stage's MFMAs are issued and before the epilogue; it
// passes a workgroup barrier, after which no wave reads this tile's LDS ring, and returns the next
// unit.  When that unit has this tile's configuration its prologue is issued here, ahead of the
// epilogue (returns true), so the operand ring keeps streaming across tiles.
template <class C, bool kPacked, bool kFresh, class Claim, class Next>
__device__ __forceinline__ bool run_tile(uint8_t* lds, const i8_problem* __restrict__ probs,
                                         const I8Epi* __restrict__ epis, int pi, int tm, int tn, Claim&& claim,
                                         Next&& next, const int* rmap = nullptr, const int* cmap = nullptr,
                                         int nr = 0, int nc = 0) {
  const i8_problem& P = probs[pi];
  const I8Epi epi = epi_of(epis, pi);
  constexpr int FM = C::FM, FN = C::FN, NST = C::NST;
  const TileSrc<C, kPacked> src = rmap ? TileSrc<C, kPacked>(P, tm, tn, rmap, cmap, nr, nc) : TileSrc<C, kPacked>(P, tm, tn);
  const int tid = tile_tid(), lane = tid & 63, wave = src.wave;
  const int wm = wave % C::WGM, wn = wave / C::WGM;
  const int kp = P.kp;
  constexpr int BK = C::BK, BS = 16 * BK;   // stage width, bytes of 16 LDS rows (one fragment block)
  const int nk = (kp + BK - 1) / BK;
  __builtin_assume(nk > 0);   // scheduled tiles have kp > 0
  bool prefetched = false;
  auto handoff = [&]() {
    const Unit nx = next();
    if (nx.pi >= 0 && nx.cfg == C::ID && ((epi_of(epis, nx.pi).mode & kEpiPacked) != 0) == kPacked) {
      TileSrc<C, kPacked>(probs[nx.pi], nx.tm, nx.tn).prologue(lds);
      prefetched = true;
    }
  };

  // fragment addresses: rows wm WM + 16 i + lane % 16 (A), wn WN + 16 j + lane % 16 (B), chunk lane / 16
  // (+ 4 for the second 64-byte half of a 128-byte stage); the swizzle depends on row / 2 mod CH
  // only, so blocks i, j sit at fixed immediates BS bytes apart
  const int fr = lane & 15, fc = lane >> 4;
  const uint32_t lbase = (uint32_t)(uintptr_t)GGEMM_LDS(lds);
  const int ra = wm * C::WM + fr, rb = wn * C::WN + fr;
  const uint32_t a_addr = lbase + ra * BK + swz<C::CH>(ra, fc) * 16;
  const uint32_t b_addr = lbase + rb * BK + swz<C::CH>(rb, fc) * 16;

  const int a0 = (epi.mode & kEpiAccBias) ? (int)epi.bias : 0;   // accumulator start
  v4i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4i{a0, a0, a0, a0};

  // a final partial stage (k in [kp, kp + BK) not all inside the row): zero A's chunks from the
  // first one past kp (B's are duplicates of chunk 0)
  const int tail = kp % BK;   // valid bytes of the last stage (0: all)
  auto zero_half = [&](uint8_t* st) {
    const int c0 = tail / 16, nz = C::CH - c0;
    for (int c = tid; c < C::BM * nz; c += C::NT) {
      const int row = c / nz, ch = c0 + c % nz;
      *reinterpret_cast<uint4*>(st + row * BK + swz<C::CH>(row, ch) * 16) = make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto mfmas = [&](const v4i* a, const v4i (&b)[FN], int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
  };
  if constexpr (BK == 128) {
    // 128-byte stages, stage s in ring slot s mod 2; a stage is two 64-byte k-halves.  Iteration kt
    // holds stage kt's first-half fragments: it issues their MFMAs, reads and waits for the second
    // half's, issues the MFMAs of its first H A blocks, then (those queued on the matrix core) waits
    // for stage kt + 1 and passes the barrier, refills slot kt with stage kt + 2, reads stage kt + 1's
    // first-half A fragments of blocks 0 .. H into the registers just consumed, issues the second
    // half's remaining MFMAs and reads the rest of stage kt + 1's first-half fragments.
    constexpr int H = FM / 2;
    const uint32_t a_addr2 = lbase + ra * BK + swz<C::CH>(ra, fc + 4) * 16;
    const uint32_t b_addr2 = lbase + rb * BK + swz<C::CH>(rb, fc + 4) * 16;
    // stage 0 landed (with kFresh, stage 1 may still be in flight)
    if (kFresh && 1 < nk) wait_barrier<C::VM>(); else wait_barrier<0>();
    if (nk == 1) claim();
    if (nk == 1 && tail) {
      zero_half(lds);
      wait_barrier<0>();
    }
    v4i a[FM], b[FN];
    read_frags<FN, C::SA, BS>(b, b_addr);
    read_frags<FM, 0, BS>(a, a_addr);
    int buf = 0;
    for (int kt = 0; kt < nk; ++kt) {
      const uint32_t so = (uint32_t)(buf * C::STAGE);
      lds_wait_frags<FM, FN>(a, b);   // stage kt, first half
      mfmas(a, b, 0, FM);
      read_frags<FN, C::SA, BS>(b, b_addr2 + so);
      read_frags<FM, 0, BS>(a, a_addr2 + so);
      lds_wait_frags<FM, FN>(a, b);   // stage kt, second half
      mfmas(a, b, 0, H);
      const bool more = kt + 1 < nk;
      const int nb = buf ^ 1;
      const uint32_t sn = (uint32_t)(nb * C::STAGE);
      if (more) {
        // stage kt + 1 landed (the only DMA in flight) and every wave has read stage kt
        wait_barrier<0>();
        if (kt + 2 == nk) claim();   // the last stage landed
        if (kt + 2 < nk) src.load(kt + 2, lds + buf * C::STAGE);
        if (kt + 2 == nk && tail) {
          zero_half(lds + nb * C::STAGE);
          wait_barrier<0>();
        }
        read_frags<H, 0, BS>(a, a_addr + sn);
      }
      mfmas(a, b, H, FM);
      if (more) {
        read_frags<FM - H, H * BS, BS>(a + H, a_addr + sn);
        read_frags<FN, C::SA, BS>(b, b_addr + sn);
      }
      buf = nb;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    handoff();   // every wave has issued the last stage's MFMAs: the ring is free
  } else if constexpr (C::kSplit) {
    // Stage s in ring slot s mod NST.  Iteration kt holds stage kt's fragments in registers: it
    // issues the MFMAs of the first half of the A blocks, then (those queued on the matrix core)
    // waits for stage kt + 1 and passes the barrier, refills slot kt (every wave holds its
    // fragments) with stage kt + NST, reads stage kt + 1's first-half A fragments into the
    // registers just consumed, issues the second half and reads the rest of stage kt + 1.  The
    // barrier and the LDS latency overlap queued MFMA work (16-wave kernel: 2.4 % at k = 16384).
    constexpr int H = FM / 2;
    // stage 0 landed (with kFresh, stages 1 .. NST - 1 may still be in flight)
    if (kFresh && NST - 1 < nk) wait_barrier<(NST - 1) * C::VM>(); else wait_barrier<0>();
    if (nk == 1) claim();
    if (nk == 1 && tail) {
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
        if (kt + 2 == nk) claim();   // the last stage landed
        if (kt + NST < nk) src.load(kt + NST, lds + buf * C::STAGE);
        if (kt + 2 == nk && tail) {
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
    handoff();   // every wave has issued the last stage's MFMAs: the ring is free
  } else {
    // Stage kt waits, passes the barrier (every wave is done with stage kt - 1), refills slot
    // kt - 1 with stage kt + NST - 1, reads all its fragments and issues every MFMA.  With two
    // workgroups per compute unit the other workgroup's MFMAs cover this one's waits.
    int buf = 0;
    for (int kt = 0; kt < nk; ++kt) {
      // stage kt landed (the NST - 2 stages after it may still be in flight; near the end fewer
      // were issued, and at kt = 0 the previous tile's stores may be, so wait for everything) and
      // every wave is done with stage kt - 1
      if ((kFresh || kt > 0) && kt + NST - 2 < nk) wait_barrier<(NST - 2) * C::VM>(); else wait_barrier<0>();
      if (kt + NST - 1 < nk) {
        int b2 = buf + NST - 1;   // the ring slot of stage kt - 1
        if (b2 >= NST) b2 -= NST;
        src.load(kt + NST - 1, lds + b2 * C::STAGE);
      }
      if (kt == nk - 1 && tail) {
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
    // after the last MFMAs (a claim any earlier in this loop took the kernel past 128 VGPRs, i.e.
    // one workgroup per compute unit); the other workgroup's MFMAs cover the fetch
    claim();
    handoff();   // every wave has issued the last stage's MFMAs: the ring is free
  }

  // the epilogue's descriptor fields are read again here rather than kept live through the k loop
  int pi_e = pi;
  asm volatile("" : "+s"(pi_e));
  tile_epilogue<C>(acc, probs[pi_e], epi_of(epis, pi_e), src.row0, src.col0, wave, lane, rmap, cmap, nr, nc);
  return prefetched;
}

// ---------------------------------------------------------------- persistent tile scheduler
// Schedule image (ints; built by i8_build_schedule):
//   [0] units (tiles) in all, [1] entries, [2] tiles per entry when all entries have the same count
//   (else 0), [3] chunk c (> 0: queue x is chunks x, x + 8, ... of c consecutive units instead of a
//   range), [kHdrHw] the units the 256 x 256 kernel dispatches one workgroup each (its tail takes
//   the rest, through the counters below); [kHdrXcd + x], x = 0..8: first unit of XCD x's queue
//   (x = 8: the total);
//   [kHdrCtr + x], x < 8: XCD x's queue counter, [kHdrDone]: workgroups finished -- zero in the
//   uploaded image and reset by the last workgroup of every launch, so a captured graph replays
//   without clearing them; prefix[entries + 1] at kSchedHdr (first unit of each entry),
//   entry[entries] = (problem << 2) | tile config.
// Entries (whole (problem, plane) products) are dealt to the eight XCD queues by the host, heaviest
// first onto the least loaded queue, so a product's residue panels are read from HBM by one XCD
// and shared in its L2; a workgroup takes the units of its own XCD's queue (blockIdx mod 8: the
// dispatcher deals workgroups to the XCDs round-robin) through the queue counter and, once that
// is exhausted, steals from the other queues in turn.
static_assert(kHdrDone < kSchedHdr, "schedule header");

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
// the local index of tile (tm, tn) in raster<GM>'s order
template <int GM>
__device__ __forceinline__ int raster_local(int tm, int tn, int m, int n, int bm, int bn) {
  const int tiles_m = (m + bm - 1) / bm, tiles_n = (n + bn - 1) / bn;
  const int g = tm / GM, first_m = g * GM, gsz = min(GM, tiles_m - first_m);
  return g * GM * tiles_n + tn * gsz + (tm - first_m);
}
// unit u (wave-uniform, >= 0) -> problem, tile configuration and tile position
template <int GM, bool kLarge>
__device__ __forceinline__ Unit decode_unit(const int* __restrict__ sched, const i8_problem* __restrict__ probs, int u) {
  const int ne = sched[1], per = sched[2];
  const int* prefix = sched + kSchedHdr;
  const int* entry = prefix + ne + 1;
  int e, local;
  if (per > 0) {
    e = u / per;
    local = u - e * per;
  } else {
    int lo = 0, hi = ne - 1;   // largest e with prefix[e] <= u
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (prefix[mid] <= u) lo = mid; else hi = mid - 1;
    }
    e = lo;
    local = u - prefix[lo];
  }
  const int ev = entry[e];
  Unit t;
  t.pi = ev >> 2;
  t.cfg = ev & 3;
  raster<GM>(local, probs[t.pi].m, probs[t.pi].n, kLarge ? 256 : i8_tile_m(t.cfg), kLarge ? 256 : i8_tile_n(t.cfg),
             t.tm, t.tn);
  return t;
}
// the next local index of queue q from its counter: past the n_q workgroups' first tiles
__device__ __forceinline__ int fetch_local(int* __restrict__ sched, int q) {
  const int nq = ((int)gridDim.x - q + kXcds - 1) / kXcds;
  return atomicAdd(sched + kHdrCtr + q, 1) + nq;
}
// Thread 0 only.  Queue q's units in order are its local indices 0, 1, ...; the workgroups of XCD q
// (blockIdx = q mod 8, n_q of them) start on local indices 0 .. n_q - 1 without a fetch, and a
// value v fetched from the queue's counter names local index n_q + v.  So the first round of tiles
// of an XCD is one contiguous run of its queue, as every later round is approximately (a fetch that
// raced ahead of other workgroups' first tiles would scatter the first round over twice as many
// products, more than the XCD's L2 holds).  l: a local index of the queue qi steps after the own
// one.  Returns the unit it names or, when that queue is exhausted, moves to the next queue (the
// own XCD's first, then the others in turn, each once) and fetches again; -1 when all are
// exhausted.
__device__ __forceinline__ int resolve_unit(int* __restrict__ sched, int own, int& qi, int l) {
  const int ch = sched[3];
  for (;;) {
    const int q = (own + qi) & (kXcds - 1);
    if (ch > 0) {   // queue q: chunks q, q + 8, q + 16, ... of ch consecutive units
      const int u = ((l / ch) * kXcds + q) * ch + l % ch;
      if (u < sched[0]) return u;
    } else {        // queue q: the units [first(q), first(q + 1))
      const int u = sched[kHdrXcd + q] + l;
      if (u < sched[kHdrXcd + q + 1]) return u;
    }
    if (++qi == kXcds) return -1;
    l = fetch_local(sched, (own + qi) & (kXcds - 1));
  }
}

// The persistent workgroup: takes units until every queue is exhausted.  The next unit is fetched
// when the current tile's last stage has landed (its counter atomic then overlaps the last stage's
// MFMAs; fetched any earlier, the claims of an XCD's workgroups interleave across rounds and its
// tiles in flight span more products than its L2 holds -- measured 1.6 times the HBM reads), and
// handed to the current tile before its epilogue.  pro(unit) issues a unit's prologue; run(unit,
// claim, next) runs one unit and returns whether it issued the next unit's prologue.
template <int GM, bool kLarge, class Pro, class Run>
__device__ __forceinline__ void persistent(int* __restrict__ sched, const i8_problem* __restrict__ probs, Pro&& pro,
                                           Run&& run) {
  __shared__ int s_unit[2];
  const int tid = threadIdx.x;
  const int own = blockIdx.x & (kXcds - 1);
  int qi = 0, pend = 0;   // thread 0: queues exhausted so far, the local index of the fetch in flight
  if (tid == 0) s_unit[0] = resolve_unit(sched, own, qi, (int)blockIdx.x / kXcds);
  __syncthreads();
  const int u0 = __builtin_amdgcn_readfirstlane(s_unit[0]);
  Unit cur{-1, 0, 0, 0};
  if (u0 >= 0) cur = decode_unit<GM, kLarge>(sched, probs, u0);
  bool pre = false;
  for (int it = 1; cur.pi >= 0; ++it) {
    Unit nxt{-1, 0, 0, 0};
    auto claim = [&]() {
      if (tid == 0 && qi < kXcds) pend = fetch_local(sched, (own + qi) & (kXcds - 1));
    };
    auto next = [&]() -> Unit {
      if (tid == 0) s_unit[it & 1] = qi < kXcds ? resolve_unit(sched, own, qi, pend) : -1;
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      const int nu = __builtin_amdgcn_readfirstlane(s_unit[it & 1]);
      if (nu >= 0) nxt = decode_unit<GM, kLarge>(sched, probs, nu);
      return nxt;
    };
    if (!pre) pro(cur);
    pre = run(cur, claim, next);
    cur = nxt;
  }
  // every fetch of this workgroup has returned (its value was used): the last workgroup to finish
  // resets the queue counters for the next launch
  if (tid == 0) {
    __threadfence();
    if (atomicAdd(sched + kHdrDone, 1) == (int)gridDim.x - 1) {
      for (int x = 0; x < kXcds; ++x) atomicExch(sched + kHdrCtr + x, 0);
      atomicExch(sched + kHdrDone, 0);
    }
  }
}

// ---------------------------------------------------------------- hardware-dispatched kernels
// One workgroup per tile; the dispatcher hands workgroups to free compute-unit slots in index order,
// i.e. the tiles in LPT order to whichever unit frees first -- the same greedy list schedule as the
// persistent kernel's queue, kept by the command processor (measured faster on MI355X, see the
// launcher).  Workgroup b takes tile chunk (b mod 8) + 8 (b / (8 CH)) of CH consecutive tiles of the
// table, so one XCD works through contiguous runs (general kernel CH = 32: a 1024^2 product's 32
// tiles share one L2 and each plane is read from HBM once; large-tile kernel CH = 16).
constexpr int kChunk = 32, kChunkL = 16, kChunkT = 32;
// (workgroup b of the first `total` ones)
template <int CH>
__device__ __forceinline__ int dispatched_unit(int total) {
  const int b = blockIdx.x;
  const int span = kXcds * CH;
  const int full = total / span * span;
  if (b >= full) return b;
  const int x = b % kXcds, q = b / kXcds;
  return (q / CH) * span + x * CH + (q % CH);
}
// Finite-row / finite-column lists (bytes 0 / 1 in index order, 4-byte aligned, bytes past the
// list's length ignored), read as words.
__device__ __forceinline__ uint32_t flag_word(const uint32_t* __restrict__ fw, int total, int x) {
  const int nb = total - 4 * x;
  return nb >= 4 ? fw[x] : fw[x] & ((1u << (8 * nb)) - 1u);
}
__device__ __forceinline__ int flag_sum(uint32_t w) { return (int)((w * 0x01010101u) >> 24); }

// The set flags of both lists counted by the workgroup; ws: 2 NT / 64 ints of LDS.  One barrier.
template <int NT>
__device__ __forceinline__ int2 count_lists(const uint8_t* __restrict__ fr, int m, const uint8_t* __restrict__ fc,
                                            int n, int* ws) {
  const int t = tile_tid(), lane = t & 63, w = t >> 6;
  const uint32_t* __restrict__ rw = reinterpret_cast<const uint32_t*>(fr);
  const uint32_t* __restrict__ cw = reinterpret_cast<const uint32_t*>(fc);
  int cr = 0, cc = 0;
  for (int x = t; x < (m + 3) >> 2; x += NT) cr += flag_sum(flag_word(rw, m, x));
  for (int x = t; x < (n + 3) >> 2; x += NT) cc += flag_sum(flag_word(cw, n, x));
#pragma unroll
  for (int o = 32; o; o >>= 1) {
    cr += __shfl_xor(cr, o);
    cc += __shfl_xor(cc, o);
  }
  if (lane == 0) {
    ws[2 * w] = cr;
    ws[2 * w + 1] = cc;
  }
  __syncthreads();
  int2 r = make_int2(0, 0);
#pragma unroll
  for (int q = 0; q < NT / 64; ++q) {
    r.x += ws[2 * q];
    r.y += ws[2 * q + 1];
  }
  return r;
}

// Entries lo .. lo + win - 1 of the list of the set flags f[0 .. total) into map[0 .. win) (as far
// as the list goes); ws: NT / 64 ints of LDS.  Thread t takes words [t per, (t + 1) per): the
// workgroup's exclusive prefix of their flag counts gives its first list position, and it walks
// its words' flags that fall in the window.  Barriers at both ends.
template <int NT>
__device__ __forceinline__ void select_list(const uint8_t* __restrict__ f, int total, int lo, int win, int* map,
                                            int* ws) {
  const int t = tile_tid(), lane = t & 63, w = t >> 6;
  const uint32_t* __restrict__ fw = reinterpret_cast<const uint32_t*>(f);
  const int words = (total + 3) >> 2, per = (words + NT - 1) / NT;
  const int x0 = min(words, t * per), x1 = min(words, x0 + per);
  int c = 0;
  for (int x = x0; x < x1; ++x) c += flag_sum(flag_word(fw, total, x));
  int inc = c;   // inclusive prefix in the wave
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(inc, o);
    if (lane >= o) inc += y;
  }
  if (lane == 63) ws[w] = inc;
  __syncthreads();
  int pos = inc - c;
#pragma unroll
  for (int q = 0; q < NT / 64; ++q) pos += q < w ? ws[q] : 0;
  for (int x = x0; x < x1 && pos < lo + win; ++x) {
    uint32_t v = flag_word(fw, total, x);
    for (; v != 0u && pos < lo + win; v &= v - 1u, ++pos)
      if (pos >= lo) map[pos - lo] = 4 * x + (__builtin_ctz(v) >> 3);
  }
  __syncthreads();
}

// A unit of a product whose prep found NaN / Inf rows or columns computes, if any, one tile of the
// finite rows x finite columns (every other entry takes the safety fallback, which uses neither
// digits nor L): the tcm x tcn tiles over the finite-row and finite-column lists (prep's flags) are
// dealt to every s-th of the product's units in raster order, s = units / tiles, from a rotating
// offset, so that they spread over the dispatch chunks and with them over the XCDs (the first
// units of a product share one chunk); the other units end after the count.  The lists' windows go to the
// tile-check LDS area after the ring, the operand pieces are gathered row by row, and the epilogue
// stores each entry at its own row and column: the digits and L of the finite entries are those of
// the whole product's tiles, since an entry's products do not depend on its tile.
template <class C, bool kPacked>
__device__ __forceinline__ void compacted_tile(uint8_t* lds, const i8_problem* __restrict__ probs,
                                               const I8Epi* __restrict__ epis, const Unit& t, const YDesc* yd) {
  static_assert(C::BM + C::BN <= kTileCheckBytes / 4, "list windows in the tile-check area");
  static_assert(C::BM == 256 && C::BN == 256, "units of the large-tile raster");
  const i8_problem& P = probs[t.pi];
  int* const ws = reinterpret_cast<int*>(lds);   // the ring is idle until the prologue below
  // the descriptor is constant in this kernel: scalar loads
  const auto* const ydc = (const __attribute__((address_space(4))) YDesc*)yd;
  const uint8_t* const fr = ydc->fr;
  const uint8_t* const fc = ydc->fc;
  const int2 cnt = count_lists<C::NT>(fr, P.m, fc, P.n, ws);
  const int tcm = (cnt.x + C::BM - 1) / C::BM, tcn = (cnt.y + C::BN - 1) / C::BN, nt = tcm * tcn;
  if (nt == 0) return;   // workgroup-uniform
  const int units = ((P.m + C::BM - 1) / C::BM) * ((P.n + C::BN - 1) / C::BN);
  // tile i at local unit off + i s, off = (pi kChunkL) mod s: the product's first tile rotates over
  // its chunks from product to product
  const int s = units / nt, off = (int)(((unsigned)t.pi * (unsigned)kChunkL) % (unsigned)s);
  const int local = raster_local<kGroupML>(t.tm, t.tn, P.m, P.n, C::BM, C::BN) - off;
  if (local < 0 || local % s != 0 || local / s >= nt) return;
  const int i = local / s, cm = i % tcm, cn = i / tcm;
  int* const rmap = reinterpret_cast<int*>(lds + C::SMEM);
  int* const cmap = rmap + C::BM;
  int* const ws2 = ws + 2 * (C::NT / 64);   // the counts' words may still be read
  select_list<C::NT>(fr, P.m, cm * C::BM, C::BM, rmap, ws2);
  select_list<C::NT>(fc, P.n, cn * C::BN, C::BN, cmap, ws2);
  const int nr = cnt.x - cm * C::BM, nc = cnt.y - cn * C::BN;
  TileSrc<C, kPacked>(P, cm, cn, rmap, cmap, nr, nc).prologue(lds);
  run_tile<C, kPacked, true>(lds, probs, epis, t.pi, cm, cn, [] {}, [] { return Unit{-1, 0, 0, 0}; }, rmap, cmap,
                             nr, nc);
}

// One hardware-dispatched tile.  With the product's reconstruct descriptor given (epi.yd, 256 x
// 256 tiles on packed residues) and its non-finite flag set by prep, the unit computes a compacted
// tile instead (compacted_tile).  Otherwise, with the product's shifts given (epi.nf) and the flag
// set, a tile whose rows or whose columns are all non-finite is dropped: every entry of it takes
// the safety fallback.  Only on tiles of at least PRE stages.  Each wave DMAs 64 of the tile's row shifts and 64 of its
// column shifts (indices clamped to the product: a clamped copy is the last row / column, which is
// in the tile) to LDS after the ring, ahead of the first PRE stages, which are issued in the general
// form (VM DMA instructions per wave and stage, no branch between them).  With the flag set (a
// scalar load, landed by then), waiting until PRE VM DMA instructions are outstanding leaves those
// stages in flight; every wave then reads all the shifts and reaches the same verdict.  Without the
// flag the shift DMAs are only older operations ahead of the ring's own waits.
template <class C, bool kPacked>
__device__ __forceinline__ void one_tile(uint8_t* lds, const i8_problem* __restrict__ probs,
                                         const I8Epi* __restrict__ epis, const Unit& t) {
  static_assert(C::BM % 64 == 0 && C::BN % 64 == 0 && C::BM <= 256 && C::BN <= 256, "shift rows");
  static_assert(C::NW >= C::BM / 64 && C::NW >= C::BN / 64, "one shift DMA per wave and operand");
  constexpr int PRE = C::kSplit ? C::NST : C::NST - 1;
  const i8_problem& P = probs[t.pi];
  const TileSrc<C, kPacked> src(P, t.tm, t.tn);
  const I8Epi e = epi_of(epis, t.pi);
  // compacted tiles in the 256 x 256 kernel on packed residues only: a second copy of the tile's k
  // loop takes the general kernel past the 128 VGPRs of its two workgroups per CU, and the
  // row-major copy the large kernel past its budget (spills); the others keep the tile check below
  constexpr bool kCompact = C::kSplit && kPacked;
  if (kCompact && e.yd != nullptr) {   // workgroup-uniform: a product whose finite rows / columns prep lists
    // the flag first (a scalar load): a compacted product's units that hold no tile then end
    // without any operand load in flight
    if (*(const __attribute__((address_space(4))) int*)e.nf) {
      if constexpr (kCompact) compacted_tile<C, kPacked>(lds, probs, epis, t, e.yd);
      return;
    }
    src.prologue(lds);
  } else if (e.nf != nullptr && P.kp > (PRE - 1) * C::BK) {   // workgroup-uniform
    // written by prep, an earlier kernel of the call, and constant here: a scalar load
    const int nff = *(const __attribute__((address_space(4))) int*)e.nf;
    const int lane = src.lane, wave = src.wave;
    uint8_t* const chk = lds + C::SMEM;
    const int wr = wave % (C::BM / 64), wc = wave % (C::BN / 64);
    const int r = min(src.row0 + 64 * wr + lane, P.m - 1), c = min(src.col0 + 64 * wc + lane, P.n - 1);
    __builtin_amdgcn_global_load_lds((const void*)(e.rs + r), GGEMM_LDS(chk + 256 * wr), 4, 0, 0);
    __builtin_amdgcn_global_load_lds((const void*)(e.cs + c), GGEMM_LDS(chk + 1024 + 256 * wc), 4, 0, 0);
#pragma unroll
    for (int q = 0; q < PRE; ++q) src.load_general(q, lds + q * C::STAGE);
    if (nff) {
      wait_barrier<PRE * C::VM>();   // every wave's shift DMAs have landed
      const uint32_t base = (uint32_t)(uintptr_t)GGEMM_LDS(chk) + 16 * lane;
      v4i sr = lds_read<0>(base), sc = lds_read<1024>(base);
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(sr), "+v"(sc));
      bool fr = false, fc = false;
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        fr = fr || (4 * lane + x < C::BM && sr[x] != OZ2_SHIFT_NONFINITE);
        fc = fc || (4 * lane + x < C::BN && sc[x] != OZ2_SHIFT_NONFINITE);
      }
      if (__ballot(fr) == 0 || __ballot(fc) == 0) {   // no finite row, or no finite column
        wait_barrier<0>();   // the stages have landed before the workgroup ends
        return;
      }
    }
  } else {
    src.prologue(lds);
  }
  run_tile<C, kPacked, true>(lds, probs, epis, t.pi, t.tm, t.tn, [] {}, [] { return Unit{-1, 0, 0, 0}; });
}

__global__ void __launch_bounds__(kThreads, 2) i8_grouped_kernel(const i8_problem* __restrict__ probs,
                                                                 const I8Epi* __restrict__ epis,
                                                                 int* __restrict__ sched) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  const Unit t = decode_unit<kGroupM, false>(sched, probs, dispatched_unit<kChunk>(sched[0]));
  const bool pk = (epi_of(epis, t.pi).mode & kEpiPacked) != 0;
  switch (t.cfg) {
    case 0: pk ? one_tile<Cfg0, true>(lds, probs, epis, t) : one_tile<Cfg0, false>(lds, probs, epis, t); break;
    case 1: pk ? one_tile<Cfg1, true>(lds, probs, epis, t) : one_tile<Cfg1, false>(lds, probs, epis, t); break;
    default: pk ? one_tile<Cfg2, true>(lds, probs, epis, t) : one_tile<Cfg2, false>(lds, probs, epis, t); break;
  }
}

// Every tile of the schedule is a 256 x 256 tile.  kTail false: one workgroup per unit.  kTail
// true (launched when the schedule puts the products that may compact last, sched[kHdrHw] = hw
// units before them): workgroups below hw take one unit each, and the tail workgroups, the rest of
// the grid, take the units [hw, total) from work queues (below), so that a compacting product's
// units without a tile cost a loop step, not a workgroup dispatch.  Two instantiations, so that the
// one-workgroup-per-unit kernel keeps its registers and code without the tail loop.
template <bool kTail>
__global__ void __launch_bounds__(kThreadsL, 1) i8_large_kernel(const i8_problem* __restrict__ probs,
                                                                const I8Epi* __restrict__ epis,
                                                                int* __restrict__ sched) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  if constexpr (!kTail) {
    const Unit t = decode_unit<kGroupML, true>(sched, probs, dispatched_unit<kChunkL>(sched[0]));
    if (epi_of(epis, t.pi).mode & kEpiPacked) one_tile<CfgL, true>(lds, probs, epis, t);
    else one_tile<CfgL128, false>(lds, probs, epis, t);
    return;
  }
  __shared__ int s_unit, s_hw, s_total, s_q;   // tail: the next unit (< 0: none), the header's hw and
                                               // total, queues left behind (thread 0's state)
  const int hw0 = sched[kHdrHw];
  if ((int)blockIdx.x < hw0) {   // workgroup-uniform
    const Unit t = decode_unit<kGroupML, true>(sched, probs, dispatched_unit<kChunkL>(hw0));
    if (epi_of(epis, t.pi).mode & kEpiPacked) one_tile<CfgL, true>(lds, probs, epis, t);
    else one_tile<CfgL128, false>(lds, probs, epis, t);
    return;
  }
  // The tail's queues: queue q holds the chunks q, q + 8, q + 16, ... of kChunkT consecutive units
  // of [hw, total); the tail workgroups of XCD q (blockIdx = q mod 8: the dispatcher deals
  // workgroups to the XCDs round-robin) start on its local indices 0 .. n_q - 1 and then fetch
  // n_q + counter q, so an XCD works through contiguous runs of units (a product's operand panels
  // shared in its L2); an exhausted queue sends the workgroup to the next one in turn.  Thread 0
  // keeps the state in LDS, not across the tile in registers.
  if (threadIdx.x == 0) {
    s_hw = hw0;
    s_total = sched[0];
    s_q = 0;
  }
  const int own = (int)blockIdx.x & (kXcds - 1);
  auto tail_wgs = [&](int q) {   // tail workgroups of XCD q
    const int f = s_hw + (((q - s_hw) % kXcds) + kXcds) % kXcds;
    return f < (int)gridDim.x ? ((int)gridDim.x - f + kXcds - 1) / kXcds : 0;
  };
  auto unit_of = [&](int q, int l) {   // local index l of queue q -> unit, or -1 past its end
    const long long v = s_hw + ((long long)(l / kChunkT) * kXcds + q) * kChunkT + l % kChunkT;
    return v < s_total ? (int)v : -1;
  };
  // thread 0: the unit of local index l of the current queue, else the next queues' fetches; -1
  // when every queue is exhausted
  auto resolve = [&](int l) {
    for (;;) {
      const int q = (own + s_q) & (kXcds - 1);
      const int v = unit_of(q, l);
      if (v >= 0) return v;
      if (++s_q == kXcds) return -1;
      const int q2 = (own + s_q) & (kXcds - 1);
      l = tail_wgs(q2) + atomicAdd(sched + kHdrCtr + q2, 1);
    }
  };
  auto fetch = [&]() {   // thread 0: the next local index of the current queue
    const int q = (own + s_q) & (kXcds - 1);
    return s_q < kXcds ? tail_wgs(q) + atomicAdd(sched + kHdrCtr + q, 1) : 0;
  };
  if (threadIdx.x == 0) {
    const int b = (int)blockIdx.x;
    s_unit = resolve((b - (s_hw + (((own - s_hw) % kXcds) + kXcds) % kXcds)) / kXcds);
  }
  __syncthreads();
  auto compacts = [&](const Unit& t) {   // its product lists finite rows / columns and prep flagged it
    const I8Epi e = epi_of(epis, t.pi);
    return e.yd != nullptr && *(const __attribute__((address_space(4))) int*)e.nf != 0;
  };
  // every tail unit is a 256 x 256 tile on packed residues.  A unit of a flagged product runs as
  // compacted_tile; the others as tiles whose next unit's stages go out before the epilogue when
  // that unit does not compact (run_tile's handoff), so that the epilogue's stores drain under them.
  int u = __builtin_amdgcn_readfirstlane(s_unit);
  bool pre = false;   // u's stages are in flight
  int pend = 0;       // thread 0: the local index fetched for the next unit
  while (u >= 0) {
    const Unit t = decode_unit<kGroupML, true>(sched, probs, u);
    if (!pre && compacts(t)) {
      compacted_tile<CfgL, true>(lds, probs, epis, t, epi_of(epis, t.pi).yd);
      if (threadIdx.x == 0) s_unit = s_q < kXcds ? resolve(fetch()) : -1;
      __syncthreads();
      u = __builtin_amdgcn_readfirstlane(s_unit);
      continue;
    }
    if (!pre) TileSrc<CfgL, true>(probs[t.pi], t.tm, t.tn).prologue(lds);
    int nu = -1;
    pre = run_tile<CfgL, true, false>(
        lds, probs, epis, t.pi, t.tm, t.tn,
        [&]() {
          if (threadIdx.x == 0) pend = fetch();
        },
        [&]() -> Unit {
          if (threadIdx.x == 0) s_unit = s_q < kXcds ? resolve(pend) : -1;
          asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
          nu = __builtin_amdgcn_readfirstlane(s_unit);
          if (nu < 0) return Unit{-1, 0, 0, 0};
          Unit nx = decode_unit<kGroupML, true>(sched, probs, nu);
          if (compacts(nx)) nx.cfg = -1;   // no stages: it runs as a compacted tile
          return nx;
        });
    u = nu;
  }
  if (threadIdx.x == 0) {   // every fetch of this workgroup has returned
    __threadfence();
    if (atomicAdd(sched + kHdrDone, 1) == (int)gridDim.x - hw0 - 1) {
      for (int x = 0; x < kXcds; ++x) atomicExch(sched + kHdrCtr + x, 0);
      atomicExch(sched + kHdrDone, 0);
    }
  }
}

// ---------------------------------------------------------------- persistent kernels
__global__ void __launch_bounds__(kThreads, 2) i8_grouped_persistent_kernel(const i8_problem* __restrict__ probs,
                                                                            const I8Epi* __restrict__ epis,
                                                                            int* __restrict__ sched) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  auto pro = [&](const Unit& t) {
    const bool pk = (epi_of(epis, t.pi).mode & kEpiPacked) != 0;
    switch (t.cfg) {
      case 0: pk ? TileSrc<Cfg0, true>(probs[t.pi], t.tm, t.tn).prologue(lds)
                 : TileSrc<Cfg0, false>(probs[t.pi], t.tm, t.tn).prologue(lds); break;
      case 1: pk ? TileSrc<Cfg1, true>(probs[t.pi], t.tm, t.tn).prologue(lds)
                 : TileSrc<Cfg1, false>(probs[t.pi], t.tm, t.tn).prologue(lds); break;
      default: pk ? TileSrc<Cfg2, true>(probs[t.pi], t.tm, t.tn).prologue(lds)
                  : TileSrc<Cfg2, false>(probs[t.pi], t.tm, t.tn).prologue(lds); break;
    }
  };
  persistent<kGroupM, false>(sched, probs, pro, [&](const Unit& t, auto& claim, auto& next) -> bool {
    const bool pk = (epi_of(epis, t.pi).mode & kEpiPacked) != 0;
    switch (t.cfg) {
      case 0: return pk ? run_tile<Cfg0, true, false>(lds, probs, epis, t.pi, t.tm, t.tn, claim, next)
                        : run_tile<Cfg0, false, false>(lds, probs, epis, t.pi, t.tm, t.tn, claim, next);
      case 1: return pk ? run_tile<Cfg1, true, false>(lds, probs, epis, t.pi, t.tm, t.tn, claim, next)
                        : run_tile<Cfg1, false, false>(lds, probs, epis, t.pi, t.tm, t.tn, claim, next);
      default: return pk ? run_tile<Cfg2, true, false>(lds, probs, epis, t.pi, t.tm, t.tn, claim, next)
                         : run_tile<Cfg2, false, false>(lds, probs, epis, t.pi, t.tm, t.tn, claim, next);
    }
  });
}

__global__ void __launch_bounds__(kThreadsL, 1) i8_large_persistent_kernel(const i8_problem* __restrict__ probs,
                                                                           const I8Epi* __restrict__ epis,
                                                                           int* __restrict__ sched) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  auto pro = [&](const Unit& t) {
    if (epi_of(epis, t.pi).mode & kEpiPacked) TileSrc<CfgL, true>(probs[t.pi], t.tm, t.tn).prologue(lds);
    else TileSrc<CfgL, false>(probs[t.pi], t.tm, t.tn).prologue(lds);
  };
  persistent<kGroupML, true>(sched, probs, pro, [&](const Unit& t, auto& claim, auto& next) -> bool {
    return (epi_of(epis, t.pi).mode & kEpiPacked)
               ? run_tile<CfgL, true, false>(lds, probs, epis, t.pi, t.tm, t.tn, claim, next)
               : run_tile<CfgL, false, false>(lds, probs, epis, t.pi, t.tm, t.tn, claim, next);
  });
}

// ----------------------------------------------------------------------------- host side
struct Ent {
  double cost;
  int tiles, prob, cfg;
};
// Host scratch of the schedule builder (entries, their order, the XCD queue of each entry), sized
// by i8_grouped_gemm_reserve at handle / plan creation so that building a schedule allocates
// nothing; a larger call still works and grows it, which i8_grouped_gemm_host_allocs counts
// (src/int8_grouped_gemm.cu:541-589).  The kernel-level i8_grouped_gemm_ex keeps its schedule
// image in a buffer of its own, reserved and counted the same way.
std::mutex g_mu;
Ent* g_ents = nullptr;
int* g_order = nullptr;
int* g_xq = nullptr;
size_t g_cap = 0;
std::mutex g_img_mu;
int* g_img = nullptr;
size_t g_img_cap = 0;
std::atomic<long long> g_host_allocs{0};

// capacity for n schedule images (g_img_mu held)
bool ensure_img_capacity(size_t n) {
  const size_t img = sched_bytes((int)std::min<size_t>(std::max<size_t>(n, 1), 0x3fffffff)) / sizeof(int) + 1;
  if (img > g_img_cap) {
    int* q = new (std::nothrow) int[img];
    if (!q) return false;
    delete[] g_img;
    g_img = q;
    g_img_cap = img;
    ++g_host_allocs;
  }
  return true;
}

// capacity for n schedule entries (g_mu held); false when the host is out of memory
bool ensure_capacity(size_t n) {
  n = std::max<size_t>(n, 1);
  if (n > g_cap) {
    Ent* e = new (std::nothrow) Ent[n];
    int* o = new (std::nothrow) int[n];
    int* x = new (std::nothrow) int[n];
    if (!e || !o || !x) {
      delete[] e;
      delete[] o;
      delete[] x;
      return false;
    }
    delete[] g_ents;
    delete[] g_order;
    delete[] g_xq;
    g_ents = e;
    g_order = o;
    g_xq = x;
    g_cap = n;
    ++g_host_allocs;
  }
  return true;
}

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

int i8_auto_tile_cfg(int m, int n) { return auto_cfg(m, n); }

bool i8_env_persistent() {
  const char* e = std::getenv("GGEMM_I8_SCHED");
  return e && !std::strcmp(e, "persistent");
}

int i8_build_schedule(const i8_problem* h, int num, void* h_ws, size_t ws_bytes, i8_sched_info* info, int num_cus,
                      int large, int* kernel, bool persistent, const I8Epi* epis, int* hw_units) {
  if (num < 0 || (num > 0 && !h) || !h_ws || !info) return 1;
  if (ws_bytes < sched_bytes(num)) return 2;
  if (kernel) *kernel = kI8General;
  if (hw_units) *hw_units = -1;
  std::lock_guard<std::mutex> lk(g_mu);
  if (!ensure_capacity((size_t)num)) return 6;
  Ent* const ents = g_ents;
  size_t ne = 0;
  for (int i = 0; i < num; ++i) {
    if (!valid_problem(h[i])) return 3;
    if (h[i].m == 0 || h[i].n == 0 || h[i].kp == 0) continue;
    int c = h[i].tile_cfg;
    if (c < 0) c = auto_cfg(h[i].m, h[i].n);
    if (c >= kI8NumCfg) c = kI8NumCfg - 1;
    ents[ne++] = {(double)i8_tile_m(c) * i8_tile_n(c) * (double)(h[i].kp + 128), tiles_of(c, h[i].m, h[i].n), i, c};
  }
  Ent* const ents_end = ents + ne;
  bool all_auto = ne > 0;
  for (const Ent* e = ents; e != ents_end; ++e) all_auto = all_auto && h[e->prob].tile_cfg < 0;
  const bool force_large = large == kLargeForce && all_auto;
  // group-level fill: fewer tiles than workgroup slots (2 per compute unit) -> shrink automatic
  // tiles one step
  for (int pass = 0; pass < 2 && !force_large; ++pass) {
    long long t = 0;
    for (const Ent* e = ents; e != ents_end; ++e) t += e->tiles;
    if (t >= 2LL * num_cus) break;
    for (Ent* e = ents; e != ents_end; ++e)
      if (e->cfg < kI8NumCfg - 1 && h[e->prob].tile_cfg < 0) {
        ++e->cfg;
        e->tiles = tiles_of(e->cfg, h[e->prob].m, h[e->prob].n);
        e->cost = (double)i8_tile_m(e->cfg) * i8_tile_n(e->cfg) * (double)(h[e->prob].kp + 128);
      }
  }
  // large-tile kernel: every product on automatic large tiles, and enough 256 x 256 tiles to give
  // every compute unit one
  bool large_chosen = false;
  if (large != kLargeNever && ne > 0) {
    bool all = true;
    long long t = 0;
    for (const Ent* e = ents; e != ents_end; ++e) {
      all = all && e->cfg == 0 && h[e->prob].tile_cfg < 0;
      t += (long long)((h[e->prob].m + 255) / 256) * ((h[e->prob].n + 255) / 256);
    }
    if (force_large || (all && t >= num_cus)) {
      for (Ent* e = ents; e != ents_end; ++e) {
        e->cfg = 0;
        e->tiles = ((h[e->prob].m + 255) / 256) * ((h[e->prob].n + 255) / 256);
        e->cost = 256.0 * 256.0 * (double)(h[e->prob].kp + 128);
      }
      large_chosen = true;
      if (kernel) *kernel = kI8Large;
    }
  }
  if (kernel && persistent) *kernel |= kI8Persistent;
  // longest-processing-time order (heaviest tiles first; ties by problem index, i.e. the order a
  // stable sort keeps -- std::sort takes no temporary buffer)
  std::sort(ents, ents_end, [](const Ent& a, const Ent& b) {
    if (a.cost != b.cost) return a.cost > b.cost;
    if (a.tiles != b.tiles) return a.tiles > b.tiles;
    return a.prob < b.prob;
  });
  // Queues of the persistent kernels: chunks of c consecutive tiles of the LPT table dealt
  // round-robin to the XCDs (c = 32, GGEMM_I8_CHUNK=c overrides; same-box GEMM times at c = 32 vs
  // whole products per XCD: 121.5 vs 129.2 ms on 8 x 8192^2 x 16384, equal on 1024^3 products), or
  // with c = 0 whole entries, each in turn onto the least loaded queue (ties: lowest index), every
  // queue in LPT order.  The hardware-dispatched kernels map workgroups to tiles themselves and
  // take the table in LPT order.
  static const int env_chunk = [] {
    const char* e = std::getenv("GGEMM_I8_CHUNK");
    return e ? std::max(0, std::atoi(e)) : kChunk;
  }();
  const int chunk = persistent ? env_chunk : 1;
  int* const order = g_order;
  int* const xq = g_xq;
  double load[kXcds] = {};
  int count[kXcds] = {};
  for (size_t j = 0; j < ne; ++j) {
    int best = 0;
    for (int x = 1; x < kXcds && chunk == 0; ++x)
      if (load[x] < load[best]) best = x;
    xq[j] = best;
    load[best] += ents[j].cost * ents[j].tiles;
    ++count[best];
  }
  int first[kXcds + 1] = {};
  for (int x = 0; x < kXcds; ++x) first[x + 1] = first[x] + count[x];
  {
    int pos[kXcds];
    for (int x = 0; x < kXcds; ++x) pos[x] = first[x];
    for (size_t j = 0; j < ne; ++j) order[pos[xq[j]]++] = (int)j;
  }
  // large-tile kernel, one workgroup per tile: the products that may compact (packed residues and
  // a reconstruct descriptor) after the others, each part in LPT order
  auto compacts = [&](const Ent& e) {
    return epis && (epis[e.prob].mode & kEpiPacked) != 0 && epis[e.prob].yd != nullptr;
  };
  long long hw = -1;
  if (large_chosen && !persistent && epis) {
    size_t k = 0;
    hw = 0;
    for (size_t j = 0; j < ne; ++j)
      if (!compacts(ents[j])) {
        order[k++] = (int)j;
        hw += ents[j].tiles;
      }
    if (k == ne) {
      hw = -1;   // nothing compacts: every unit dispatched
    } else {
      for (size_t j = 0; j < ne; ++j)
        if (compacts(ents[j])) order[k++] = (int)j;
    }
  }
  int* img = static_cast<int*>(h_ws);
  int* prefix = img + kSchedHdr;
  int* entry = prefix + ne + 1;
  std::memset(img, 0, sizeof(int) * kSchedHdr);
  long long tot = 0;
  for (size_t j = 0, x = 0; j < ne; ++j) {
    while ((int)x < kXcds && first[x] == (int)j) img[kHdrXcd + x++] = (int)tot;
    const Ent& e = ents[order[j]];
    prefix[j] = (int)tot;
    tot += e.tiles;
    entry[j] = (e.prob << 2) | e.cfg;
  }
  if (tot > 0x7fffffffLL - 1000000) return 5;
  for (int x = 0; x <= kXcds; ++x)
    if (first[x] == (int)ne) img[kHdrXcd + x] = (int)tot;
  prefix[ne] = (int)tot;
  img[0] = (int)tot;
  img[1] = (int)ne;
  img[kHdrHw] = hw >= 0 ? (int)hw : (int)tot;
  if (hw_units) *hw_units = hw >= 0 ? (int)hw : -1;
  img[3] = persistent ? chunk : 0;
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
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static bool done[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  std::lock_guard<std::mutex> lk(mu);
  if (!done[dev]) {
    if (hipFuncSetAttribute((const void*)i8_grouped_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kSmem) !=
            hipSuccess ||
        hipFuncSetAttribute((const void*)i8_large_kernel<false>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            kSmemL) != hipSuccess ||
        hipFuncSetAttribute((const void*)i8_large_kernel<true>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            kSmemL) != hipSuccess ||
        hipFuncSetAttribute((const void*)i8_grouped_persistent_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                            kSmem) != hipSuccess ||
        hipFuncSetAttribute((const void*)i8_large_persistent_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                            kSmemL) != hipSuccess)
      return false;
    done[dev] = true;
  }
  return true;
}
}  // namespace

void i8_reserve_host(size_t entries) {
  {
    std::lock_guard<std::mutex> lk(g_mu);
    ensure_capacity(entries);
  }
  std::lock_guard<std::mutex> lk(g_img_mu);
  ensure_img_capacity(entries);
}

int i8_launch(const i8_problem* d_probs, const I8Epi* d_epi, const void* d_sched, const i8_sched_info* info,
              hipStream_t s, int kernel, int hw_units) {
  if (!info) return 1;
  if (info->num_launches == 0 || info->tiles_main == 0) return 0;
  if (!d_probs || !d_sched) return 1;
  if (!lds_attrs_set()) return 6;
  int* sched = static_cast<int*>(const_cast<void*>(d_sched));
  const bool large = (kernel & kI8Large) != 0;
  if (kernel & kI8Persistent) {
    // persistent workgroups: as many as the compute units hold at once (one 16-wave workgroup or two
    // 8-wave workgroups per unit), at most one per tile; the schedule image carries the queue
    // counters the kernel updates.  Same-box GEMM times against one workgroup per tile (the
    // default): 1.31 vs 1.25 ms on 64 x 1024^3 (16 planes), 2.81 vs 2.53 ms on the ragged group,
    // 121.5 vs 120.0 ms on 8 x 8192^2 x 16384 -- the dispatcher starts a new workgroup on a freed
    // slot while the unit's other workgroup computes, which the persistent loop's per-tile handoff
    // (a workgroup barrier, the counter fetch and the next tile's lookup) does not beat.
    const DevCtx* c = dev_ctx();
    if (!c) return 6;
    const int slots = (large ? 1 : 2) * c->num_cus;
    const unsigned grid = (unsigned)std::min(info->tiles_main, slots);
    if (large)
      hipLaunchKernelGGL(i8_large_persistent_kernel, dim3(grid), dim3(kThreadsL), kSmemL, s, d_probs, d_epi, sched);
    else
      hipLaunchKernelGGL(i8_grouped_persistent_kernel, dim3(grid), dim3(kThreads), kSmem, s, d_probs, d_epi, sched);
  } else if (large) {
    // units [0, hw_units) one workgroup each, then the tail: a workgroup per compute unit over the
    // rest (when there are fewer of them, one workgroup per unit throughout)
    unsigned grid = (unsigned)info->tiles_main;
    bool tail = false;
    if (hw_units >= 0 && hw_units < info->tiles_main) {
      const DevCtx* c = dev_ctx();
      if (!c) return 6;
      tail = info->tiles_main - hw_units > c->num_cus;
      if (tail) grid = (unsigned)(hw_units + c->num_cus);
    }
    if (tail)
      hipLaunchKernelGGL(i8_large_kernel<true>, dim3(grid), dim3(kThreadsL), kSmemL, s, d_probs, d_epi, sched);
    else
      hipLaunchKernelGGL(i8_large_kernel<false>, dim3(grid), dim3(kThreadsL), kSmemL, s, d_probs, d_epi, sched);
  } else {
    hipLaunchKernelGGL(i8_grouped_kernel, dim3((unsigned)info->tiles_main), dim3(kThreads), kSmem, s, d_probs, d_epi,
                       sched);
  }
  return hipGetLastError() == hipSuccess ? 0 : 6;
}

}  // namespace ggemm

using namespace ggemm;

extern "C" size_t i8_grouped_gemm_sched_ws_bytes(int max_problems, size_t) {
  return sched_bytes(max_problems < 0 ? 0 : max_problems);
}

extern "C" void i8_grouped_gemm_reserve(int max_problems, size_t) {
  i8_reserve_host(max_problems > 0 ? (size_t)max_problems : 1);
}

extern "C" long long i8_grouped_gemm_host_allocs() { return g_host_allocs.load(); }

extern "C" int i8_grouped_gemm_build_schedule(const i8_problem* h_probs, int num, void* h_ws, size_t ws_bytes,
                                              i8_sched_info* info) {
  DevCtx* c = dev_ctx();
  return i8_build_schedule(h_probs, num, h_ws, ws_bytes, info, c ? c->num_cus : 256, kLargeNever, nullptr,
                           i8_env_persistent());
}

extern "C" int i8_grouped_gemm_launch(const i8_problem* d_probs, int, const void* d_sched_ws,
                                      const i8_sched_info* info, hipStream_t s) {
  return i8_launch(d_probs, nullptr, d_sched_ws, info, s, i8_env_persistent() ? kI8Persistent : kI8General);
}

extern "C" int i8_grouped_gemm_ex(const i8_problem* d_probs, int num, const i8_problem* h_probs, void* d_sched_ws,
                                  size_t sched_ws_bytes, hipStream_t s, int* num_launches) {
  if (num_launches) *num_launches = 0;
  if (num == 0) return 0;
  if (!d_sched_ws) return 1;
  const size_t need = sched_bytes(num);
  if (need > sched_ws_bytes) return 2;
  // the image goes through the reserved host buffer (one call at a time: the copy below is waited
  // for before the buffer is released)
  std::lock_guard<std::mutex> lk(g_img_mu);
  if (!ensure_img_capacity((size_t)num)) return 6;
  int* const img = g_img;
  i8_sched_info info;
  int rc = i8_grouped_gemm_build_schedule(h_probs, num, img, need, &info);
  if (rc) return rc;
  if (info.num_launches == 0) return 0;
  if (hipMemcpyAsync(d_sched_ws, img, info.bytes_used, hipMemcpyHostToDevice, s) != hipSuccess) return 7;
  // the pageable source must stay valid until the copy has consumed it
  if (hipStreamSynchronize(s) != hipSuccess) return 7;
  rc = i8_launch(d_probs, nullptr, d_sched_ws, &info, s, i8_env_persistent() ? kI8Persistent : kI8General);
  if (!rc && num_launches) *num_launches = info.num_launches;
  return rc;
}
