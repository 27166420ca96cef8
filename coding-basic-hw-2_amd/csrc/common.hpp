// common.hpp -- internal contract of the MI355X grouped Ozaki-II DGEMM library.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "ggemm.h"
#include "ggemm_graph.h"
#include "ggemm_oz2.h"

namespace ggemm {

constexpr int kMaxModuli = GGEMM_MAX_MODULI;
constexpr int kMaxPlanes = kMaxModuli + OZ2_EXTRA_PLANES;   // residues + abs plane
constexpr int kS2Bits = 18;                                 // fractional bits of s2
constexpr int kKpAlign = 32;                                // Kp = round_up(k, 32)
constexpr size_t kBufAlign = 256;                           // byte alignment of every block

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }
inline int kp_of(int k) { return (int)align_up((size_t)k, kKpAlign); }

// CRT constants for N = 1..20 moduli (the quantities of src/moduli.h:43-58), built on the host
// with exact big-integer arithmetic and copied once per device into global memory.
struct CrtTables {
  int32_t p[kMaxModuli];
  uint32_t magic[kMaxModuli];                  // floor(2^32 / p)
  float ipf[kMaxModuli];                       // 1 / p, nearest float
  float cf[kMaxModuli];                        // (floor(p / 2) + 1/2) / p + 2048, nearest float
  // byte weights of the digit words, four per word, for word kind k:
  //   k = 0: unsigned bytes 2^(8 i) mod p, i = 0..3        (low word, unsigned digits)
  //   k = 1: unsigned bytes 2^(8 i) mod p, i = 4..7        (wide middle word, unsigned digits)
  //   k = 2: signed bytes sym(2^(8 i) mod p), i = 4..7     (narrow top word, signed digits)
  //   k = 3: signed bytes sym(2^(8 i) mod p), i = 8..11    (wide top word, signed digits)
  // [0][l][k] plain, [N][l][k] with the CRT inverse q_(N,l) folded in (q 2^(8 i) mod p);
  // sym(r) in [-floor(p/2), p - 1 - floor(p/2)]
  uint32_t wb[kMaxModuli + 1][kMaxModuli][4];
  uint64_t s1[kMaxModuli + 1][kMaxModuli];     // floor(M_l / u1)
  uint32_t s2[kMaxModuli + 1][kMaxModuli];     // round(frac(M_l / u1) 2^18)
  int32_t qinv[kMaxModuli + 1][kMaxModuli];    // M_l^-1 mod p_l
  int64_t P1[kMaxModuli + 1];                  // floor(P / u1)
  double P2[kMaxModuli + 1];                   // frac(P / u1)
  double inv_Pu[kMaxModuli + 1];               // u1 / P
  int32_t log2_u1[kMaxModuli + 1];
  double T[kMaxModuli + 1];                    // per-row / per-column 2-norm budget
  double log2P[kMaxModuli + 1];
};

// Host tables (built once per process); returns nullptr if the moduli are inconsistent.
const CrtTables* host_tables();

// Process-wide per-device state: the tables and the four sticky counters
// {nonfinite vectors, uncertified, repaired, safety fallback}.  Created on first use on the
// current device and kept until the process ends.  Each counter is kept in kCounterSlots copies,
// one 128-byte line per slot (counter q of slot s at s kCounterStride + q): a workgroup adds to the
// slot of its index, so the one atomic per workgroup and counter does not queue on one address when
// a call has a hundred thousand workgroups that count; readers sum the slots.
constexpr int kCounterSlots = 64, kCounterStride = 16;
__device__ inline unsigned long long* counter_slot(unsigned long long* cnt) {
  return cnt + ((blockIdx.x + blockIdx.y) % kCounterSlots) * kCounterStride;
}
struct DevCtx {
  int device;
  int num_cus;
  const CrtTables* tab;             // device copy
  unsigned long long* counters;     // device, 4 entries
};
DevCtx* dev_ctx();                  // current device; nullptr on failure
// Device addresses of the resident tables and counters on the current device (0 on success).
int device_state(void** tables, void** counters);

// Native FP64 problem descriptor (device-resident so a captured graph can be re-pointed).
struct F64Problem {
  int m, n, k, lda, ldb, ldc;
  const double* A;
  const double* B;
  double* C;
  double alpha, beta;
};

// Schedule image shared by the tile-based kernels (INT8 GEMM, FP64 GEMM):
//   int[0] total tiles, int[1] entries, int[2] tiles per entry when all entries have the same
//   count (INT8 GEMM; 0 otherwise), int[3] the persistent queues' chunk, int[kHdrHw] the units the
//   256 x 256 kernel dispatches one workgroup each (the rest go to its tail workgroups), int[5..7]
//   reserved, INT8 GEMM only: int[kHdrXcd + x], x = 0..8, first tile of XCD x's queue (x = 8: the
//   total); int[kHdrCtr + x], x < 8, the queue counters and int[kHdrDone] the finished-workgroup
//   count of the persistent kernel and of the tail (zero when uploaded, reset by the kernel itself),
//   prefix[entries + 1] at kSchedHdr (first tile of each entry), entry[entries] = (problem << 2) | cfg.
constexpr int kXcds = 8;   // MI355X: accelerator complex dies, each with its own L2
constexpr int kHdrHw = 4, kHdrXcd = 8, kHdrCtr = 32, kHdrDone = 40;
constexpr int kSchedHdr = 64;
inline size_t sched_bytes(int entries) {
  return sizeof(int) * (size_t)(kSchedHdr + 2 * (size_t)entries + 1 + 8);
}

// INT8 GEMM tile configurations (output tile rows x columns).
constexpr int kI8NumCfg = 3;
__host__ __device__ inline int i8_tile_m(int cfg) { return cfg == 0 ? 256 : (cfg == 1 ? 128 : 64); }
__host__ __device__ inline int i8_tile_n(int cfg) { return cfg == 0 ? 128 : (cfg == 1 ? 128 : 64); }
// Per-product epilogue of the INT8 GEMM, mode bits:
//   kEpiResidue  one byte per entry, the residue C mod p in [0, p), from u = C + bias >= 0
//                by a Barrett step q = umulhi(u, mc), mc = ceil(2^32 / p) (q = floor(u / p) or one
//                more), r = u - q p in [-p, p) and one correction; without it the int32 product.
//                In the production pipeline the A residues of plane l carry the CRT inverse q_l
//                (prep with fold_q), so this byte is the CRT digit y_l = (C_l q_l) mod p_l.
//   kEpiAccBias  (with kEpiResidue, kp <= 32768) bias = p ceil(2^29 / p) >= |C| is the MFMA
//                accumulators' initial value, so u is the accumulator itself, u < 2^30 + p,
//                q < 2^23 and r = u - q p is one 24-bit multiply-add; otherwise (long k)
//                bias = p ceil(2^31 / p), u = C + bias < 2^32 and r takes a 32-bit multiply.
//   kEpiBlocked  16 x 16 blocked output (below) instead of column-major with ld m.
// Blocked layout of an m x n plane: blocks (bi, bj) of 16 x 16 entries in column-major block
// order (MB = ceil(m / 16) block rows), each block stored as one MFMA result block: lane
// l = 16 q + c holds rows 4 q .. 4 q + 3 of column c, i.e. 4 consecutive bytes (digits) or 16
// bytes (int32) per lane, 256 / 1024 contiguous bytes per block.  Entries beyond m x n inside a
// block are padding.
//   kEpiPacked   the residue operands are in the packed layout (below) instead of row-major.
// Packed layout of a rows x Kp residue plane (production pipeline, same size as row-major): k-blocks
// of 64 bytes, block b holding the bytes k in [64 b, 64 b + 64) of every row contiguously
// ([b][row][64]); with Kp % 64 == 32 the last block holds 32 bytes per row.  A 64-byte k-stage of
// consecutive rows is then one contiguous span.
enum : uint32_t { kEpiResidue = 1u, kEpiBlocked = 2u, kEpiPacked = 4u, kEpiAccBias = 8u };
constexpr int kAccBiasMaxKp = 32768;   // |C| <= 128^2 kp <= 2^29
constexpr int kPackedMaxKp = 4096;   // production problems whose Kp is at most this use packing
constexpr int kKpMaxPacked = 1 << 30;   // packed_kp of a call that packs every problem
__host__ __device__ inline size_t packed_offset(int row, int k, int rows, int kp) {
  const int b = k >> 6;
  const int rb = b == (kp >> 6) ? 32 : 64;
  return (size_t)b * (size_t)rows * 64 + (size_t)row * rb + (size_t)(k & 63);
}
// rs, cs, nf (or all nullptr): the product's row / column shifts (the first m / n int32 of prep's
// row_shift, col_shift) and its non-finite flag (YDesc::nff).  When prep has set the flag, a tile
// whose rows, or whose columns, all carry OZ2_SHIFT_NONFINITE is not computed: each of its entries
// takes the safety fallback, which uses none of the tile's outputs.
struct YDesc;
struct I8Epi {
  uint32_t mode, p, mc, bias;
  const int32_t* rs;
  const int32_t* cs;
  const int* nf;
  // the product's reconstruct descriptor (blocked grouped calls, nullptr otherwise): with its
  // non-finite flag set, the 256 x 256 kernel on packed residues computes only the finite rows x
  // finite columns (the descriptor's finite-row / finite-column lists), each tile over consecutive
  // entries of the lists
  const YDesc* yd;
};
I8Epi i8_epi_residue(uint32_t p, int kp);
__host__ __device__ inline size_t blocked_plane_entries(int m, int n) {
  return (size_t)((m + 15) / 16) * (size_t)((n + 15) / 16) * 256;
}
// offset in entries of the word holding rows r4 .. r4 + 3 (r4 % 4 == 0) of column c
__host__ __device__ inline size_t blocked_word(int r4, int c, int mb) {
  return ((size_t)(c >> 4) * (size_t)mb + (size_t)(r4 >> 4)) * 256 + (size_t)(16 * ((r4 & 15) >> 2) + (c & 15)) * 4;
}
// INT8 GEMM kernels: the general one (tile configs 0..2, two workgroups per compute unit) and the
// large-tile one (every tile 256 x 256, one 16-wave workgroup per compute unit); kI8Persistent
// added: their persistent work-stealing form instead of one workgroup per tile.
enum { kI8General = 0, kI8Large = 1, kI8Persistent = 2 };
// Builds the INT8 schedule (LPT order); cfg < 0 in a problem selects automatically.
// large: kLargeNever, kLargeAuto (the large-tile kernel when every product is on automatic large
// tiles and they fill the GPU) or kLargeForce (whenever every product's tile is automatic);
// persistent: schedule for the persistent kernels (queues per XCD);
// *kernel receives the choice, which i8_launch must be given.  epis (host copies, or nullptr):
// with the large-tile kernel dispatched one workgroup per tile, the products that may compact
// (packed residues and a reconstruct descriptor) go last in the table, and *hw_units receives the
// units before them, which i8_launch must be given: those run one workgroup each, the rest are
// taken in chunks by as many workgroups as there are compute units (-1: every unit dispatched).
enum { kLargeNever = 0, kLargeAuto = 1, kLargeForce = 2 };
int i8_build_schedule(const i8_problem* h, int num, void* h_ws, size_t ws_bytes, i8_sched_info* info,
                      int num_cus, int large = kLargeNever, int* kernel = nullptr, bool persistent = false,
                      const I8Epi* epis = nullptr, int* hw_units = nullptr);
// The tile configuration i8_build_schedule gives an m x n product with tile_cfg < 0 (before the
// group-level shrink).
int i8_auto_tile_cfg(int m, int n);
// Sizes the schedule builder's host scratch for `entries` (problem, plane) products, so that
// i8_build_schedule allocates nothing for calls of at most that many (handle / plan creation).
void i8_reserve_host(size_t entries);
// GGEMM_I8_SCHED=persistent in the environment (read at each call): the kernel-level INT8 API
// (i8_grouped_gemm_*) builds for and runs the persistent kernels
bool i8_env_persistent();
// d_epi: per-problem epilogues in device memory, or nullptr for int32 products everywhere.
int i8_launch(const i8_problem* d_probs, const I8Epi* d_epi, const void* d_sched, const i8_sched_info* info,
              hipStream_t s, int kernel = kI8General, int hw_units = -1);

// Where the reconstruct reads a problem's plane products in the production pipeline: CRT digits
// y_l (one byte per entry, plane l at Y + l * y_stride) and the abs-plane product L (int32), both
// column-major with ld m, or both blocked (layout above) when the call's descriptors say so.
// F (blocked layout only): per 16 x 16 block (blocked order) four 64-bit words, bit l of word e set
// when entry e of MFMA lane l of the block takes an FP64 dot product; written by the reconstruct for
// every block of the problem, read by the dot-product pass.
// t0 / d0: the problem's first tile in the grouped call's compact reconstruct / dot-product grid (the
// tiles of all problems back to back, so no workgroup of the grid lies outside its problem).
// nf (blocked layout, or nullptr): kNfWords words per row of A (row i at nf + kNfWords i) and per
// column of B (column j at nf + kNfWords (m + j)), written by prep for the rows / columns that hold a
// NaN or an Inf (the others are never written nor read):
//   word 0: bit 0 a NaN, bit 1 more than kNfCap infinities, bits 8.. the infinities listed (<= kNfCap)
//   word 1: ilogb of the largest finite nonzero magnitude, kNfNoFinite if there is none
//   words 2 ..: the infinities' positions k, bit 31 set for -Inf (any order)
// The dot-product pass evaluates the safety-fallback entries of such rows / columns from them.
constexpr int kNfWords = 16, kNfCap = kNfWords - 2, kNfNoFinite = -2000;
// nff: zero in every call's descriptors; prep sets it when a row or column of the problem is
// non-finite (NaN / Inf), and the reconstruct then reads the shifts before the digits, skipping the
// digits of lanes whose every entry takes the safety fallback.
// fla: zero in every call's descriptors; the reconstruct sets it when it flags an entry of the
// problem, and the dot-product pass returns at once for problems without (a replayed graph may
// find it set from an earlier run: the pass then reads the flags, as always).
struct YDesc {
  const uint8_t* Y;
  size_t y_stride;
  const int32_t* L;
  uint64_t* F;
  int32_t* nf;
  // crossings sets of the dot pass (blocked layout): ceil(m / 64) row words, ceil(n / 64) column
  // words and one word of counts, behind the flags; AT: row-major copies of the crossings rows in
  // the residue workspace (free once the INT8 GEMM is done), nullptr: the dot pass defers nothing
  uint64_t* X;
  double* AT;
  // finite rows of A / columns of B (blocked layout): fr[i], fc[j] 1 for a finite row / column, 0
  // else, written by prep every call; each list starts 4-byte aligned (fc at fr + m rounded up to 4)
  uint8_t* fr;
  uint8_t* fc;
  int t0, d0, b0, x0;   // the problem's first workgroup in the reconstruct, dot-pass, row-band and
                        // crossings grids
  int xn;               // the problem's crossings workgroups
  int nff, fla;
};
// Compact grids of a grouped call (ne problems): tiles in all and, when every problem has the same
// count, that count (else 0) -- for the reconstruct, the dot-product pass, the row bands of its
// crossings pass and the crossings pass's workgroups.
struct ReconGrid {
  int ne, tiles, per, dtiles, dper, bands, bper, xwgs, xper;
};
// Reconstruct tile shapes (rows x columns per workgroup): blocked digits / column-major, and the
// dot-product pass's tile
constexpr int kReconTileMB = 64, kReconTileNB = 16, kReconTileMC = 128, kReconTileNC = 8, kDotTile = 64;
// Bytes of a problem's flags plus its crossings sets and finite-row / finite-column bytes (blocked
// layout)
inline size_t flag_bytes(int m, int n, size_t plane_entries) {
  return plane_entries / 8 + sizeof(uint64_t) * (size_t)((m + 63) / 64 + (n + 63) / 64 + 1) +
         (((size_t)m + 3) & ~(size_t)3) + (((size_t)n + 3) & ~(size_t)3);
}
// Prep workgroup shapes: rows of A per A-row block, columns of B per B-column block
constexpr int kPrepRows = 32, kPrepCols = 8;

// FP64 MFMA grouped GEMM (native routes).  h_ws receives the schedule image; *launch receives the
// launch word for f64_launch: the tile count in bits 0-29, kF64Tile128 set for 128 x 128 tiles (0:
// nothing to launch).  tile_mode 0 chooses the tile edge from the group's shapes, 64 or 128 forces it.
constexpr int kF64Tile128 = 1 << 30;
int f64_build_schedule(const F64Problem* h, int num, void* h_ws, size_t ws_bytes, int* launch, size_t* bytes_used,
                       int tile_mode = 0);
int f64_launch(const F64Problem* d_probs, const void* d_sched, int launch, hipStream_t s);

// Launchers used by the orchestration (return 0 on success).
// fold_q != 0 (production): the residues of A plane l are (q_l r) mod p_l (symmetric) instead of r,
// with q_l the CRT inverse of modulus l for the problem's N (the abs plane and B are unchanged), and
// the planes of non-finite rows / columns are left unwritten; fold_q = 0: plain residues, zeros for
// non-finite rows / columns.
// packed_kp: the residue planes of problems with Kp <= packed_kp are in the packed layout, the others row-major (0: every problem row-major)
// max_moduli: the largest num_moduli among the num problems (selects the digit width)
// yd (or nullptr): descriptors parallel to d whose nf summaries prep writes
// order (or nullptr: 0 .. num - 1): the problems in the order their workgroups are dispatched
// pofs (with order, or nullptr): a compact grid of total_blocks workgroups, problem order[i] owning
// blocks pofs[i] .. pofs[i + 1] - 1 (ceil(m / 32) A-row blocks, then ceil(n / 8) B-column blocks;
// none for problems prep skips)
int prep_launch(const oz2_problem* d, int num, int max_m, int max_n, hipStream_t s, int fold_q, int packed_kp,
                int max_moduli, const YDesc* yd = nullptr, const int* order = nullptr, const int* pofs = nullptr,
                long long total_blocks = 0);
// yd == nullptr: read the int32 planes of oz2_problem::C32 (kernel-level API); else the digits.
// blocked: the digits and L of every problem are in the blocked layout (production, yd != nullptr);
// the reconstruct then flags the entries that take FP64 dot products and a second kernel computes
// them.  *launches (if given) receives the number of kernels launched.
// grid (production calls): the compact grids of the yd[].t0 / d0 offsets; nullptr: one grid row per
// problem, as wide as the largest problem's tile count (kernel-level API, per-problem launches).
// dot_form: the dot-product pass's choice of forms -- kDotFormAuto, or for tests kDotFormDense (every
// tile with flagged entries computes all its chains), kDotFormBlocks (per-block and listed entries
// only), kDotFormList (listed entries only), kDotFormTile (as auto, but no tile defers its chains
// to the crossings pass)
enum { kDotFormAuto = 0, kDotFormDense = 1, kDotFormBlocks = 2, kDotFormList = 3, kDotFormTile = 4 };
int recon_launch(const oz2_problem* d, const YDesc* yd, int num, int max_m, int max_n, hipStream_t s, int mode,
                 bool blocked = false, int* launches = nullptr, const ReconGrid* grid = nullptr,
                 int dot_form = kDotFormAuto);

}  // namespace ggemm

// ----------------------------------------------------------------------------- handle
struct ggemm_handle_s {
  hipStream_t stream;
  int device, num_cus;
  int max_problems;
  size_t max_A_elems, max_B_elems, max_C_elems;
  int min_k;

  int8_t* A8; size_t A8_bytes;
  int8_t* B8; size_t B8_bytes;
  int32_t* C32; size_t C32_bytes;
  int32_t* row_shift; size_t row_shift_elems;
  int32_t* col_shift; size_t col_shift_elems;

  // one device descriptor blob mirrored by two pinned host slots (double-buffered)
  void* h_desc; void* d_desc; size_t desc_bytes;
  hipEvent_t desc_done[2]; int desc_next;

  // host scratch sized at create
  ggemm_plan_entry_t* plan;
  int* plan_memo; size_t plan_memo_cap;
  int* emu_idx; int* nat_idx;
  i8_sched_info* loop_info;

  ggemm_device_model_t dm;
  int ws_diag_printed;
  int stats_repair;

  // operand reuse (path EMU_GROUPED_REUSE): host pass storage and per-unique-operand offsets
  struct reuse_arena_s* reuse;
  int* reuse_nmod;
  size_t *ua_off8, *ua_offs, *ub_off8, *ub_offs;
  int reuse_promote;   // GGEMM_REUSE_PROMOTE=1 at create: PROMOTE policy, else EXACT_N
  int digits_colmajor; // GGEMM_DIGITS_COLMAJOR=1 at create: row-major residues and column-major digits
  int i8_mode;         // GGEMM_I8_KERNEL at create: 0 automatic, 1 general kernel only, 2 large-tile kernel
                       // only, the kernel-level layouts (testing)
  int f64_tile;        // GGEMM_F64_TILE at create: 0 automatic, 64 or 128 forces the native GEMM's tile edge
  int packed_max_kp;   // GGEMM_PACKED_MAX_KP at create: calls whose largest Kp is at most this use packed residues
  int packed_env;      // GGEMM_PACKED_MAX_KP was given: its threshold holds for every call
  int i8_persistent;   // GGEMM_I8_SCHED=persistent at create: the persistent work-stealing INT8 kernels
  int safety_chains;   // GGEMM_SAFETY_CHAINS=1 at create: safety-fallback entries always run their fma
                       // chains instead of being decided from prep's non-finite summaries (testing)
  int dot_form;        // GGEMM_DOT_FORM at create: kDotForm* (testing)
  int compact;         // GGEMM_COMPACT at create (default 1; 0: INT8 tiles over all rows / columns, testing)
};
