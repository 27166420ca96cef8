// ggemm.cpp -- handle, validation, path switch and launch sequencing (host, HIP runtime).
//
// Mirrors the reference's orchestration semantics (src/ggemm.cu): all device workspace and host
// scratch are allocated in ggemm_create_ex; a call validates, plans, writes every descriptor into
// a double-buffered pinned slot, issues ONE H2D of the used part of the blob and then the
// kernels: prep -> grouped INT8 GEMM -> reconstruct -> FP64 dot products of the entries the
// reconstruct flagged (4 launches for any group size; 3 when the digits are column-major, where the
// reconstruct computes them itself) plus one grouped native FP64 GEMM launch when some problems
// take a native route.
#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>

#include "call.hpp"
#include "ggemm_profile.h"

namespace ggemm {

// ---- stage timing (include/ggemm_profile.h): a ring of event sets, drained lazily
namespace prof {
constexpr int kRing = 32;
constexpr int kMarks = 5;   // before prep, after prep, after INT8 GEMM, after reconstruct, after native
bool on = false;
bool ready = false;
hipEvent_t ev[kRing][kMarks];
int used[kRing];            // marks recorded in the set (0 = free)
int next = 0;
double sum_ms[4] = {0, 0, 0, 0};
long long calls = 0;
int last_i8 = -1;           // INT8 GEMM kernel of the last grouped call that launched one

void drain(int s) {
  if (!used[s]) return;
  if (hipEventSynchronize(ev[s][kMarks - 1]) == hipSuccess) {
    for (int q = 0; q < 4; ++q) {
      float t = 0.f;
      if (hipEventElapsedTime(&t, ev[s][q], ev[s][q + 1]) == hipSuccess) sum_ms[q] += t;
    }
    ++calls;
  }
  used[s] = 0;
}
// Returns the event set for this call (drained first), or -1 when timing is off.
int begin() {
  if (!on || !ready) return -1;
  const int s = next;
  next = (next + 1) % kRing;
  drain(s);
  return s;
}
void mark(int s, int q, hipStream_t st) {
  if (s < 0) return;
  (void)hipEventRecord(ev[s][q], st);
  if (q == kMarks - 1) used[s] = 1;
}
}  // namespace prof

BlobLayout layout_for(size_t ne, size_t nprep, size_t n_i8, size_t nn, size_t sched_f64, size_t sched_i8) {
  BlobLayout L;
  L.off_oz = 0;
  L.off_yd = align_up(ne * sizeof(oz2_problem), kBufAlign);
  L.off_prep = align_up(L.off_yd + ne * sizeof(YDesc), kBufAlign);
  L.off_po = align_up(L.off_prep + nprep * sizeof(oz2_problem), kBufAlign);
  L.off_i8 = align_up(L.off_po + 2 * (ne + nprep) * sizeof(int), kBufAlign);
  L.off_epi = align_up(L.off_i8 + n_i8 * sizeof(i8_problem), kBufAlign);
  L.off_f64 = align_up(L.off_epi + n_i8 * sizeof(I8Epi), kBufAlign);
  L.off_sf64 = align_up(L.off_f64 + nn * sizeof(F64Problem), kBufAlign);
  L.off_si8 = align_up(L.off_sf64 + sched_f64, kBufAlign);
  L.total = L.off_si8 + sched_i8;
  return L;
}

// src/ggemm.cu:83-100
int validate(ggemm_handle_t h, const ggemm_problem_t* p, int num) {
  if (num < 0 || num > h->max_problems || (num > 0 && !p)) return GGEMM_ERR_INVALID;
  size_t ta = 0, tb = 0, tc = 0;
  for (int g = 0; g < num; ++g) {
    const ggemm_problem_t& q = p[g];
    if (q.m < 0 || q.n < 0 || q.k < 0) return GGEMM_ERR_INVALID;
    if (q.lda < std::max(1, q.m) || q.ldb < std::max(1, q.k) || q.ldc < std::max(1, q.m)) return GGEMM_ERR_INVALID;
    if (q.m > 0 && q.n > 0) {
      if (!q.C) return GGEMM_ERR_INVALID;
      if (q.k > 0 && (!q.A || !q.B)) return GGEMM_ERR_INVALID;
    }
    ta += (size_t)q.m * q.k;
    tb += (size_t)q.k * q.n;
    tc += (size_t)q.m * q.n;
  }
  if (ta > h->max_A_elems || tb > h->max_B_elems || tc > h->max_C_elems) return GGEMM_ERR_WORKSPACE;
  return GGEMM_OK;
}

// src/ggemm.cu:56-65: public GGEMM_REPAIR_* = OZ2_REPAIR_* + 1; default COUNT (EMU_*) / ON (AUTO)
int repair_mode_of(ggemm_path_t path, const ggemm_config_t* cfg) {
  switch (cfg ? cfg->repair_mode : GGEMM_REPAIR_DEFAULT) {
    case GGEMM_REPAIR_DEFAULT: return path == GGEMM_PATH_AUTO ? OZ2_REPAIR_ON : OZ2_REPAIR_COUNT;
    case GGEMM_REPAIR_OFF: return OZ2_REPAIR_OFF;
    case GGEMM_REPAIR_COUNT: return OZ2_REPAIR_COUNT;
    case GGEMM_REPAIR_ON: return OZ2_REPAIR_ON;
    default: return -1;
  }
}

int counters_reset(ggemm_handle_t h, hipStream_t s) {
  if (!h->stats_repair) return GGEMM_OK;
  return oz2_read_counters(nullptr, 1, s) ? GGEMM_ERR_NUMERICS : GGEMM_OK;
}

int counters_read(ggemm_handle_t h, hipStream_t s, ggemm_stats_t* st) {
  st->num_repaired = st->num_uncertified = st->num_safety_fallback = -1;
  if (!h->stats_repair) return GGEMM_OK;
  oz2_counters c{};
  if (oz2_read_counters(&c, 1, s)) return GGEMM_ERR_NUMERICS;
  st->num_repaired = (long long)c.repaired;
  st->num_uncertified = (long long)c.uncertified;
  st->num_safety_fallback = (long long)c.safety_fallback;
  return GGEMM_OK;
}

static void workspace_diag(ggemm_handle_t h, const ggemm_problem_t* probs, const int* emu_idx, int ne) {
  if (h->ws_diag_printed) return;
  h->ws_diag_printed = 1;
  int kmin = 0;
  for (int j = 0; j < ne; ++j) kmin = j ? std::min(kmin, probs[emu_idx[j]].k) : probs[emu_idx[j]].k;
  std::fprintf(stderr,
               "[ggemm] GGEMM_ERR_WORKSPACE: residue/shift workspace exceeded (smallest emulated k = %d, "
               "handle min_k = %d; Kp = round_up(k,32) inflates residues for k < 32 -> create with "
               "ggemm_create_ex(..., min_k <= %d))\n",
               kmin, h->min_k, kmin);
}

// INT8 kernel choice: with packed residues (every Kp small) the general kernel's two workgroups
// per compute unit overlap one tile's epilogue with the other's MFMA work and win; with
// row-major residues (long k) the large tiles' halved operand stream per MFMA wins.
int large_mode(ggemm_handle_t h, const GroupedCall& c) {
  if (h->i8_mode == 1) return kLargeNever;
  if (h->i8_mode == 2) return kLargeForce;
  return c.packed ? kLargeNever : kLargeAuto;
}

// Whether i8_build_schedule can give this call the 256 x 256 kernel under kLargeAuto: every
// (problem, plane) product on automatic 256 x 128 tiles, kept by the group-level fill rule (at
// least two such tiles per compute unit), and a 256 x 256 tile for every compute unit.
bool large_auto_fits(ggemm_handle_t h, const ggemm_problem_t* probs, const int* emu_idx,
                     const ggemm_plan_entry_t* plan, int ne) {
  long long t0 = 0, t256 = 0;
  for (int j = 0; j < ne; ++j) {
    const ggemm_problem_t& p = probs[emu_idx[j]];
    if (i8_auto_tile_cfg(p.m, p.n) != 0) return false;
    const long long planes = plan[emu_idx[j]].num_moduli + 1;
    t0 += planes * ((p.m + 255) / 256) * ((p.n + 127) / 128);
    t256 += planes * ((p.m + 255) / 256) * ((p.n + 255) / 256);
  }
  return ne > 0 && t0 >= 2LL * h->num_cus && t256 >= h->num_cus;
}

int build_grouped(ggemm_handle_t h, const ggemm_problem_t* probs, int num, const ggemm_plan_entry_t* plan,
                  int* emu_idx, int* nat_idx, char* hb, const char* db, size_t cap, GroupedCall* out,
                  ggemm_stats_t* st, const reuse_plan* rp) {
  GroupedCall c;
  int nmax = 0, pmax = 0;
  size_t SA = 0, SB = 0, SC = 0, rows = 0, cols = 0;
  for (int g = 0; g < num; ++g) {
    const ggemm_plan_entry_t& e = plan[g];
    if (e.route == GGEMM_ROUTE_EMPTY) continue;
    if (e.route != GGEMM_ROUTE_EMU) { nat_idx[c.nn++] = g; continue; }
    const ggemm_problem_t& p = probs[g];
    const size_t kp = (size_t)kp_of(p.k);
    emu_idx[c.ne++] = g;
    if (!rp) {   // every emulated problem owns its residue and shift blocks
      SA += align_up((size_t)p.m * kp, kBufAlign);
      SB += align_up((size_t)p.n * kp, kBufAlign);
      rows += align_up((size_t)OZ2_ROW_WS_PER_ROW * p.m, 64);
      cols += align_up((size_t)OZ2_ROW_WS_PER_ROW * p.n, 64);
    }
    SC += align_up((size_t)p.m * p.n, kBufAlign / 4);
    const int planes = e.num_moduli + OZ2_EXTRA_PLANES;
    c.n_i8 += planes;
    nmax = std::max(nmax, e.num_moduli);
    pmax = std::max(pmax, planes);
  }
  if (rp) {   // residue and shift blocks per unique operand (src/ggemm.cu:428-449)
    for (int u = 0; u < rp->num_ua; ++u) {
      const ggemm_problem_t& p = probs[rp->ua_rep[u]];
      h->ua_off8[u] = SA;
      h->ua_offs[u] = rows;
      SA += align_up((size_t)p.m * kp_of(p.k), kBufAlign);
      rows += align_up((size_t)OZ2_ROW_WS_PER_ROW * p.m, 64);
      pmax = std::max(pmax, rp->ua_nmod[u] + OZ2_EXTRA_PLANES);
      c.pmax_m = std::max(c.pmax_m, p.m);
    }
    for (int u = 0; u < rp->num_ub; ++u) {
      const ggemm_problem_t& p = probs[rp->ub_rep[u]];
      h->ub_off8[u] = SB;
      h->ub_offs[u] = cols;
      SB += align_up((size_t)p.n * kp_of(p.k), kBufAlign);
      cols += align_up((size_t)OZ2_ROW_WS_PER_ROW * p.n, 64);
      pmax = std::max(pmax, rp->ub_nmod[u] + OZ2_EXTRA_PLANES);
      c.pmax_n = std::max(c.pmax_n, p.n);
    }
    c.nprep = rp->num_ua + rp->num_ub;
    if (c.nprep > 65535) return GGEMM_ERR_INVALID;
  }
  if ((size_t)pmax * SA > h->A8_bytes || (size_t)pmax * SB > h->B8_bytes ||
      (size_t)pmax * SC * sizeof(int32_t) > h->C32_bytes || rows > h->row_shift_elems || cols > h->col_shift_elems) {
    workspace_diag(h, probs, emu_idx, c.ne);
    return GGEMM_ERR_WORKSPACE;
  }
  if (c.ne > 65535) return GGEMM_ERR_INVALID;

  st->num_fallback = 0;
  for (int i = 0; i < c.nn; ++i) {
    const int r = plan[nat_idx[i]].route;
    st->num_fallback += (r != GGEMM_ROUTE_EMU && r != GGEMM_ROUTE_EMPTY && r != GGEMM_ROUTE_K_ZERO &&
                         r != GGEMM_ROUTE_ALPHA_ZERO);
  }
  c.nmax = nmax;
  st->moduli_min = c.ne ? GGEMM_MAX_MODULI : 0;
  st->moduli_max = nmax;
  for (int j = 0; j < c.ne; ++j) st->moduli_min = std::min(st->moduli_min, plan[emu_idx[j]].num_moduli);
  st->reuse_enabled = rp ? 1 : 0;
  st->num_unique_A = rp ? rp->num_ua : c.ne;
  st->num_unique_B = rp ? rp->num_ub : c.ne;
  st->num_promoted = rp ? rp->num_promoted : 0;

  const size_t s_i8 = c.ne ? sched_bytes((int)c.n_i8) : 0;
  const size_t s_f64 = c.nn ? sched_bytes(c.nn) : 0;
  c.L = layout_for(c.ne, c.nprep, c.n_i8, c.nn, s_f64, s_i8);
  if (c.L.total > cap) return GGEMM_ERR_INVALID;
  oz2_problem* hoz = reinterpret_cast<oz2_problem*>(hb + c.L.off_oz);
  YDesc* hyd = reinterpret_cast<YDesc*>(hb + c.L.off_yd);
  i8_problem* hi8 = reinterpret_cast<i8_problem*>(hb + c.L.off_i8);
  I8Epi* hepi = reinterpret_cast<I8Epi*>(hb + c.L.off_epi);
  F64Problem* hf = reinterpret_cast<F64Problem*>(hb + c.L.off_f64);
  const CrtTables* tab = host_tables();
  // product workspace (the C32 buffer): CRT digit planes [plane < nmax][problem] of SY bytes
  // each, then the int32 abs-plane products.  Column-major fits because nmax SY + 4 SC <=
  // pmax 4 SC; the blocked layout (whole 16 x 16 blocks) is used when its padded planes fit too.
  // The blocked layout also keeps the dot-product flags (32 bytes per 16 x 16 block) after the L planes,
  // and after them, when they fit and every problem preps its own operands, the non-finite row /
  // column summaries (kNfWords words per row and column).
  size_t SY = 0, SYb = 0, SLb = 0, SFb = 0, SNF = 0;
  for (int j = 0; j < c.ne; ++j) {
    const ggemm_problem_t& p = probs[emu_idx[j]];
    SY += align_up((size_t)p.m * p.n, kBufAlign);
    SYb += align_up(blocked_plane_entries(p.m, p.n), kBufAlign);
    SLb += align_up(blocked_plane_entries(p.m, p.n), kBufAlign / 4) * sizeof(int32_t);
    SFb += align_up(flag_bytes(p.m, p.n, blocked_plane_entries(p.m, p.n)), kBufAlign);
    SNF += align_up((size_t)(p.m + p.n) * kNfWords * sizeof(int32_t), kBufAlign);
  }
  c.blocked = !h->digits_colmajor && (size_t)nmax * SYb + SLb + SFb <= h->C32_bytes;
  const bool nfsum = c.blocked && !rp && !h->safety_chains && (size_t)nmax * SYb + SLb + SFb + SNF <= h->C32_bytes;
  // Packed residue planes make every 64-byte k-stage of a tile's rows contiguous, which the INT8
  // GEMM's operand stream prefers at moderate k (measured: 1024^3 products 14 % faster together
  // with the blocked digits); at k = 16384 the 256 x 256 kernel streams row-major planes better
  // (5 % slower packed).  The choice is per problem (Kp <= packed_kp), so the long-k problems of a
  // ragged group do not put its short ones on row-major planes; and when the call cannot take the
  // 256 x 256 kernel at all, every problem is packed -- the general kernel streams packed planes
  // better at long k too (ragged group G = 128, k up to 8192: GEMM 2.27 -> 2.13 ms, prep 1.87 ->
  // 1.76 ms, same box).
  int max_kp = 0;
  for (int j = 0; j < c.ne; ++j) max_kp = std::max(max_kp, kp_of(probs[emu_idx[j]].k));
  c.packed_kp = h->digits_colmajor ? 0 : h->packed_max_kp;
  if (!h->digits_colmajor && !h->packed_env && max_kp > c.packed_kp && h->i8_mode != 2 &&
      (h->i8_mode == 1 || !large_auto_fits(h, probs, emu_idx, plan, c.ne)))
    c.packed_kp = kKpMaxPacked;
  c.packed = max_kp <= c.packed_kp;
  c.dot_form = h->dot_form;
  if (c.blocked) SY = SYb;
  uint8_t* ybase = reinterpret_cast<uint8_t*>(h->C32);
  int32_t* lbase = reinterpret_cast<int32_t*>(ybase + (size_t)nmax * SY);
  uint8_t* fbase = reinterpret_cast<uint8_t*>(lbase) + SLb;
  uint8_t* nbase = fbase + SFb;
  size_t oa = 0, ob = 0, orow = 0, ocol = 0, q = 0, oy = 0, ol = 0, of = 0, onf = 0, oat = 0;
  for (int j = 0; j < c.ne; ++j) {
    const int g = emu_idx[j];
    const ggemm_problem_t& p = probs[g];
    const ggemm_plan_entry_t& e = plan[g];
    const size_t kp = (size_t)kp_of(p.k);
    oz2_problem& o = hoz[j];
    o.m = p.m; o.n = p.n; o.k = p.k; o.kp = (int)kp; o.num_moduli = e.num_moduli;
    o.lda = p.lda; o.ldb = p.ldb; o.ldc = p.ldc;
    o.A = p.A; o.B = p.B; o.C = p.C; o.alpha = p.alpha; o.beta = p.beta;
    if (rp) {
      // the shared operands were prepped with their unique operand's N: it must be this problem's
      const int ua = rp->prob_a[g], ub = rp->prob_b[g];
      if (ua < 0 || ub < 0 || rp->ua_nmod[ua] != e.num_moduli || rp->ub_nmod[ub] != e.num_moduli)
        return GGEMM_ERR_NUMERICS;
      o.A8 = h->A8 + h->ua_off8[ua]; o.row_shift = h->row_shift + h->ua_offs[ua];
      o.B8 = h->B8 + h->ub_off8[ub]; o.col_shift = h->col_shift + h->ub_offs[ub];
    } else {
      o.A8 = h->A8 + oa; o.row_shift = h->row_shift + orow;
      o.B8 = h->B8 + ob; o.col_shift = h->col_shift + ocol;
    }
    o.a8_mod_stride = SA;
    o.b8_mod_stride = SB;
    YDesc& yd = hyd[j];
    yd.Y = ybase + oy;
    yd.y_stride = SY;
    yd.L = lbase + ol;
    yd.F = c.blocked ? reinterpret_cast<uint64_t*>(fbase + of) : nullptr;
    yd.nf = nfsum ? reinterpret_cast<int32_t*>(nbase + onf) : nullptr;
    yd.X = c.blocked ? reinterpret_cast<uint64_t*>(fbase + of + blocked_plane_entries(p.m, p.n) / 8) : nullptr;
    yd.fr = c.blocked ? reinterpret_cast<uint8_t*>(yd.X + ((p.m + 63) / 64 + (p.n + 63) / 64 + 1)) : nullptr;
    yd.fc = c.blocked ? yd.fr + (((size_t)p.m + 3) & ~(size_t)3) : nullptr;
    {   // the gather workspace: the problem's m k doubles in the residue planes, while they last
      const size_t at = align_up((size_t)p.m * (size_t)p.k * sizeof(double), kBufAlign);
      yd.AT = nullptr;
      if (c.blocked && oat + at <= h->A8_bytes) {
        yd.AT = reinterpret_cast<double*>(reinterpret_cast<char*>(h->A8) + oat);
        oat += at;
      }
    }
    yd.nff = 0;
    yd.fla = 0;
    {   // compact reconstruct / dot-product grids
      const int rm = c.blocked ? kReconTileMB : kReconTileMC, rn = c.blocked ? kReconTileNB : kReconTileNC;
      const long long rt = (long long)((p.m + rm - 1) / rm) * ((p.n + rn - 1) / rn);
      const long long dt = c.blocked ? (long long)((p.m + kDotTile - 1) / kDotTile) * ((p.n + kDotTile - 1) / kDotTile) : 0;
      const long long bt = c.blocked ? (long long)((p.m + kDotTile - 1) / kDotTile) : 0;   // row bands
      ReconGrid& rg = c.rgrid;
      if (rg.tiles + rt > 0x7fffffffLL || rg.dtiles + dt > 0x7fffffffLL || rg.bands + bt > 0x7fffffffLL)
        return GGEMM_ERR_INVALID;
      yd.t0 = rg.tiles;
      yd.d0 = rg.dtiles;
      yd.b0 = rg.bands;
      rg.per = j == 0 ? (int)rt : (rg.per == (int)rt ? rg.per : 0);
      rg.dper = j == 0 ? (int)dt : (rg.dper == (int)dt ? rg.dper : 0);
      rg.bper = j == 0 ? (int)bt : (rg.bper == (int)bt ? rg.bper : 0);
      rg.tiles += (int)rt;
      rg.dtiles += (int)dt;
      rg.bands += (int)bt;
      rg.ne = j + 1;
    }
    o.C32 = lbase + ol; o.c32_mod_stride = 0;   // the reconstruct reads yd, not C32
    const int N = e.num_moduli;
    for (int l = 0; l <= N; ++l, ++q) {
      i8_problem& d = hi8[q];
      d.m = p.m; d.n = p.n; d.kp = (int)kp;
      d.A = o.A8 + (size_t)l * SA; d.B = o.B8 + (size_t)l * SB;
      d.tile_cfg = -1;
      if (l < N) {
        d.C = reinterpret_cast<int32_t*>(ybase + oy + (size_t)l * SY);
        hepi[q] = i8_epi_residue((uint32_t)tab->p[l], (int)kp);   // A residues carry q_l: the byte is y_l
      } else {
        d.C = lbase + ol;
        hepi[q] = I8Epi{0u, 1u, 0u, 0u};
      }
      if (c.blocked) hepi[q].mode |= kEpiBlocked;
      if ((int)kp <= c.packed_kp) hepi[q].mode |= kEpiPacked;
      hepi[q].rs = o.row_shift;
      hepi[q].cs = o.col_shift;
      hepi[q].nf = reinterpret_cast<const int*>(db + c.L.off_yd + j * sizeof(YDesc) + offsetof(YDesc, nff));
      // finite rows x finite columns only, for problems prep finds non-finite (its own residues)
      hepi[q].yd = (c.blocked && !rp && h->compact) ? reinterpret_cast<const YDesc*>(db + c.L.off_yd + j * sizeof(YDesc))
                                                    : nullptr;
    }
    const size_t plane = c.blocked ? blocked_plane_entries(p.m, p.n) : (size_t)p.m * p.n;
    oy += align_up(plane, kBufAlign);
    ol += align_up(plane, kBufAlign / 4);
    of += align_up(flag_bytes(p.m, p.n, blocked_plane_entries(p.m, p.n)), kBufAlign);
    onf += align_up((size_t)(p.m + p.n) * kNfWords * sizeof(int32_t), kBufAlign);
    oa += align_up((size_t)p.m * kp, kBufAlign);
    ob += align_up((size_t)p.n * kp, kBufAlign);
    orow += align_up((size_t)OZ2_ROW_WS_PER_ROW * p.m, 64);
    ocol += align_up((size_t)OZ2_ROW_WS_PER_ROW * p.n, 64);
    c.max_m = std::max(c.max_m, p.m);
    c.max_n = std::max(c.max_n, p.n);
  }
  if (c.blocked && c.ne > 0) {
    // crossings workgroups: about 4 per CU over the call, each problem's share in proportion to its
    // dot-pass tiles (at least one, at most one per tile); a workgroup loops over its problem's tiles
    ReconGrid& rg = c.rgrid;
    const long long budget = 4LL * std::max(1, h->num_cus), T = std::max(1, rg.dtiles);
    long long x0 = 0;
    for (int j = 0; j < c.ne; ++j) {
      YDesc& yd = hyd[j];
      const long long dt = (j + 1 < c.ne ? hyd[j + 1].d0 : rg.dtiles) - yd.d0;
      const long long xn = std::max(1LL, std::min(dt, (budget * dt + T - 1) / T));
      if (x0 + xn > 0x7fffffffLL) return GGEMM_ERR_INVALID;
      yd.x0 = (int)x0;
      yd.xn = (int)xn;
      rg.xper = j == 0 ? (int)xn : (rg.xper == (int)xn ? rg.xper : 0);
      x0 += xn;
    }
    rg.xwgs = (int)x0;
  }
  if (rp) {
    // prep descriptors (src/ggemm.cu:544-569): unique A as A-only problems (n = 0), then unique B
    // as B-only problems (m = 0); alpha = 1 so the prep runs; N = the operand's moduli count
    oz2_problem* hpr = reinterpret_cast<oz2_problem*>(hb + c.L.off_prep);
    for (int u = 0; u < rp->num_ua; ++u) {
      const ggemm_problem_t& p = probs[rp->ua_rep[u]];
      oz2_problem& o = hpr[u];
      std::memset(&o, 0, sizeof o);
      o.m = p.m; o.n = 0; o.k = p.k; o.kp = kp_of(p.k); o.num_moduli = rp->ua_nmod[u];
      o.lda = p.lda; o.ldb = p.ldb; o.ldc = std::max(1, p.m);
      o.A = p.A; o.alpha = 1.0;
      o.A8 = h->A8 + h->ua_off8[u]; o.a8_mod_stride = SA; o.b8_mod_stride = SB;
      o.row_shift = h->row_shift + h->ua_offs[u];
    }
    for (int u = 0; u < rp->num_ub; ++u) {
      const ggemm_problem_t& p = probs[rp->ub_rep[u]];
      oz2_problem& o = hpr[rp->num_ua + u];
      std::memset(&o, 0, sizeof o);
      o.m = 0; o.n = p.n; o.k = p.k; o.kp = kp_of(p.k); o.num_moduli = rp->ub_nmod[u];
      o.lda = 1; o.ldb = p.ldb; o.ldc = 1;
      o.B = p.B; o.alpha = 1.0;
      o.B8 = h->B8 + h->ub_off8[u]; o.a8_mod_stride = SA; o.b8_mod_stride = SB;
      o.col_shift = h->col_shift + h->ub_offs[u];
    }
  }
  {   // prep order: descriptors by descending Kp, then by descending operand volume (m + n) Kp.  A
      // block (32 A rows or 8 B columns) takes time in proportion to Kp, and a problem's blocks run
      // side by side, so the longest blocks go first (list scheduling of the blocks) and the short
      // ones fill in behind them; by volume alone, a long-k problem with few rows came last and
      // its blocks ran on after all others (ragged group: 0.6 ms of 1.8)
    const oz2_problem* pd = rp ? reinterpret_cast<const oz2_problem*>(hb + c.L.off_prep) : hoz;
    const int np = rp ? c.nprep : c.ne;
    int* po = reinterpret_cast<int*>(hb + c.L.off_po);
    for (int i = 0; i < np; ++i) po[i] = i;
    auto vol = [&](int i) { return ((long long)pd[i].m + pd[i].n) * pd[i].kp; };
    // ties by index (the order a stable sort keeps; std::sort takes no temporary buffer)
    std::sort(po, po + np, [&](int a, int b) {
      if (pd[a].kp != pd[b].kp) return pd[a].kp > pd[b].kp;
      return vol(a) != vol(b) ? vol(a) > vol(b) : a < b;
    });
    // compact grid: each problem's first block, in dispatch order (problems prep skips get none)
    int* pof = po + np;
    long long tot = 0;
    for (int i = 0; i < np; ++i) {
      const oz2_problem& o = pd[po[i]];
      if (tot > 0x7fffffffLL) return GGEMM_ERR_INVALID;
      pof[i] = (int)tot;
      if (o.alpha != 0.0 && o.num_moduli >= 1 && o.num_moduli <= kMaxModuli)
        tot += (long long)(o.m + kPrepRows - 1) / kPrepRows + (o.n + kPrepCols - 1) / kPrepCols;
    }
    if (tot > 0x7fffffffLL) return GGEMM_ERR_INVALID;
    c.prep_blocks = tot;
  }
  for (int i = 0; i < c.nn; ++i) hf[i] = f64_of(probs[nat_idx[i]]);
  if (c.nn && f64_build_schedule(hf, c.nn, hb + c.L.off_sf64, s_f64, &c.f64_tiles, nullptr, h->f64_tile))
    return GGEMM_ERR_INVALID;
  if (c.ne && i8_build_schedule(hi8, (int)c.n_i8, hb + c.L.off_si8, s_i8, &c.i8info, h->num_cus, large_mode(h, c),
                                   &c.i8_kernel, h->i8_persistent != 0, hepi, &c.i8_hw))
    return GGEMM_ERR_I8GEMM;
  c.h2d_bytes = c.ne ? c.L.off_si8 + c.i8info.bytes_used : c.L.off_si8;
  *out = c;
  return GGEMM_OK;
}

int enqueue_grouped(const GroupedCall& c, const char* db, hipStream_t s, int repair, int* launches, int prof_set) {
  const oz2_problem* doz = reinterpret_cast<const oz2_problem*>(db + c.L.off_oz);
  const YDesc* dyd = reinterpret_cast<const YDesc*>(db + c.L.off_yd);
  prof::mark(prof_set, 0, s);
  if (c.ne > 0) {
    const bool shared = c.nprep > 0;   // operand reuse: prep once per unique operand
    if (prep_launch(shared ? reinterpret_cast<const oz2_problem*>(db + c.L.off_prep) : doz, shared ? c.nprep : c.ne,
                    shared ? c.pmax_m : c.max_m, shared ? c.pmax_n : c.max_n, s, 1, c.packed_kp, c.nmax,
                    shared ? nullptr : dyd, reinterpret_cast<const int*>(db + c.L.off_po),
                    reinterpret_cast<const int*>(db + c.L.off_po) + (shared ? c.nprep : c.ne), c.prep_blocks))
      return GGEMM_ERR_NUMERICS;
    ++*launches;
    prof::mark(prof_set, 1, s);
    if (i8_launch(reinterpret_cast<const i8_problem*>(db + c.L.off_i8), reinterpret_cast<const I8Epi*>(db + c.L.off_epi),
                  db + c.L.off_si8, &c.i8info, s, c.i8_kernel, c.i8_hw))
      return GGEMM_ERR_I8GEMM;
    *launches += c.i8info.num_launches;
    prof::last_i8 = c.i8_kernel;
    prof::mark(prof_set, 2, s);
    int nr = 0;
    if (recon_launch(doz, dyd, c.ne, c.max_m, c.max_n, s, repair, c.blocked, &nr, &c.rgrid, c.dot_form))
      return GGEMM_ERR_NUMERICS;
    *launches += nr;
    prof::mark(prof_set, 3, s);
  } else {
    prof::mark(prof_set, 1, s);
    prof::mark(prof_set, 2, s);
    prof::mark(prof_set, 3, s);
  }
  if (c.nn > 0 && c.f64_tiles > 0) {
    if (f64_launch(reinterpret_cast<const F64Problem*>(db + c.L.off_f64), db + c.L.off_sf64, c.f64_tiles, s))
      return GGEMM_ERR_CUBLAS;
    ++*launches;
  }
  prof::mark(prof_set, 4, s);
  return GGEMM_OK;
}

}  // namespace ggemm

using namespace ggemm;

namespace {

constexpr int kSlots = 2;
#define HIPC(x) do { if ((x) != hipSuccess) return GGEMM_ERR_CUDA; } while (0)

char* host_slot(ggemm_handle_t h, int s) { return static_cast<char*>(h->h_desc) + (size_t)s * h->desc_bytes; }

// A slot may be rewritten only after the call that used it two calls ago has drained.
int acquire_slot(ggemm_handle_t h, int* slot) {
  const int s = h->desc_next;
  h->desc_next = (s + 1) % kSlots;
  HIPC(hipEventSynchronize(h->desc_done[s]));
  *slot = s;
  return GGEMM_OK;
}
int release_slot(ggemm_handle_t h, int slot) {
  HIPC(hipEventRecord(h->desc_done[slot], h->stream));
  return GGEMM_OK;
}

// max over k >= min_k of round_up(k, 32) / k (attained in [min_k, min_k + 32))
double kp_inflation(int min_k) {
  double f = 1.0;
  for (int k = min_k; k < min_k + kKpAlign; ++k) f = std::max(f, (double)align_up((size_t)k, kKpAlign) / k);
  return f;
}

}  // namespace

// src/ggemm.cu:228-341 sizing rules (see ggemm_create_ex)
void ggemm::size_workspace(ggemm_handle_s* h, int max_problems, size_t max_A, size_t max_B, size_t max_C, int min_k) {
  const size_t P = (size_t)max_problems;
  const size_t M = (size_t)kMaxPlanes;
  const double infl = std::max(2.0, kp_inflation(min_k));
  const size_t planeA = (size_t)std::ceil(infl * (double)max_A) + P * kBufAlign;
  const size_t planeB = (size_t)std::ceil(infl * (double)max_B) + P * kBufAlign;
  h->A8_bytes = M * planeA;
  h->B8_bytes = M * planeB;
  h->C32_bytes = M * (max_C + P * (kBufAlign / 4)) * sizeof(int32_t);
  const size_t rowsA = std::min(max_A, M * planeA / (3 * kKpAlign));
  const size_t colsB = std::min(max_B, M * planeB / (3 * kKpAlign));
  h->row_shift_elems = OZ2_ROW_WS_PER_ROW * rowsA + P * 64;
  h->col_shift_elems = OZ2_ROW_WS_PER_ROW * colsB + P * 64;
  // descriptor blob: worst case over the paths (grouped, per-plane and per-problem images)
  const size_t n_i8 = P * M;
  const size_t si8 = std::max({sched_img((int)n_i8), n_i8 * sched_img(1), P * sched_img(kMaxPlanes)});
  const size_t sf64 = std::max(sched_img((int)P), P * sched_img(1));
  const BlobLayout Lw = layout_for(P, 2 * P, n_i8, P, sf64, sched_img((int)n_i8));
  h->desc_bytes = align_up(Lw.total + si8 + kBufAlign, kBufAlign);
}

namespace {

// Native problems idx[0..cnt): one grouped FP64 launch, or one launch per problem (loop).
int run_native(ggemm_handle_t h, const ggemm_problem_t* probs, const int* idx, int cnt, bool grouped, int* launches) {
  if (cnt == 0) return GGEMM_OK;
  int slot, r;
  if ((r = acquire_slot(h, &slot))) return r;
  char* hb = host_slot(h, slot);
  char* db = static_cast<char*>(h->d_desc);
  const size_t per = grouped ? sched_img(cnt) : sched_img(1);
  const size_t simg = grouped ? per : per * cnt;
  const BlobLayout L = layout_for(0, 0, 0, cnt, simg, 0);
  F64Problem* hf = reinterpret_cast<F64Problem*>(hb + L.off_f64);
  for (int i = 0; i < cnt; ++i) hf[i] = f64_of(probs[idx[i]]);
  int tiles[1] = {0};
  int* tl = grouped ? tiles : h->emu_idx;   // per-problem tile counts (host scratch)
  for (int i = 0; i < (grouped ? 1 : cnt); ++i) {
    const F64Problem* src = grouped ? hf : hf + i;
    if (f64_build_schedule(src, grouped ? cnt : 1, hb + L.off_sf64 + (size_t)i * per, per, &tl[i], nullptr,
                           h->f64_tile)) {
      release_slot(h, slot);
      return GGEMM_ERR_INVALID;
    }
  }
  if (hipMemcpyAsync(db, hb, L.total, hipMemcpyHostToDevice, h->stream) != hipSuccess) {
    release_slot(h, slot);
    return GGEMM_ERR_CUDA;
  }
  const F64Problem* df = reinterpret_cast<const F64Problem*>(db + L.off_f64);
  for (int i = 0; i < (grouped ? 1 : cnt) && !r; ++i) {
    if (tl[i] == 0) continue;
    if (f64_launch(grouped ? df : df + i, db + L.off_sf64 + (size_t)i * per, tl[i], h->stream)) r = GGEMM_ERR_CUBLAS;
    else ++*launches;
  }
  const int r2 = release_slot(h, slot);
  return r ? r : r2;
}

int path_native(ggemm_handle_t h, bool grouped, const ggemm_problem_t* probs, int num, ggemm_stats_t* st) {
  int cnt = 0;
  for (int g = 0; g < num; ++g)
    if (probs[g].m > 0 && probs[g].n > 0) h->nat_idx[cnt++] = g;
  return run_native(h, probs, h->nat_idx, cnt, grouped && cnt >= 2, &st->kernel_launches);
}

// EMU_LOOP (one INT8 launch per plane) and EMU_LOOP_BATCHED (one per problem): same descriptors
// and kernels as the grouped path, launched per problem.
int path_emu_loop(ggemm_handle_t h, bool batched, const ggemm_problem_t* probs, int num, ggemm_stats_t* st,
                  int repair) {
  GroupedCall c;
  int slot, r;
  if ((r = acquire_slot(h, &slot))) return r;
  char* hb = host_slot(h, slot);
  char* db = static_cast<char*>(h->d_desc);
  r = build_grouped(h, probs, num, h->plan, h->emu_idx, h->nat_idx, hb, db, h->desc_bytes, &c, st);
  if (r) { release_slot(h, slot); return r; }
  // per-problem (or per-plane) schedule images after the grouped layout
  const size_t per = batched ? sched_img(kMaxPlanes) : sched_img(1);
  const size_t base = align_up(c.L.total, kBufAlign);
  const size_t nimg = batched ? (size_t)c.ne : c.n_i8;
  if (base + nimg * per > h->desc_bytes) { release_slot(h, slot); return GGEMM_ERR_INVALID; }
  const i8_problem* hi8 = reinterpret_cast<const i8_problem*>(hb + c.L.off_i8);
  const oz2_problem* hoz = reinterpret_cast<const oz2_problem*>(hb + c.L.off_oz);
  size_t q = 0;
  for (int j = 0; j < c.ne && !r; ++j) {
    const int planes = hoz[j].num_moduli + OZ2_EXTRA_PLANES;
    if (batched) {
      if (i8_build_schedule(hi8 + q, planes, hb + base + j * per, per, &h->loop_info[j], h->num_cus, kLargeNever,
                            nullptr, h->i8_persistent != 0))
        r = GGEMM_ERR_I8GEMM;
    } else {
      for (int l = 0; l < planes && !r; ++l)
        if (i8_build_schedule(hi8 + q + l, 1, hb + base + (q + l) * per, per, &h->loop_info[q + l], h->num_cus,
                              kLargeNever, nullptr, h->i8_persistent != 0))
          r = GGEMM_ERR_I8GEMM;
    }
    q += planes;
  }
  if (!r && hipMemcpyAsync(db, hb, base + nimg * per, hipMemcpyHostToDevice, h->stream) != hipSuccess) r = GGEMM_ERR_CUDA;
  int& nl = st->kernel_launches;
  const oz2_problem* doz = reinterpret_cast<const oz2_problem*>(db + c.L.off_oz);
  const YDesc* dyd = reinterpret_cast<const YDesc*>(db + c.L.off_yd);
  const i8_problem* di8 = reinterpret_cast<const i8_problem*>(db + c.L.off_i8);
  const I8Epi* depi = reinterpret_cast<const I8Epi*>(db + c.L.off_epi);
  q = 0;
  const int i8k = h->i8_persistent ? kI8Persistent : kI8General;
  for (int j = 0; j < c.ne && !r; ++j) {
    const int planes = hoz[j].num_moduli + OZ2_EXTRA_PLANES;
    if (prep_launch(doz + j, 1, hoz[j].m, hoz[j].n, h->stream, 1, c.packed_kp, hoz[j].num_moduli, dyd + j)) {
      r = GGEMM_ERR_NUMERICS;
      break;
    }
    ++nl;
    if (batched) {
      if (i8_launch(di8 + q, depi + q, db + base + j * per, &h->loop_info[j], h->stream, i8k)) {
        r = GGEMM_ERR_I8GEMM;
        break;
      }
      nl += h->loop_info[j].num_launches;
    } else {
      for (int l = 0; l < planes && !r; ++l) {
        if (i8_launch(di8 + q + l, depi + q + l, db + base + (q + l) * per, &h->loop_info[q + l], h->stream, i8k))
          r = GGEMM_ERR_I8GEMM;
        else nl += h->loop_info[q + l].num_launches;
      }
      if (r) break;
    }
    q += planes;
    int nr = 0;
    if (recon_launch(doz + j, dyd + j, 1, hoz[j].m, hoz[j].n, h->stream, repair, c.blocked, &nr, nullptr, c.dot_form)) {
      r = GGEMM_ERR_NUMERICS;
      break;
    }
    nl += nr;
  }
  if (!r && c.nn > 0 && c.f64_tiles > 0) {
    if (f64_launch(reinterpret_cast<const F64Problem*>(db + c.L.off_f64), db + c.L.off_sf64, c.f64_tiles, h->stream))
      r = GGEMM_ERR_CUBLAS;
    else
      ++nl;
  }
  const int r2 = release_slot(h, slot);
  return r ? r : r2;
}

// src/ggemm.cu:375-403: REUSE plans like EMU_GROUPED, EMU_LOOP_BATCHED like EMU_LOOP
int path_emu(ggemm_handle_t h, ggemm_path_t path, const ggemm_config_t* cfg, const ggemm_problem_t* probs, int num,
             ggemm_stats_t* st, int repair) {
  const bool reuse = path == GGEMM_PATH_EMU_GROUPED_REUSE;
  const ggemm_path_t plan_path = path == GGEMM_PATH_EMU_LOOP_BATCHED ? GGEMM_PATH_EMU_LOOP
                                 : reuse                            ? GGEMM_PATH_EMU_GROUPED
                                                                    : path;
  int r = ggemm_plan_ex(probs, num, cfg, plan_path, &h->dm, h->plan, h->plan_memo, h->plan_memo_cap);
  if (r) return r;
  if (path == GGEMM_PATH_EMU_LOOP || path == GGEMM_PATH_EMU_LOOP_BATCHED)
    return path_emu_loop(h, path == GGEMM_PATH_EMU_LOOP_BATCHED, probs, num, st, repair);
  reuse_plan rp{};
  if (reuse) {   // after the plan, before any sizing
    for (int g = 0; g < num; ++g)
      h->reuse_nmod[g] = h->plan[g].route == GGEMM_ROUTE_EMU ? h->plan[g].num_moduli : 0;
    rp = build_operand_reuse(h->reuse, probs, num, h->reuse_nmod, h->reuse_promote ? REUSE_PROMOTE : REUSE_EXACT_N);
    if (rp.status != REUSE_OK) return rp.status == REUSE_ERR_CAPACITY ? GGEMM_ERR_WORKSPACE : GGEMM_ERR_INVALID;
    if (h->reuse_promote)   // every problem of a sharing component runs with the component's largest N
      for (int g = 0; g < num; ++g)
        if (h->plan[g].route == GGEMM_ROUTE_EMU) h->plan[g].num_moduli = rp.eff_nmod[g];
  }
  int slot;
  if ((r = acquire_slot(h, &slot))) return r;
  char* hb = host_slot(h, slot);
  char* db = static_cast<char*>(h->d_desc);
  GroupedCall c;
  r = build_grouped(h, probs, num, h->plan, h->emu_idx, h->nat_idx, hb, db, h->desc_bytes, &c, st,
                    reuse ? &rp : nullptr);
  if (!r && c.h2d_bytes && hipMemcpyAsync(db, hb, c.h2d_bytes, hipMemcpyHostToDevice, h->stream) != hipSuccess)
    r = GGEMM_ERR_CUDA;
  if (!r) r = enqueue_grouped(c, db, h->stream, repair, &st->kernel_launches, prof::begin());
  const int r2 = release_slot(h, slot);
  return r ? r : r2;
}

}  // namespace

extern "C" int ggemm_profile_enable(int on) {
  using namespace ggemm::prof;
  if (on && !ready) {
    for (int s = 0; s < kRing; ++s)
      for (int q = 0; q < kMarks; ++q)
        if (hipEventCreate(&ev[s][q]) != hipSuccess) return GGEMM_ERR_CUDA;
    ready = true;
  }
  ggemm::prof::on = on != 0;
  return GGEMM_OK;
}

extern "C" int ggemm_profile_read(double* ms, long long* n, int reset) {
  using namespace ggemm::prof;
  if (ready)
    for (int s = 0; s < kRing; ++s) drain(s);
  if (ms)
    for (int q = 0; q < 4; ++q) ms[q] = sum_ms[q];
  if (n) *n = calls;
  if (reset) {
    for (int q = 0; q < 4; ++q) sum_ms[q] = 0;
    calls = 0;
  }
  return GGEMM_OK;
}

extern "C" const char* ggemm_profile_i8_kernel(void) {
  switch (ggemm::prof::last_i8) {
    case ggemm::kI8General: return "i8_grouped_kernel";
    case ggemm::kI8Large: return "i8_large_kernel";
    case ggemm::kI8General | ggemm::kI8Persistent: return "i8_grouped_persistent_kernel";
    case ggemm::kI8Large | ggemm::kI8Persistent: return "i8_large_persistent_kernel";
    default: return "";
  }
}

extern "C" void ggemm_destroy(ggemm_handle_t h) {
  if (!h) return;
  (void)hipStreamSynchronize(h->stream);
  for (int s = 0; s < kSlots; ++s)
    if (h->desc_done[s]) (void)hipEventDestroy(h->desc_done[s]);
  if (h->A8) (void)hipFree(h->A8);
  if (h->B8) (void)hipFree(h->B8);
  if (h->C32) (void)hipFree(h->C32);
  if (h->row_shift) (void)hipFree(h->row_shift);
  if (h->col_shift) (void)hipFree(h->col_shift);
  if (h->d_desc) (void)hipFree(h->d_desc);
  if (h->h_desc) (void)hipHostFree(h->h_desc);
  delete[] h->plan;
  delete[] h->plan_memo;
  delete[] h->emu_idx;
  delete[] h->nat_idx;
  delete[] h->loop_info;
  reuse_arena_destroy(h->reuse);
  delete[] h->reuse_nmod;
  delete[] h->ua_off8;
  delete[] h->ua_offs;
  delete[] h->ub_off8;
  delete[] h->ub_offs;
  ::operator delete(h);
}

extern "C" int ggemm_create(ggemm_handle_t* out, int max_problems, size_t max_A, size_t max_B, size_t max_C,
                            hipStream_t stream) {
  return ggemm_create_ex(out, max_problems, max_A, max_B, max_C, stream, kKpAlign);
}

// src/ggemm.cu:228-341 sizing rules:
//   A8/B8 bytes = 21 planes x (ceil(max(2, kp_inflation(min_k)) max_elems) + 256 P)
//   C32 bytes   = 21 x (max_C + 64 P) x 4
//   shifts      = 4 x (rows an accepted call can have) + 64 P.  A call passing the A8 check has
//                 sum_g m_g <= min(max_A, 21 (A8 plane budget) / (3 x 32)) (N >= 2, kp >= 32),
//                 so this bound admits every call the reference's 4 max_A + 64 P sizing admits.
extern "C" int ggemm_create_ex(ggemm_handle_t* out, int max_problems, size_t max_A, size_t max_B, size_t max_C,
                               hipStream_t stream, int min_k) {
  if (!out || max_problems <= 0 || min_k < 1) return GGEMM_ERR_INVALID;
  *out = nullptr;
  void* mem = ::operator new(sizeof(ggemm_handle_s), std::nothrow);
  if (!mem) return GGEMM_ERR_ALLOC;
  std::memset(mem, 0, sizeof(ggemm_handle_s));
  ggemm_handle_t h = static_cast<ggemm_handle_t>(mem);
  h->stream = stream;
  h->max_problems = max_problems;
  h->max_A_elems = max_A;
  h->max_B_elems = max_B;
  h->max_C_elems = max_C;
  h->min_k = min_k;
  const size_t P = (size_t)max_problems;
  const size_t M = (size_t)kMaxPlanes;
#define FAIL(code) do { ggemm_destroy(h); return (code); } while (0)
#define HIPA(x) do { if ((x) != hipSuccess) FAIL(GGEMM_ERR_ALLOC); } while (0)
  hipDeviceProp_t prop;
  if (hipGetDevice(&h->device) != hipSuccess || hipGetDeviceProperties(&prop, h->device) != hipSuccess)
    FAIL(GGEMM_ERR_CUDA);
  h->num_cus = prop.multiProcessorCount;
  ggemm_device_model_init(&h->dm, prop.gcnArchName, prop.major, prop.minor, h->num_cus);
  if (oz2_init_constants() != 0) FAIL(GGEMM_ERR_NUMERICS);

  size_workspace(h, max_problems, max_A, max_B, max_C, min_k);
  HIPA(hipMalloc(&h->A8, h->A8_bytes));
  HIPA(hipMalloc(&h->B8, h->B8_bytes));
  HIPA(hipMalloc(&h->C32, h->C32_bytes));
  HIPA(hipMalloc(&h->row_shift, h->row_shift_elems * sizeof(int32_t)));
  HIPA(hipMalloc(&h->col_shift, h->col_shift_elems * sizeof(int32_t)));
  HIPA(hipMalloc(&h->d_desc, h->desc_bytes));
  HIPA(hipHostMalloc(&h->h_desc, h->desc_bytes * kSlots, hipHostMallocDefault));
  for (int s = 0; s < kSlots; ++s) {
    HIPA(hipEventCreateWithFlags(&h->desc_done[s], hipEventDisableTiming));
    HIPA(hipEventRecord(h->desc_done[s], stream));
  }
  h->plan = new (std::nothrow) ggemm_plan_entry_t[P];
  h->plan_memo_cap = ggemm_plan_memo_cap(max_problems);
  h->plan_memo = new (std::nothrow) int[h->plan_memo_cap];
  h->emu_idx = new (std::nothrow) int[P];
  h->nat_idx = new (std::nothrow) int[P];
  h->loop_info = new (std::nothrow) i8_sched_info[P * M];
  if (!h->plan || !h->plan_memo || !h->emu_idx || !h->nat_idx || !h->loop_info) FAIL(GGEMM_ERR_ALLOC);
  // the INT8 schedule builder's host scratch for P (problem, plane) products of every call
  // (src/ggemm.cu:287): calls through this handle allocate no host memory
  i8_reserve_host(P * M);
  // operand reuse: host arena and offset scratch (nothing is allocated inside calls)
  if (reuse_arena_create(max_problems, &h->reuse) != REUSE_OK) FAIL(h->reuse ? GGEMM_ERR_INVALID : GGEMM_ERR_ALLOC);
  h->reuse_nmod = new (std::nothrow) int[P];
  h->ua_off8 = new (std::nothrow) size_t[P];
  h->ua_offs = new (std::nothrow) size_t[P];
  h->ub_off8 = new (std::nothrow) size_t[P];
  h->ub_offs = new (std::nothrow) size_t[P];
  if (!h->reuse_nmod || !h->ua_off8 || !h->ua_offs || !h->ub_off8 || !h->ub_offs) FAIL(GGEMM_ERR_ALLOC);
  const char* ep = std::getenv("GGEMM_REUSE_PROMOTE");
  h->reuse_promote = (ep && std::atoi(ep) == 1) ? 1 : 0;
  const char* ec = std::getenv("GGEMM_DIGITS_COLMAJOR");
  h->digits_colmajor = (ec && std::atoi(ec) == 1) ? 1 : 0;
  const char* eg = std::getenv("GGEMM_I8_KERNEL");
  h->i8_mode = !eg ? 0 : !std::strcmp(eg, "general") ? 1 : !std::strcmp(eg, "large") ? 2 : 0;
  const char* et = std::getenv("GGEMM_F64_TILE");
  h->f64_tile = !et ? 0 : std::atoi(et) == 64 ? 64 : std::atoi(et) == 128 ? 128 : 0;
  const char* e = std::getenv("GGEMM_STATS_REPAIR");
  h->stats_repair = (e && std::atoi(e) == 1) ? 1 : 0;
  const char* esc = std::getenv("GGEMM_I8_SCHED");
  h->i8_persistent = (esc && !std::strcmp(esc, "persistent")) ? 1 : 0;
  const char* epk = std::getenv("GGEMM_PACKED_MAX_KP");
  h->packed_max_kp = epk ? std::max(0, std::atoi(epk)) : kPackedMaxKp;
  h->packed_env = epk ? 1 : 0;
  const char* esf = std::getenv("GGEMM_SAFETY_CHAINS");
  h->safety_chains = (esf && std::atoi(esf) == 1) ? 1 : 0;
  const char* ecp = std::getenv("GGEMM_COMPACT");
  h->compact = (ecp && std::atoi(ecp) == 0) ? 0 : 1;
  const char* edf = std::getenv("GGEMM_DOT_FORM");
  h->dot_form = !edf                          ? kDotFormAuto
                : !std::strcmp(edf, "dense")  ? kDotFormDense
                : !std::strcmp(edf, "blocks") ? kDotFormBlocks
                : !std::strcmp(edf, "list")   ? kDotFormList
                : !std::strcmp(edf, "tile")   ? kDotFormTile
                                              : kDotFormAuto;
  if (hipStreamSynchronize(stream) != hipSuccess) FAIL(GGEMM_ERR_CUDA);
#undef HIPA
#undef FAIL
  *out = h;
  return GGEMM_OK;
}

// src/ggemm.cu:698-741
extern "C" int ggemm_grouped_dgemm(ggemm_handle_t h, ggemm_path_t path, const ggemm_config_t* cfg,
                                   const ggemm_problem_t* problems, int num_problems, ggemm_stats_t* stats) {
  ggemm_stats_t local;
  ggemm_stats_t* st = stats ? stats : &local;
  std::memset(st, 0, sizeof(*st));
  st->num_problems = num_problems;
  st->num_repaired = st->num_uncertified = st->num_safety_fallback = -1;
  if (!h) return GGEMM_ERR_INVALID;
  int r = validate(h, problems, num_problems);
  if (r) return r;
  static const ggemm_config_t kDefault = {0, 1e-15, 1, 0};
  if (!cfg) cfg = &kDefault;
  if (cfg->num_moduli < 0 || cfg->num_moduli == 1 || cfg->num_moduli > GGEMM_MAX_MODULI) return GGEMM_ERR_INVALID;
  const int repair = repair_mode_of(path, cfg);
  if (repair < 0) return GGEMM_ERR_INVALID;
  switch (path) {
    case GGEMM_PATH_NATIVE_LOOP: return path_native(h, false, problems, num_problems, st);
    case GGEMM_PATH_NATIVE_GROUPED: return path_native(h, true, problems, num_problems, st);
    case GGEMM_PATH_EMU_LOOP:
    case GGEMM_PATH_EMU_GROUPED:
    case GGEMM_PATH_AUTO:
    case GGEMM_PATH_EMU_GROUPED_REUSE:
    case GGEMM_PATH_EMU_LOOP_BATCHED: {
      if ((r = counters_reset(h, h->stream))) return r;
      r = path_emu(h, path, cfg, problems, num_problems, st, repair);
      if (!r) r = counters_read(h, h->stream, st);
      return r;
    }
    default:
      return GGEMM_ERR_INVALID;
  }
}
