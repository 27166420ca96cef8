// planner.cpp -- per-problem route, moduli count and tile configuration (host only).
//
// Same decisions as the reference planner (src/planner.cpp:214-413), so that AUTO routes,
// fallback counts and moduli ranges agree on the same device model:
//   EMPTY (m or n == 0), K_ZERO, ALPHA_ZERO, K_TOO_LARGE (k > 131040, else ERR_UNSAFE without
//   fallback), AUTO: SMALL_K (k <= 16), N = choose_cw(k, rho) [AUTO adaptive] or the fixed /
//   target-driven N, PRECISION when no N reaches the target; AUTO only: tile by padding
//   efficiency, TINY (m n k below tiny_mnk) and UNPROFITABLE from the three-stage cost model,
//   then the wave-quantisation tile shrink and one re-costing.
// The cost model keeps the reference's constants (128/64/32 tiles with efficiencies 1/.63/.30,
// two resident tiles per compute unit, two prep passes) -- they define the routes being matched.
// The device model is keyed on the architecture name: gfx950 gets MI355X nominal peaks
// (FP64 78.6 TF, INT8 5.03 POPS, HBM 8 TB/s) times the reference's efficiency factors, unless a
// calibration JSON (env GGEMM_CALIB_JSON, or GGEMM_CALIB_DIR/params_<arch>.json) or the env
// overrides GGEMM_FP64_FLOPS / GGEMM_INT8_OPS / GGEMM_MEM_BW / GGEMM_TINY_MNK say otherwise.
#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <dlfcn.h>

#include "common.hpp"

namespace {

double env_pos(const char* name, double dflt) {
  const char* s = std::getenv(name);
  if (!s || !*s) return dflt;
  char* end = nullptr;
  const double v = std::strtod(s, &end);
  return (end != s && v > 0) ? v : dflt;
}

struct Range {
  const char* key;
  double lo, hi;
};
const Range kFP64 = {"fp64_flops", 1e11, 1e16};
const Range kI8 = {"int8_ops", 1e12, 1e17};
const Range kBW = {"mem_bw", 1e10, 1e14};

bool in_range(const Range& r, double v, const char* src) {
  if (v >= r.lo && v <= r.hi) return true;
  std::fprintf(stderr, "[ggemm] WARNING: %s %s=%g outside [%g, %g], ignored\n", src, r.key, v, r.lo, r.hi);
  return false;
}
bool env_in_range(const char* name, const Range& r, double* v) {
  const char* s = std::getenv(name);
  if (!s || !*s) return false;
  char* end = nullptr;
  const double x = std::strtod(s, &end);
  if (end == s || !in_range(r, x, name)) return false;
  *v = x;
  return true;
}
// "key": number, anywhere in the text
bool json_number(const char* txt, const char* key, double* v) {
  char pat[96];
  std::snprintf(pat, sizeof pat, "\"%s\"", key);
  const char* p = std::strstr(txt, pat);
  if (!p) return false;
  p = std::strchr(p + std::strlen(pat), ':');
  if (!p) return false;
  char* end = nullptr;
  const double x = std::strtod(p + 1, &end);
  if (end == p + 1 || !(x > 0)) return false;
  *v = x;
  return true;
}
// Architecture slug: leading alphanumerics of the name ("gfx950:sramecc+:xnack-" -> "gfx950"),
// else lower-cased alphanumeric runs joined by '_'.
void slug_of(const char* name, char* out, size_t cap) {
  size_t n = 0;
  bool sep = false;
  for (const char* c = name ? name : ""; *c && n + 1 < cap; ++c) {
    if (*c == ':') break;
    if (std::isalnum((unsigned char)*c)) {
      if (sep && n) out[n++] = '_';
      sep = false;
      out[n++] = (char)std::tolower((unsigned char)*c);
    } else {
      sep = true;
    }
  }
  out[n] = 0;
}

void load_calib(const char* gpu_name, double* fp64, double* i8, double* bw, char* used, size_t used_sz, bool* got) {
  char path[1024];
  const char* env = std::getenv("GGEMM_CALIB_JSON");
  if (env && *env) {
    std::snprintf(path, sizeof path, "%s", env);
  } else {
    // GGEMM_CALIB_DIR, else the calib/ directory beside this library's ggemm/ directory (the
    // reference compiles its calibration directory in, src/planner.cpp:62-78)
    char dir[1024];
    const char* env_dir = std::getenv("GGEMM_CALIB_DIR");
    if (env_dir && *env_dir) {
      std::snprintf(dir, sizeof dir, "%s", env_dir);
    } else {
      Dl_info info;
      if (!dladdr(reinterpret_cast<void*>(&ggemm_device_model_init), &info) || !info.dli_fname) return;
      std::snprintf(dir, sizeof dir, "%s", info.dli_fname);
      char* slash = std::strrchr(dir, '/');
      if (!slash) return;
      std::snprintf(slash, sizeof dir - (size_t)(slash - dir), "/../calib");
    }
    char slug[256];
    slug_of(gpu_name, slug, sizeof slug);
    std::snprintf(path, sizeof path, "%s/params_%s.json", dir, slug);
  }
  FILE* f = std::fopen(path, "rb");
  if (!f) return;
  static char buf[1 << 16];
  const size_t n = std::fread(buf, 1, sizeof buf - 1, f);
  buf[n] = 0;
  std::fclose(f);
  double v;
  if (json_number(buf, "f64_peak_flops", &v) && in_range(kFP64, v, path)) { *fp64 = v; got[0] = true; }
  if (json_number(buf, "i8_peak_ops", &v) && in_range(kI8, v, path)) { *i8 = v; got[1] = true; }
  if (json_number(buf, "bw_Bps", &v) && in_range(kBW, v, path)) { *bw = v; got[2] = true; }
  if (used) std::snprintf(used, used_sz, "%s", path);
}

inline int tile_dim(int cfg) { return cfg == 0 ? 128 : (cfg == 1 ? 64 : 32); }
inline size_t kp_of(int k) { return ggemm::align_up((size_t)k, ggemm::kKpAlign); }
inline double rup(double x, double q) { return std::ceil(x / q) * q; }

int tile_by_padding(int m, int n) {
  int best = 2;
  double best_eff = -1;
  for (int c = 0; c < 3; ++c) {
    const double t = tile_dim(c);
    const double eff = (double)m * n / (rup(m, t) * rup(n, t));
    if (eff >= 0.75) return c;
    if (eff > best_eff) { best_eff = eff; best = c; }
  }
  return best;
}
double tiles_of(int m, int n, int cfg) {
  const double t = tile_dim(cfg);
  return std::ceil(m / t) * std::ceil(n / t);
}

constexpr double kPrepPasses = 2.0;
constexpr double kTileEff[3] = {1.0, 0.63, 0.30};
constexpr int kResidentTiles = 2;   // per compute unit, in the cost model

void cost(const ggemm_problem_t& p, int nm, int cfg, const ggemm_device_model_t* dm, double* t_emu, double* t_nat) {
  const double m = p.m, n = p.n, k = p.k, kp = (double)kp_of(p.k), t = tile_dim(cfg);
  const double c_rw = (p.beta != 0.0) ? 2.0 : 1.0;
  const double np = nm + OZ2_EXTRA_PLANES;
  const double prep = (kPrepPasses * (m * k + k * n) * 8 + np * (m + n) * kp + 4.0 * OZ2_ROW_WS_PER_ROW * (m + n)) /
                      dm->mem_bw;
  const double slots = (double)dm->num_sms * kResidentTiles;
  const double per_tile = 2.0 * t * t * kp / (dm->int8_ops * kTileEff[cfg] / slots);
  const double gemm = std::ceil(np * tiles_of(p.m, p.n, cfg) / slots) * per_tile + np * m * n * 4 / dm->mem_bw;
  const double recon = (np * m * n * 4 + c_rw * m * n * 8) / dm->mem_bw;
  *t_emu = prep + gemm + recon;
  const double nat_c = 2.0 * m * n * k / dm->fp64_flops;
  const double nat_m = (m * k + k * n + c_rw * m * n) * 8 / dm->mem_bw;
  *t_nat = std::max(nat_c, nat_m);
}

bool tune_tiles(const ggemm_problem_t* probs, int num, const ggemm_device_model_t* dm, ggemm_plan_entry_t* out) {
  const double slots = (double)dm->num_sms * kResidentTiles;
  bool any = false;
  for (int pass = 0; pass < 3; ++pass) {
    double W = 0;
    for (int g = 0; g < num; ++g) {
      if (out[g].route != GGEMM_ROUTE_EMU) continue;
      const double t = tile_dim(out[g].tile_cfg);
      W += (out[g].num_moduli + OZ2_EXTRA_PLANES) * tiles_of(probs[g].m, probs[g].n, out[g].tile_cfg) * t * t *
           (double)kp_of(probs[g].k);
    }
    if (W <= 0) return any;
    const double per_slot = W / slots;
    bool changed = false;
    for (int g = 0; g < num; ++g) {
      if (out[g].route != GGEMM_ROUTE_EMU || out[g].tile_cfg >= 2) continue;
      const double t = tile_dim(out[g].tile_cfg);
      if (t * t * (double)kp_of(probs[g].k) > per_slot) { out[g].tile_cfg++; changed = true; }
    }
    if (!changed) return any;
    any = true;
  }
  return any;
}

int plan_shape(const ggemm_problem_t& p, const ggemm_config_t* cfg, bool autop, int allow_fb, double rho,
               const ggemm_device_model_t* dm, ggemm_plan_entry_t& e) {
  if (p.k > GGEMM_MAX_K_EXACT) {
    if (!allow_fb) return GGEMM_ERR_UNSAFE;
    e.route = GGEMM_ROUTE_K_TOO_LARGE;
    return GGEMM_OK;
  }
  if (autop && allow_fb && p.k <= GGEMM_AUTO_NATIVE_MAX_K) {
    e.route = GGEMM_ROUTE_SMALL_K;
    return GGEMM_OK;
  }
  if (autop && !(cfg && cfg->num_moduli > 0)) {
    e.num_moduli = oz2_choose_num_moduli_cw(p.k, rho);
    if (e.num_moduli >= 0) e.num_moduli = std::min(std::max(e.num_moduli, 2), GGEMM_MAX_MODULI);
  } else {
    e.num_moduli = ggemm_plan_num_moduli(cfg, p.k);
  }
  if (e.num_moduli < 0) {
    if (!allow_fb) return GGEMM_ERR_UNSAFE;
    e.route = GGEMM_ROUTE_PRECISION;
    e.num_moduli = 0;
    return GGEMM_OK;
  }
  if (!autop) return GGEMM_OK;
  e.tile_cfg = tile_by_padding(p.m, p.n);
  cost(p, e.num_moduli, e.tile_cfg, dm, &e.t_emu_s, &e.t_native_s);
  if (allow_fb) {
    if ((double)p.m * p.n * p.k < dm->tiny_mnk) e.route = GGEMM_ROUTE_TINY;
    else if (e.t_emu_s > e.t_native_s) e.route = GGEMM_ROUTE_UNPROFITABLE;
  }
  return GGEMM_OK;
}

// The planner reads a problem only through (m, n, k, beta != 0) past the alpha == 0 check.
bool same_shape(const ggemm_problem_t& a, const ggemm_problem_t& b) {
  return a.m == b.m && a.n == b.n && a.k == b.k && (a.beta != 0.0) == (b.beta != 0.0);
}
uint32_t shape_hash(const ggemm_problem_t& p) {
  uint64_t h = 0x9E3779B97F4A7C15ull;
  const uint64_t parts[4] = {(uint64_t)(uint32_t)p.m, (uint64_t)(uint32_t)p.n, (uint64_t)(uint32_t)p.k,
                             (uint64_t)(p.beta != 0.0)};
  for (uint64_t x : parts) {
    h ^= x + 0x9E3779B97F4A7C15ull + (h << 6) + (h >> 2);
    h *= 0xBF58476D1CE4E5B9ull;
  }
  return (uint32_t)(h ^ (h >> 32));
}

}  // namespace

extern "C" void ggemm_device_model_init(ggemm_device_model_t* dm, const char* gpu_name, int cc_major, int cc_minor,
                                        int num_sms) {
  (void)cc_major;
  (void)cc_minor;
  double fp64, i8, bw;
  const bool mi355 = gpu_name && (std::strstr(gpu_name, "gfx950") || std::strstr(gpu_name, "MI355"));
  if (mi355) {   // MI355X nominal: FP64 MFMA 78.6 TF, INT8 dense 5.03 POPS, HBM3E 8 TB/s
    fp64 = 78.6e12 * 0.8;
    i8 = 5.03e15 * 0.5;
    bw = 8.0e12 * 0.8;
  } else {       // unknown device: conservative guess, calibrate via env / JSON
    fp64 = 10e12;
    i8 = 200e12;
    bw = 1e12;
  }
  char used[1024] = "none";
  bool got[3] = {false, false, false};
  load_calib(gpu_name, &fp64, &i8, &bw, used, sizeof used, got);
  const char* src[4];
  for (int i = 0; i < 3; ++i) src[i] = got[i] ? "json" : "nominal";
  if (env_in_range("GGEMM_FP64_FLOPS", kFP64, &fp64)) src[0] = "env";
  if (env_in_range("GGEMM_INT8_OPS", kI8, &i8)) src[1] = "env";
  if (env_in_range("GGEMM_MEM_BW", kBW, &bw)) src[2] = "env";
  dm->num_sms = num_sms > 0 ? num_sms : 1;
  dm->fp64_flops = fp64;
  dm->int8_ops = i8;
  dm->mem_bw = bw;
  dm->tiny_mnk = 32.0 * 32.0 * 32.0;
  src[3] = "default";
  if (const char* s = std::getenv("GGEMM_TINY_MNK")) {   // 0 disables the TINY route
    char* end = nullptr;
    const double v = std::strtod(s, &end);
    if (end != s && v >= 0) { dm->tiny_mnk = v; src[3] = "env"; }
  }
  static bool printed = false;
  if (!printed) {
    printed = true;
    std::fprintf(stderr, "[ggemm] calib fp64_flops=%.3g(%s) int8_ops=%.3g(%s) mem_bw=%.3g(%s) tiny_mnk=%.3g(%s) json=%s\n",
                 fp64, src[0], i8, src[1], bw, src[2], dm->tiny_mnk, src[3], used);
  }
}

// Normwise target: |C_ij - (AB)_ij| <= target ||A(i,:)|| ||B(:,j)||, bounded by oz2_error_bound.
extern "C" int ggemm_plan_num_moduli(const ggemm_config_t* cfg, int k) {
  int nm;
  if (cfg && cfg->num_moduli > 0) {
    nm = cfg->num_moduli;
  } else {
    const double tgt = (cfg && cfg->target_rel_err > 0) ? cfg->target_rel_err : 1e-15;
    nm = oz2_choose_num_moduli(k, tgt);
    if (nm < 0) return -1;   // unreachable target: never clamp (the caller falls back / fails)
  }
  return std::min(std::max(nm, 2), GGEMM_MAX_MODULI);
}

extern "C" size_t ggemm_plan_memo_cap(int num) {
  size_t cap = 1;
  while (cap < 2 * (size_t)std::max(num, 1)) cap <<= 1;
  return cap;
}

extern "C" int ggemm_plan_ex(const ggemm_problem_t* probs, int num, const ggemm_config_t* cfg, ggemm_path_t path,
                             const ggemm_device_model_t* dm, ggemm_plan_entry_t* out, int* memo, size_t memo_cap) {
  const int allow_fb = cfg ? cfg->allow_fallback : 0;
  const bool autop = (path == GGEMM_PATH_AUTO);
  static const double rho = env_pos("GGEMM_RHO_BUDGET", GGEMM_RHO_BUDGET_DEFAULT);
  size_t mask = 0;
  if (memo && num > 0) {
    const size_t cap = ggemm_plan_memo_cap(num);
    if (cap <= memo_cap) {
      std::fill(memo, memo + cap, -1);
      mask = cap - 1;
    } else {
      memo = nullptr;
    }
  }
  for (int g = 0; g < num; ++g) {
    const ggemm_problem_t& p = probs[g];
    ggemm_plan_entry_t& e = out[g];
    e.route = GGEMM_ROUTE_EMU;
    e.num_moduli = 0;
    e.tile_cfg = 0;
    e.t_emu_s = e.t_native_s = 0;
    if (p.m == 0 || p.n == 0) { e.route = GGEMM_ROUTE_EMPTY; continue; }
    if (p.k == 0) { e.route = GGEMM_ROUTE_K_ZERO; continue; }
    if (p.alpha == 0.0) { e.route = GGEMM_ROUTE_ALPHA_ZERO; continue; }
    if (memo) {
      size_t s = shape_hash(p) & mask;
      int rep;
      while ((rep = memo[s]) >= 0 && !same_shape(probs[rep], p)) s = (s + 1) & mask;
      if (rep >= 0) { e = out[rep]; continue; }
      memo[s] = g;
    }
    const int r = plan_shape(p, cfg, autop, allow_fb, rho, dm, e);
    if (r) return r;
  }
  if (autop && tune_tiles(probs, num, dm, out)) {
    for (int g = 0; g < num; ++g) {
      ggemm_plan_entry_t& e = out[g];
      if (e.route != GGEMM_ROUTE_EMU) continue;
      cost(probs[g], e.num_moduli, e.tile_cfg, dm, &e.t_emu_s, &e.t_native_s);
      if (allow_fb && e.t_emu_s > e.t_native_s) e.route = GGEMM_ROUTE_UNPROFITABLE;
    }
  }
  return GGEMM_OK;
}

extern "C" int ggemm_plan(const ggemm_problem_t* probs, int num, const ggemm_config_t* cfg, ggemm_path_t path,
                          const ggemm_device_model_t* dm, ggemm_plan_entry_t* out) {
  return ggemm_plan_ex(probs, num, cfg, path, dm, out, nullptr, 0);
}
