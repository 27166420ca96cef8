// planner.cpp -- per-problem route, moduli count and tile configuration (host only).
//
// The routing rules are the reference planner's (src/planner.cpp:137-330), kept so that AUTO
// routes, fallback counts and moduli ranges agree on the same device model:
//   EMPTY (m or n == 0), K_ZERO, ALPHA_ZERO, K_TOO_LARGE (k > 131040; ERR_UNSAFE without
//   fallback), AUTO: SMALL_K (k <= 16), N = choose_cw(k, rho) [AUTO adaptive] or the fixed /
//   target-driven N, PRECISION when no N reaches the target; AUTO only: tile by padding
//   efficiency, TINY (m n k below tiny_mnk) and UNPROFITABLE from the three-stage cost model,
//   then the wave-quantisation tile shrink and one re-costing.
// The cost model keeps the reference's constants (128/64/32 tiles with efficiencies 1/.63/.30,
// two resident tiles per compute unit, two prep passes) and its operation order, so the cost
// doubles are the reference's to the last bit.
//
// Device model: nominal figures for the architecture (gfx950: MI355X FP64 78.6 TF, INT8 5.03 POPS,
// HBM 8 TB/s, times the reference's efficiency factors), then a calibration file in the
// reference's params schema, then per-quantity environment overrides; every figure outside its
// plausible range is ignored with a warning.
#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <dlfcn.h>

#include "common.hpp"

namespace {

// ------------------------------------------------------------------------- device model
enum Quantity { kQFp64 = 0, kQInt8 = 1, kQBw = 2, kNumQuantities = 3 };
struct QuantitySpec {
  const char* file_key;   // key in the calibration file
  const char* env;        // overriding environment variable
  const char* label;      // name in messages
  double lo, hi;          // plausible range (FLOP/s, OP/s, B/s)
};
constexpr QuantitySpec kQuantities[kNumQuantities] = {
    {"f64_peak_flops", "GGEMM_FP64_FLOPS", "fp64_flops", 1e11, 1e16},
    {"i8_peak_ops", "GGEMM_INT8_OPS", "int8_ops", 1e12, 1e17},
    {"bw_Bps", "GGEMM_MEM_BW", "mem_bw", 1e10, 1e14},
};

bool plausible(const QuantitySpec& q, double v, const char* origin) {
  if (v >= q.lo && v <= q.hi) return true;
  std::fprintf(stderr, "[ggemm] WARNING: %s %s=%g outside [%g, %g], ignored\n", origin, q.label, v, q.lo, q.hi);
  return false;
}

// The numeric members at the top level of a JSON object ("key": number), found by walking the text
// with a nesting depth: members of nested objects / arrays and string contents are skipped.
class TopLevelNumbers {
 public:
  explicit TopLevelNumbers(const char* text) : text_(text) {}
  // true and *v when the key is a top-level member whose value is a number
  bool get(const char* key, double* v) const {
    const size_t klen = std::strlen(key);
    int depth = 0;
    for (const char* p = text_; *p; ++p) {
      if (*p == '{' || *p == '[') { ++depth; continue; }
      if (*p == '}' || *p == ']') { --depth; continue; }
      if (*p != '"') continue;
      const char* s = p + 1;
      const char* e = s;
      while (*e && *e != '"') e += (*e == '\\' && e[1]) ? 2 : 1;
      if (!*e) return false;
      p = e;   // the loop's ++p moves past the closing quote
      if (depth != 1 || (size_t)(e - s) != klen || std::strncmp(s, key, klen) != 0) continue;
      const char* c = e + 1;
      while (std::isspace((unsigned char)*c)) ++c;
      if (*c != ':') continue;   // a string value equal to the key, not a member name
      char* end = nullptr;
      const double x = std::strtod(c + 1, &end);
      if (end == c + 1) return false;
      *v = x;
      return true;
    }
    return false;
  }

 private:
  const char* text_;
};

// Architecture slug of a device name: its leading alphanumerics up to a ':' ("gfx950:sramecc+:xnack-"
// -> "gfx950"); other characters separate lower-cased alphanumeric runs joined by '_'.
void arch_slug(const char* name, char* out, size_t cap) {
  size_t n = 0;
  bool pending_sep = false;
  for (const char* c = name ? name : ""; *c && *c != ':' && n + 1 < cap; ++c) {
    const unsigned char ch = (unsigned char)*c;
    if (!std::isalnum(ch)) { pending_sep = n > 0; continue; }
    if (pending_sep && n + 2 < cap) out[n++] = '_';
    pending_sep = false;
    out[n++] = (char)std::tolower(ch);
  }
  out[n] = 0;
}

// Calibration file path: GGEMM_CALIB_JSON, else params_<slug>.json in GGEMM_CALIB_DIR or in the
// calib/ directory beside the directory of this library (the reference compiles its calibration
// directory in).  False when no path can be formed.
bool calib_path(const char* gpu_name, char* path, size_t cap) {
  if (const char* f = std::getenv("GGEMM_CALIB_JSON"); f && *f) {
    std::snprintf(path, cap, "%s", f);
    return true;
  }
  char dir[1024];
  if (const char* d = std::getenv("GGEMM_CALIB_DIR"); d && *d) {
    std::snprintf(dir, sizeof dir, "%s", d);
  } else {
    Dl_info info;
    if (!dladdr(reinterpret_cast<void*>(&ggemm_device_model_init), &info) || !info.dli_fname) return false;
    const char* slash = std::strrchr(info.dli_fname, '/');
    if (!slash) return false;
    std::snprintf(dir, sizeof dir, "%.*s/../calib", (int)(slash - info.dli_fname), info.dli_fname);
  }
  char slug[128];
  arch_slug(gpu_name, slug, sizeof slug);
  std::snprintf(path, cap, "%s/params_%s.json", dir, slug);
  return true;
}

// Reads the file's quantities into v[] (positive, plausible values only); returns whether the file
// was read, origin[q] = "json" for each quantity taken from it.
bool apply_calib_file(const char* path, double* v, const char** origin) {
  FILE* f = std::fopen(path, "rb");
  if (!f) return false;
  static char text[1 << 16];   // the scalars sit at the top of the file
  const size_t len = std::fread(text, 1, sizeof text - 1, f);
  std::fclose(f);
  text[len] = 0;
  const TopLevelNumbers doc(text);
  for (int q = 0; q < kNumQuantities; ++q) {
    double x;
    if (doc.get(kQuantities[q].file_key, &x) && x > 0 && plausible(kQuantities[q], x, path)) {
      v[q] = x;
      origin[q] = "json";
    }
  }
  return true;
}

// ------------------------------------------------------------------------- planning
constexpr int kNumTiles = 3;
constexpr double kTileEff[kNumTiles] = {1.0, 0.63, 0.30};   // relative INT8 rate of tiles 128 / 64 / 32
constexpr double kPrepPasses = 2.0;                          // prep reads A and B twice
constexpr double kTilesPerCu = 2.0;                          // resident tiles per compute unit
inline double tile_edge(int cfg) { return cfg == 0 ? 128.0 : (cfg == 1 ? 64.0 : 32.0); }
inline double padded_kp(int k) { return (double)ggemm::kp_of(k); }
inline double tile_count(int m, int n, int cfg) {
  const double t = tile_edge(cfg);
  return std::ceil(m / t) * std::ceil(n / t);
}

struct Costs {
  double emu, native;
};

class Planner {
 public:
  Planner(const ggemm_config_t* cfg, ggemm_path_t path, const ggemm_device_model_t* dm, double rho)
      : cfg_(cfg), dm_(dm), rho_(rho), auto_(path == GGEMM_PATH_AUTO), fallback_(cfg ? cfg->allow_fallback : 0),
        slots_((double)dm->num_sms * kTilesPerCu) {}

  // Route, N, tile and costs of one problem past the EMPTY / K_ZERO / ALPHA_ZERO checks; e enters
  // as route EMU with zeroed fields.  Depends on p only through (m, n, k, beta != 0).
  int plan_one(const ggemm_problem_t& p, ggemm_plan_entry_t& e) const {
    if (p.k > GGEMM_MAX_K_EXACT) {
      if (!fallback_) return GGEMM_ERR_UNSAFE;
      e.route = GGEMM_ROUTE_K_TOO_LARGE;
      return GGEMM_OK;
    }
    if (auto_ && fallback_ && p.k <= GGEMM_AUTO_NATIVE_MAX_K) {
      e.route = GGEMM_ROUTE_SMALL_K;
      return GGEMM_OK;
    }
    e.num_moduli = moduli_for(p.k);
    if (e.num_moduli < 0) {
      if (!fallback_) return GGEMM_ERR_UNSAFE;
      e.route = GGEMM_ROUTE_PRECISION;
      e.num_moduli = 0;
      return GGEMM_OK;
    }
    if (!auto_) return GGEMM_OK;   // emulated paths: tile 0, no cost-based fallback
    e.tile_cfg = tile_for_padding(p.m, p.n);
    price(p, e);
    if (fallback_) {
      if ((double)p.m * p.n * p.k < dm_->tiny_mnk) e.route = GGEMM_ROUTE_TINY;
      else if (e.t_emu_s > e.t_native_s) e.route = GGEMM_ROUTE_UNPROFITABLE;
    }
    return GGEMM_OK;
  }

  // Wave quantisation over the whole group: a tile heavier than the average work per resident
  // slot shrinks one step; repeated until stable.  True if any tile changed.
  bool shrink_tiles(const ggemm_problem_t* probs, int num, ggemm_plan_entry_t* out) const {
    bool changed_any = false;
    for (int round = 0; round < kNumTiles; ++round) {
      double work = 0;
      for (int g = 0; g < num; ++g) {
        if (out[g].route != GGEMM_ROUTE_EMU) continue;
        const double t = tile_edge(out[g].tile_cfg);
        work += planes(out[g].num_moduli) * tile_count(probs[g].m, probs[g].n, out[g].tile_cfg) * t * t *
                padded_kp(probs[g].k);
      }
      if (work <= 0) return changed_any;
      const double per_slot = work / slots_;
      bool changed = false;
      for (int g = 0; g < num; ++g) {
        ggemm_plan_entry_t& e = out[g];
        if (e.route != GGEMM_ROUTE_EMU || e.tile_cfg >= kNumTiles - 1) continue;
        const double t = tile_edge(e.tile_cfg);
        if (t * t * padded_kp(probs[g].k) > per_slot) {
          ++e.tile_cfg;
          changed = true;
        }
      }
      if (!changed) return changed_any;
      changed_any = true;
    }
    return changed_any;
  }

  // After a tile shrink: new costs, and the profitability route once more.
  void reprice(const ggemm_problem_t* probs, int num, ggemm_plan_entry_t* out) const {
    for (int g = 0; g < num; ++g) {
      ggemm_plan_entry_t& e = out[g];
      if (e.route != GGEMM_ROUTE_EMU) continue;
      price(probs[g], e);
      if (fallback_ && e.t_emu_s > e.t_native_s) e.route = GGEMM_ROUTE_UNPROFITABLE;
    }
  }

  bool is_auto() const { return auto_; }

 private:
  static double planes(int nm) { return (double)(nm + OZ2_EXTRA_PLANES); }

  int moduli_for(int k) const {
    if (auto_ && !(cfg_ && cfg_->num_moduli > 0)) {   // AUTO adaptive: componentwise budget
      const int nm = oz2_choose_num_moduli_cw(k, rho_);
      return nm < 0 ? nm : std::min(std::max(nm, 2), GGEMM_MAX_MODULI);
    }
    return ggemm_plan_num_moduli(cfg_, k);
  }

  // The largest tile whose padded area is at least 3/4 useful, else the least padded one.
  static int tile_for_padding(int m, int n) {
    int best = kNumTiles - 1;
    double best_fill = -1;
    for (int c = 0; c < kNumTiles; ++c) {
      const double t = tile_edge(c);
      const double fill = (double)m * n / (std::ceil(m / t) * t * (std::ceil(n / t) * t));
      if (fill >= 0.75) return c;
      if (fill > best_fill) {
        best_fill = fill;
        best = c;
      }
    }
    return best;
  }

  // Three dependent stages (prep, INT8 GEMM with its C32 write, reconstruct) against the native
  // FP64 GEMM's compute / memory bound; byte terms as in the reference's calibration fit.
  void price(const ggemm_problem_t& p, ggemm_plan_entry_t& e) const {
    const Costs c = costs(p, e.num_moduli, e.tile_cfg);
    e.t_emu_s = c.emu;
    e.t_native_s = c.native;
  }
  Costs costs(const ggemm_problem_t& p, int nm, int cfg) const {
    const double m = p.m, n = p.n, k = p.k, kp = padded_kp(p.k), t = tile_edge(cfg);
    const double c_rw = p.beta != 0.0 ? 2.0 : 1.0;
    const double np = planes(nm);
    const double bw = dm_->mem_bw;
    const double prep_s =
        (kPrepPasses * (m * k + k * n) * 8 + np * (m + n) * kp + 4.0 * OZ2_ROW_WS_PER_ROW * (m + n)) / bw;
    const double tile_s = 2.0 * t * t * kp / (dm_->int8_ops * kTileEff[cfg] / slots_);
    const double gemm_s = std::ceil(np * tile_count(p.m, p.n, cfg) / slots_) * tile_s + np * m * n * 4 / bw;
    const double recon_s = (np * m * n * 4 + c_rw * m * n * 8) / bw;
    const double native_flop_s = 2.0 * m * n * k / dm_->fp64_flops;
    const double native_mem_s = (m * k + k * n + c_rw * m * n) * 8 / bw;
    return Costs{prep_s + gemm_s + recon_s, std::max(native_flop_s, native_mem_s)};
  }

  const ggemm_config_t* cfg_;
  const ggemm_device_model_t* dm_;
  double rho_;
  bool auto_;
  int fallback_;
  double slots_;
};

// Shape memo: open addressing over problem indices keyed by (m, n, k, beta != 0), the only
// problem fields the planner reads past the alpha == 0 check.
bool same_key(const ggemm_problem_t& a, const ggemm_problem_t& b) {
  return a.m == b.m && a.n == b.n && a.k == b.k && (a.beta != 0.0) == (b.beta != 0.0);
}
uint32_t key_hash(const ggemm_problem_t& p) {
  uint64_t h = 0x9E3779B97F4A7C15ull;
  const uint64_t parts[4] = {(uint64_t)(uint32_t)p.m, (uint64_t)(uint32_t)p.n, (uint64_t)(uint32_t)p.k,
                             (uint64_t)(p.beta != 0.0)};
  for (uint64_t x : parts) {
    h ^= x + 0x9E3779B97F4A7C15ull + (h << 6) + (h >> 2);
    h *= 0xBF58476D1CE4E5B9ull;
  }
  return (uint32_t)(h ^ (h >> 32));
}

double rho_budget() {
  const char* s = std::getenv("GGEMM_RHO_BUDGET");
  if (!s || !*s) return GGEMM_RHO_BUDGET_DEFAULT;
  char* end = nullptr;
  const double v = std::strtod(s, &end);
  return (end != s && v > 0) ? v : GGEMM_RHO_BUDGET_DEFAULT;
}

}  // namespace

extern "C" void ggemm_device_model_init(ggemm_device_model_t* dm, const char* gpu_name, int cc_major, int cc_minor,
                                        int num_sms) {
  (void)cc_major;   // HIP reports gfx9 parts as major 9: the architecture name decides
  (void)cc_minor;
  double v[kNumQuantities];
  const bool mi355 = gpu_name && (std::strstr(gpu_name, "gfx950") || std::strstr(gpu_name, "MI355"));
  if (mi355) {   // MI355X nominal: FP64 MFMA 78.6 TF, INT8 dense 5.03 POPS, HBM3E 8 TB/s
    v[kQFp64] = 78.6e12 * 0.8;
    v[kQInt8] = 5.03e15 * 0.5;
    v[kQBw] = 8.0e12 * 0.8;
  } else {       // unknown device: conservative guesses (calibrate through a file or the environment)
    v[kQFp64] = 10e12;
    v[kQInt8] = 200e12;
    v[kQBw] = 1e12;
  }
  const char* origin[kNumQuantities] = {"nominal", "nominal", "nominal"};
  char path[1024] = "none";
  char tried[1024];
  if (calib_path(gpu_name, tried, sizeof tried) && apply_calib_file(tried, v, origin))
    std::snprintf(path, sizeof path, "%s", tried);
  for (int q = 0; q < kNumQuantities; ++q) {
    const char* s = std::getenv(kQuantities[q].env);
    if (!s || !*s) continue;
    char* end = nullptr;
    const double x = std::strtod(s, &end);
    if (end != s && plausible(kQuantities[q], x, kQuantities[q].env)) {
      v[q] = x;
      origin[q] = "env";
    }
  }
  dm->num_sms = num_sms > 0 ? num_sms : 1;
  dm->fp64_flops = v[kQFp64];
  dm->int8_ops = v[kQInt8];
  dm->mem_bw = v[kQBw];
  dm->tiny_mnk = 32.0 * 32.0 * 32.0;
  const char* tiny_origin = "default";
  if (const char* s = std::getenv("GGEMM_TINY_MNK")) {   // 0 disables the TINY route
    char* end = nullptr;
    const double x = std::strtod(s, &end);
    if (end != s && x >= 0) {
      dm->tiny_mnk = x;
      tiny_origin = "env";
    }
  }
  static bool reported = false;   // one line per process
  if (!reported) {
    reported = true;
    std::fprintf(stderr, "[ggemm] calib fp64_flops=%.3g(%s) int8_ops=%.3g(%s) mem_bw=%.3g(%s) tiny_mnk=%.3g(%s) json=%s\n",
                 dm->fp64_flops, origin[kQFp64], dm->int8_ops, origin[kQInt8], dm->mem_bw, origin[kQBw], dm->tiny_mnk,
                 tiny_origin, path);
  }
}

// Normwise target: |C_ij - (AB)_ij| <= target ||A(i,:)|| ||B(:,j)||, bounded by oz2_error_bound.
// An unreachable target gives -1 (never a clamped N): the caller falls back or fails.
extern "C" int ggemm_plan_num_moduli(const ggemm_config_t* cfg, int k) {
  int nm = cfg && cfg->num_moduli > 0 ? cfg->num_moduli : 0;
  if (nm == 0) {
    nm = oz2_choose_num_moduli(k, (cfg && cfg->target_rel_err > 0) ? cfg->target_rel_err : 1e-15);
    if (nm < 0) return -1;
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
  static const double rho = rho_budget();   // read once per process
  const Planner planner(cfg, path, dm, rho);
  size_t mask = 0;
  if (memo && num > 0) {   // caller-owned table (sized at handle creation): no allocation here
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
    e = ggemm_plan_entry_t{GGEMM_ROUTE_EMU, 0, 0, 0.0, 0.0};
    if (p.m == 0 || p.n == 0) { e.route = GGEMM_ROUTE_EMPTY; continue; }
    if (p.k == 0) { e.route = GGEMM_ROUTE_K_ZERO; continue; }
    if (p.alpha == 0.0) { e.route = GGEMM_ROUTE_ALPHA_ZERO; continue; }   // C = beta C, nothing read
    if (memo) {
      size_t slot = key_hash(p) & mask;
      int first;
      while ((first = memo[slot]) >= 0 && !same_key(probs[first], p)) slot = (slot + 1) & mask;
      if (first >= 0) { e = out[first]; continue; }   // first < g: its entry is final
      memo[slot] = g;
    }
    const int r = planner.plan_one(p, e);
    if (r) return r;
  }
  if (planner.is_auto() && planner.shrink_tiles(probs, num, out)) planner.reprice(probs, num, out);
  return GGEMM_OK;
}

extern "C" int ggemm_plan(const ggemm_problem_t* probs, int num, const ggemm_config_t* cfg, ggemm_path_t path,
                          const ggemm_device_model_t* dm, ggemm_plan_entry_t* out) {
  return ggemm_plan_ex(probs, num, cfg, path, dm, out, nullptr, 0);
}
