// app_util.hpp -- shared pieces of the FP64 application benchmarks (moe_ffn, block_sparse): the
// downstream consumers of the C ABI (include/ggemm.h), counterparts of the reference's
// bench/app/app_common.h.  Every GEMM goes through ggemm_grouped_dgemm; no other GEMM library.
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "ggemm.h"

#define APP_HIP(x)                                                                              \
  do {                                                                                          \
    hipError_t e_ = (x);                                                                        \
    if (e_ != hipSuccess) {                                                                     \
      std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
      std::exit(1);                                                                             \
    }                                                                                           \
  } while (0)

namespace app {

inline double median(std::vector<double> v) {
  if (v.empty()) return NAN;
  std::sort(v.begin(), v.end());
  const size_t n = v.size();
  return n % 2 ? v[n / 2] : 0.5 * (v[n / 2 - 1] + v[n / 2]);
}
inline double mean(const std::vector<double>& v) {
  if (v.empty()) return NAN;
  double s = 0;
  for (double x : v) s += x;
  return s / (double)v.size();
}
// gamma_n = n u / (1 - n u), u = 2^-53: the FP64 a-priori componentwise bound factor
inline double gamma(long long n) {
  const double u = 0x1p-53;
  return (double)n * u / (1.0 - (double)n * u);
}

inline const char* path_name(int p) {
  static const char* names[] = {"native_loop", "native_grouped", "emu_loop", "emu_grouped",
                                "auto", "emu_grouped_reuse", "emu_loop_batched"};
  return (p >= 0 && p <= 6) ? names[p] : "?";
}
// "all" or a comma list of path names
inline std::vector<int> parse_paths(const std::string& s) {
  std::vector<int> out;
  if (s == "all") {
    for (int p = 0; p <= 6; ++p) out.push_back(p);
    return out;
  }
  size_t i = 0;
  while (i <= s.size()) {
    const size_t j = std::min(s.find(',', i), s.size());
    const std::string w = s.substr(i, j - i);
    for (int p = 0; p <= 6; ++p)
      if (w == path_name(p)) out.push_back(p);
    i = j + 1;
  }
  return out;
}
// adaptive moduli at an FP64-level target; the planner path may fall back to native
inline ggemm_config_t config_for(int path, int num_moduli) {
  ggemm_config_t c;
  std::memset(&c, 0, sizeof c);
  c.num_moduli = num_moduli;
  c.target_rel_err = 1e-15;
  c.allow_fallback = path == GGEMM_PATH_AUTO ? 1 : 0;
  return c;
}
inline std::string device_name() {
  hipDeviceProp_t prop;
  APP_HIP(hipGetDeviceProperties(&prop, 0));
  std::string g = prop.gcnArchName;
  for (auto& c : g)
    if (c == ',' || c == ':') c = ' ';
  return g;
}
// library settings that change results or timing, recorded in every CSV row
inline std::string env_string() {
  const char* keys[] = {"GGEMM_REUSE_PROMOTE", "GGEMM_STATS_REPAIR", "GGEMM_CALIB_JSON", "GGEMM_CALIB_DIR"};
  std::string out;
  for (const char* k : keys) {
    const char* v = std::getenv(k);
    std::string sv = v ? v : "unset";
    for (auto& c : sv)
      if (c == ',') c = ';';
    if (!out.empty()) out += ';';
    out += std::string(k) + "=" + sv;
  }
  return out;
}
inline unsigned grid_for(size_t n) { return (unsigned)std::min<size_t>((n + 255) / 256, 16384); }

// ---------------------------------------------------------------- deterministic synthetic data
__host__ __device__ inline uint64_t mix64(uint64_t z) {   // SplitMix64 finaliser
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__host__ __device__ inline double unit(uint64_t seed, uint64_t i) {   // U[0, 1) from (seed, i)
  return (double)(mix64(seed + 0x9E3779B97F4A7C15ull * (i + 1)) >> 11) * 0x1p-53;
}
// x = (U - 0.5) exp(phi Z), Z standard normal by Box-Muller (the Ozaki-scheme test distribution)
__global__ void fill_phi(double* x, size_t n, double phi, uint64_t seed) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const double u = unit(seed, 3 * i) - 0.5;
    const double u1 = 1.0 - unit(seed, 3 * i + 1), u2 = unit(seed, 3 * i + 2);
    const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    x[i] = u * exp(phi * z);
  }
}
__global__ void fill_value(double* x, size_t n, double v) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) x[i] = v;
}
__global__ void scale_values(double* x, size_t n, double s) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) x[i] *= s;
}
__global__ void abs_values(const double* x, double* y, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    y[i] = fabs(x[i]);
}

// ---------------------------------------------------------------- componentwise comparison
// Per block: max |x - r| / den over finite pairs with den > 0, the count of "bad" entries (x or r
// non-finite, or den == 0 with x != r), and the sums of (x - r)^2 and r^2 for the relative
// Frobenius error.  The host reduces the per-block partials (no atomics).
constexpr int kCmpBlocks = 512;
struct CmpPart {
  double emax, s_diff, s_ref;
  unsigned long long bad;
};
__global__ void __launch_bounds__(256) compare_partials(const double* x, const double* r, const double* den, size_t n,
                                                        CmpPart* part) {
  __shared__ CmpPart sh[256];
  CmpPart p{0.0, 0.0, 0.0, 0ull};
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const double ri = r[i], xi = x[i], di = den[i];
    if (!isfinite(ri)) { ++p.bad; continue; }
    p.s_ref += ri * ri;
    if (!isfinite(xi) || !isfinite(di)) { ++p.bad; continue; }
    const double d = fabs(xi - ri);
    if (di > 0) p.emax = fmax(p.emax, d / di);
    else if (d != 0) ++p.bad;
    p.s_diff += d * d;
  }
  sh[threadIdx.x] = p;
  __syncthreads();
  for (int o = 128; o; o >>= 1) {
    if ((int)threadIdx.x < o) {
      CmpPart& a = sh[threadIdx.x];
      const CmpPart& b = sh[threadIdx.x + o];
      a.emax = fmax(a.emax, b.emax);
      a.s_diff += b.s_diff;
      a.s_ref += b.s_ref;
      a.bad += b.bad;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = sh[0];
}
struct Err {
  double cw = NAN, rel_fro = NAN;
  unsigned long long bad = 0;
};
// Untimed; `part` is device scratch of kCmpBlocks entries.
inline Err compare(const double* x, const double* r, const double* den, size_t n, CmpPart* part, hipStream_t s) {
  Err e;
  std::vector<CmpPart> h(kCmpBlocks, CmpPart{0.0, 0.0, 0.0, 0ull});
  const unsigned g = std::max(1u, std::min<unsigned>(kCmpBlocks, grid_for(n)));
  APP_HIP(hipMemcpyAsync(part, h.data(), sizeof(CmpPart) * kCmpBlocks, hipMemcpyHostToDevice, s));
  if (n) hipLaunchKernelGGL(compare_partials, dim3(g), dim3(256), 0, s, x, r, den, n, part);
  APP_HIP(hipGetLastError());
  APP_HIP(hipMemcpyAsync(h.data(), part, sizeof(CmpPart) * kCmpBlocks, hipMemcpyDeviceToHost, s));
  APP_HIP(hipStreamSynchronize(s));
  double emax = 0, sd = 0, sr = 0;
  unsigned long long bad = 0;
  for (const auto& p : h) {
    emax = std::max(emax, p.emax);
    sd += p.s_diff;
    sr += p.s_ref;
    bad += p.bad;
  }
  e.cw = emax;
  e.bad = bad;
  e.rel_fro = sr > 0 ? std::sqrt(sd / sr) : (sd > 0 ? INFINITY : 0.0);
  return e;
}

template <class F>
inline double wall_ms(F&& f) {
  const auto t0 = std::chrono::steady_clock::now();
  f();
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

}  // namespace app
