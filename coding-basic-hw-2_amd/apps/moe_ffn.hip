// moe_ffn.hip -- application benchmark: FP64 mixture-of-experts FFN forward pass whose two expert
// GEMMs are grouped GEMMs through ggemm_grouped_dgemm.  Scenario and pipeline of the reference's
// bench/app/moe_ffn_fp64.cu (FP64 expert networks of machine-learned interatomic potentials and
// of surrogates inside FP64 solvers: skewed, data-dependent expert loads m_e).
//
// Pipeline (column-major, T tokens, model width d, hidden width f, E experts, top-k routing):
//   route   Zipf(s) top-k expert choice per token from a counter hash (deterministic), gates
//           normalised to 1; per-expert rank of every assignment (a workgroup per expert, ballot
//           prefix counts: assignments keep token order); counts to the host, grouped descriptors
//           built there, expert offsets back (pinned buffers; part of the timed stage, as a real
//           layer's routing round trip is)
//   gather  Xg_e (m_e x d, ld m_e) <- the tokens routed to e
//   up      H_e  = Xg_e W1_e   (m_e x f)                 grouped GEMM
//   act     Ha = tanh(H) or tanh-GELU(H)
//   down    Yd_e = Ha_e W2_e   (m_e x d)                 grouped GEMM
//   scatter Y(t, :) = sum_j g_tj Yd_{e_tj}(slot_tj, :)   (j ascending: deterministic)
// Every stage is bracketed by HIP events on one stream; nothing is allocated inside the timed
// region.
//
// Correctness: each path against the same pipeline through NATIVE_LOOP:
//   err_up = max |H - H_ref| / (|Xg| |W1|)
//   err_y  = max |Y - Y_ref| / den_y,  den_y = scatter(|g|, (|Ha_ref| + L |Xg||W1|) |W2|)
// (L = sup |act'|), reported also as a multiple of the a-priori bound 2 gamma_n (n = d for up,
// max(d, f) + topk + 4 for the layer): <= 1 means agreement at FP64 level.
//
// Usage: moe_ffn [--tokens 4096] [--experts 16] [--topk 2] [--d-model 1024] [--d-ff 2048]
//                [--zipf 1.0] [--phi 0.5] [--act tanh|gelu] [--seed 1234] [--moduli 0]
//                [--paths all] [--reps 10] [--warmup 3] [--csv moe_ffn.csv] [--append]
#include "app_util.hpp"

namespace {

constexpr int kMaxTopk = 8;

// ---- route: k distinct experts from the Zipf CDF (redraw on a repeat), gates 0.05 + U, normalised
__global__ void route_kernel(int T, int E, int topk, const double* __restrict__ cdf, uint64_t seed,
                             int* __restrict__ expert, double* __restrict__ gate) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  int chosen[kMaxTopk];
  double w[kMaxTopk], ws = 0.0;
  for (int j = 0; j < topk; ++j) {
    int e = 0;
    for (int draw = 0; draw < 4096; ++draw) {
      const double u = app::unit(seed, ((uint64_t)t * kMaxTopk + j) * 4096 + draw);
      int lo = 0, hi = E - 1;   // first e with cdf[e] > u
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (cdf[mid] > u) hi = mid; else lo = mid + 1;
      }
      e = lo;
      bool seen = false;
      for (int q = 0; q < j; ++q) seen |= chosen[q] == e;
      if (!seen) break;
    }
    chosen[j] = e;
    w[j] = 0.05 + app::unit(seed ^ 0xA5A5A5A5ull, (uint64_t)t * kMaxTopk + j);
    ws += w[j];
  }
  for (int j = 0; j < topk; ++j) {
    expert[t * topk + j] = chosen[j];
    gate[t * topk + j] = w[j] / ws;
  }
}

// ---- rank: slot of every assignment within its expert in assignment order; one workgroup of four
// waves per expert: within a wave the ballot mask gives the prefix count, the wave totals are
// combined through LDS, and the running count carries across chunks of 256 assignments
__global__ void __launch_bounds__(256) rank_kernel(int A, const int* __restrict__ expert, int* __restrict__ slot,
                                                   int* __restrict__ counts) {
  __shared__ int wave_tot[4];
  const int e = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int running = 0;
  for (int base = 0; base < A; base += 256) {
    const int i = base + threadIdx.x;
    const bool mine = i < A && expert[i] == e;
    const unsigned long long mask = __ballot(mine);
    const int before = __popcll(mask & ((1ull << lane) - 1ull));
    if (lane == 0) wave_tot[wave] = __popcll(mask);
    __syncthreads();
    int off = running;
    for (int w = 0; w < wave; ++w) off += wave_tot[w];
    if (mine) slot[i] = off + before;
    running += wave_tot[0] + wave_tot[1] + wave_tot[2] + wave_tot[3];
    __syncthreads();
  }
  if (threadIdx.x == 0) counts[e] = running;
}

// Xg_e(slot, c) = X(t, c): expert blocks at row offset off[e], each column-major with ld m_e
__global__ void gather_kernel(int T, int d, int topk, const double* __restrict__ X, const int* __restrict__ expert,
                              const int* __restrict__ slot, const int* __restrict__ off,
                              const int* __restrict__ counts, double* __restrict__ Xg) {
  const size_t A = (size_t)T * topk, n = A * d;
  for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < n; idx += (size_t)gridDim.x * blockDim.x) {
    const size_t i = idx % A, c = idx / A;
    const int e = expert[i];
    Xg[(size_t)off[e] * d + slot[i] + c * (size_t)counts[e]] = X[i / topk + c * (size_t)T];
  }
}

__device__ __forceinline__ double activation(double x, int kind) {
  if (kind == 0) return tanh(x);
  const double c = 0.7978845608028654;   // sqrt(2 / pi): tanh-GELU
  return 0.5 * x * (1.0 + tanh(c * (x + 0.044715 * x * x * x)));
}
__global__ void act_kernel(const double* __restrict__ H, double* __restrict__ Ha, size_t n, int kind) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    Ha[i] = activation(H[i], kind);
}
// Y(t, c) = sum_j g_tj Yd_{e_tj}(slot_tj, c); with abs_gate the gates enter as |g| (denominator)
__global__ void scatter_kernel(int T, int d, int topk, const double* __restrict__ Yd, const int* __restrict__ expert,
                               const int* __restrict__ slot, const double* __restrict__ gate,
                               const int* __restrict__ off, const int* __restrict__ counts, double* __restrict__ Y,
                               int abs_gate) {
  const size_t n = (size_t)T * d;
  for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < n; idx += (size_t)gridDim.x * blockDim.x) {
    const int t = (int)(idx % T);
    const size_t c = idx / T;
    double acc = 0.0;
    for (int j = 0; j < topk; ++j) {
      const int i = t * topk + j, e = expert[i];
      const double g = abs_gate ? fabs(gate[i]) : gate[i];
      acc += g * Yd[(size_t)off[e] * d + slot[i] + c * (size_t)counts[e]];
    }
    Y[idx] = acc;
  }
}
__global__ void den_mix_kernel(const double* __restrict__ Ha, const double* __restrict__ P, double L,
                               double* __restrict__ Q, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    Q[i] = fabs(Ha[i]) + L * P[i];
}

struct Layer {
  int T, E, topk, d, f, act;
  size_t A;
  double *X, *W1, *W2, *Xg, *H, *Ha, *Yd, *Y, *gate, *cdf;
  int *expert, *slot, *counts, *off;
  int *h_counts, *h_off;   // pinned
  std::vector<ggemm_problem_t> up, down;
};

// grouped descriptors of the two GEMMs from the routed counts (host; inside the timed route stage)
void build_descriptors(Layer& L, const double* Xg, const double* W1, double* H, const double* Ha, const double* W2,
                       double* Yd) {
  L.up.clear();
  L.down.clear();
  int o = 0;
  for (int e = 0; e < L.E; ++e) {
    L.h_off[e] = o;
    const int me = L.h_counts[e];
    if (me > 0) {
      L.up.push_back(ggemm_problem_t{me, L.f, L.d, Xg + (size_t)o * L.d, me, W1 + (size_t)e * L.d * L.f, L.d,
                                     H + (size_t)o * L.f, me, 1.0, 0.0});
      L.down.push_back(ggemm_problem_t{me, L.d, L.f, Ha + (size_t)o * L.f, me, W2 + (size_t)e * L.f * L.d, L.f,
                                       Yd + (size_t)o * L.d, me, 1.0, 0.0});
    }
    o += me;
  }
}

}  // namespace

int main(int argc, char** argv) {
  int T = 4096, E = 16, topk = 2, d = 1024, f = 2048, reps = 10, warmup = 3, nmod = 0;
  double zipf = 1.0, phi = 0.5;
  uint64_t seed = 1234;
  std::string paths_s = "all", csv = "moe_ffn.csv", act_s = "tanh";
  bool append = false;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    auto next = [&]() { return i + 1 < argc ? std::string(argv[++i]) : std::string(); };
    if (a == "--tokens") T = std::atoi(next().c_str());
    else if (a == "--experts") E = std::atoi(next().c_str());
    else if (a == "--topk") topk = std::atoi(next().c_str());
    else if (a == "--d-model") d = std::atoi(next().c_str());
    else if (a == "--d-ff") f = std::atoi(next().c_str());
    else if (a == "--zipf") zipf = std::atof(next().c_str());
    else if (a == "--phi") phi = std::atof(next().c_str());
    else if (a == "--act") act_s = next();
    else if (a == "--seed") seed = std::strtoull(next().c_str(), nullptr, 10);
    else if (a == "--moduli") nmod = std::atoi(next().c_str());
    else if (a == "--paths") paths_s = next();
    else if (a == "--reps") reps = std::atoi(next().c_str());
    else if (a == "--warmup") warmup = std::atoi(next().c_str());
    else if (a == "--csv") csv = next();
    else if (a == "--append") append = true;
    else { std::fprintf(stderr, "unknown argument %s\n", a.c_str()); return 2; }
  }
  if (T <= 0 || d <= 0 || f <= 0 || E <= 0) { std::fprintf(stderr, "--tokens/--d-model/--d-ff/--experts must be > 0\n"); return 2; }
  if (topk < 1 || topk > kMaxTopk || topk > E) { std::fprintf(stderr, "need 1 <= topk <= min(%d, experts)\n", kMaxTopk); return 2; }
  if (act_s != "tanh" && act_s != "gelu") { std::fprintf(stderr, "--act tanh|gelu\n"); return 2; }
  const int act = act_s == "gelu" ? 1 : 0;
  const double Lact = act ? 1.13 : 1.0;   // sup |act'| (tanh-GELU: 1.129...)
  const std::vector<int> paths = app::parse_paths(paths_s);
  const std::string envs = app::env_string(), gpu = app::device_name();

  Layer L{};
  L.T = T; L.E = E; L.topk = topk; L.d = d; L.f = f; L.act = act; L.A = (size_t)T * topk;
  const size_t A = L.A;
  hipStream_t s;
  APP_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  auto dalloc = [](size_t n) { double* p; APP_HIP(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(double))); return p; };
  L.X = dalloc((size_t)T * d); L.W1 = dalloc((size_t)E * d * f); L.W2 = dalloc((size_t)E * f * d);
  L.Xg = dalloc(A * d); L.H = dalloc(A * f); L.Ha = dalloc(A * f); L.Yd = dalloc(A * d); L.Y = dalloc((size_t)T * d);
  L.gate = dalloc(A); L.cdf = dalloc(E);
  APP_HIP(hipMalloc(&L.expert, A * sizeof(int))); APP_HIP(hipMalloc(&L.slot, A * sizeof(int)));
  APP_HIP(hipMalloc(&L.counts, E * sizeof(int))); APP_HIP(hipMalloc(&L.off, E * sizeof(int)));
  APP_HIP(hipHostMalloc((void**)&L.h_counts, E * sizeof(int), hipHostMallocDefault));
  APP_HIP(hipHostMalloc((void**)&L.h_off, E * sizeof(int), hipHostMallocDefault));
  std::memset(L.h_counts, 0, E * sizeof(int));
  std::memset(L.h_off, 0, E * sizeof(int));
  L.up.reserve(E); L.down.reserve(E);
  double *H_ref = dalloc(A * f), *Ha_ref = dalloc(A * f), *Y_ref = dalloc((size_t)T * d);
  double *aXg = dalloc(A * d), *aW1 = dalloc((size_t)E * d * f), *aW2 = dalloc((size_t)E * f * d);
  double *P = dalloc(A * f), *Q = dalloc(A * f), *R = dalloc(A * d), *den_y = dalloc((size_t)T * d);
  app::CmpPart* part;
  APP_HIP(hipMalloc(&part, sizeof(app::CmpPart) * app::kCmpBlocks));
  hipEvent_t ev[7];
  for (auto& e : ev) APP_HIP(hipEventCreate(&e));

  // deterministic data; weights scaled so that the pre-activations stay O(1)
  hipLaunchKernelGGL(app::fill_phi, dim3(app::grid_for((size_t)T * d)), dim3(256), 0, s, L.X, (size_t)T * d, phi, seed ^ 0x11);
  hipLaunchKernelGGL(app::fill_phi, dim3(app::grid_for((size_t)E * d * f)), dim3(256), 0, s, L.W1, (size_t)E * d * f, phi, seed ^ 0x22);
  hipLaunchKernelGGL(app::fill_phi, dim3(app::grid_for((size_t)E * f * d)), dim3(256), 0, s, L.W2, (size_t)E * f * d, phi, seed ^ 0x33);
  hipLaunchKernelGGL(app::scale_values, dim3(app::grid_for((size_t)E * d * f)), dim3(256), 0, s, L.W1, (size_t)E * d * f, 2.0 / std::sqrt((double)d));
  hipLaunchKernelGGL(app::scale_values, dim3(app::grid_for((size_t)E * f * d)), dim3(256), 0, s, L.W2, (size_t)E * f * d, 2.0 / std::sqrt((double)f));
  {
    std::vector<double> c(E);
    double z = 0.0, acc = 0.0;
    for (int e = 0; e < E; ++e) z += std::pow(e + 1.0, -zipf);
    for (int e = 0; e < E; ++e) { acc += std::pow(e + 1.0, -zipf) / z; c[e] = acc; }
    c[E - 1] = 1.0 + 1e-12;
    APP_HIP(hipMemcpyAsync(L.cdf, c.data(), E * sizeof(double), hipMemcpyHostToDevice, s));
    APP_HIP(hipStreamSynchronize(s));
  }
  // handle budgets: the worst case over both GEMMs, independent of the routing outcome
  const size_t maxA = A * (size_t)std::max(d, f) + 1, maxB = (size_t)E * d * f + 1, maxC = A * (size_t)std::max(d, f) + 1;

  // one forward pass; e != nullptr records the stage events
  auto forward = [&](ggemm_handle_t h, int p, const ggemm_config_t& cfg, hipEvent_t* e, ggemm_stats_t* su,
                     ggemm_stats_t* sd) -> int {
    if (e) APP_HIP(hipEventRecord(e[0], s));
    hipLaunchKernelGGL(route_kernel, dim3((T + 127) / 128), dim3(128), 0, s, T, E, topk, L.cdf, seed, L.expert, L.gate);
    hipLaunchKernelGGL(rank_kernel, dim3(E), dim3(256), 0, s, (int)A, L.expert, L.slot, L.counts);
    APP_HIP(hipMemcpyAsync(L.h_counts, L.counts, E * sizeof(int), hipMemcpyDeviceToHost, s));
    APP_HIP(hipStreamSynchronize(s));
    build_descriptors(L, L.Xg, L.W1, L.H, L.Ha, L.W2, L.Yd);
    APP_HIP(hipMemcpyAsync(L.off, L.h_off, E * sizeof(int), hipMemcpyHostToDevice, s));
    if (e) APP_HIP(hipEventRecord(e[1], s));
    hipLaunchKernelGGL(gather_kernel, dim3(app::grid_for(A * d)), dim3(256), 0, s, T, d, topk, L.X, L.expert, L.slot,
                       L.off, L.counts, L.Xg);
    if (e) APP_HIP(hipEventRecord(e[2], s));
    int rc = ggemm_grouped_dgemm(h, (ggemm_path_t)p, &cfg, L.up.data(), (int)L.up.size(), su);
    if (e) APP_HIP(hipEventRecord(e[3], s));
    hipLaunchKernelGGL(act_kernel, dim3(app::grid_for(A * f)), dim3(256), 0, s, L.H, L.Ha, A * f, act);
    if (e) APP_HIP(hipEventRecord(e[4], s));
    rc |= ggemm_grouped_dgemm(h, (ggemm_path_t)p, &cfg, L.down.data(), (int)L.down.size(), sd);
    if (e) APP_HIP(hipEventRecord(e[5], s));
    hipLaunchKernelGGL(scatter_kernel, dim3(app::grid_for((size_t)T * d)), dim3(256), 0, s, T, d, topk, L.Yd, L.expert,
                       L.slot, L.gate, L.off, L.counts, L.Y, 0);
    if (e) APP_HIP(hipEventRecord(e[6], s));
    return rc;
  };

  // ---- NATIVE_LOOP reference and the error denominators
  int ref_ok = 0, load_max = 0, load_min = 0, active = 0;
  {
    ggemm_handle_t h = nullptr;
    if (ggemm_create(&h, E, maxA, maxB, maxC, s) == 0 && h) {
      const ggemm_config_t cfg = app::config_for(GGEMM_PATH_NATIVE_LOOP, 0);
      ggemm_stats_t st;
      if (forward(h, GGEMM_PATH_NATIVE_LOOP, cfg, nullptr, &st, &st) == 0) {
        APP_HIP(hipMemcpyAsync(H_ref, L.H, A * f * sizeof(double), hipMemcpyDeviceToDevice, s));
        APP_HIP(hipMemcpyAsync(Ha_ref, L.Ha, A * f * sizeof(double), hipMemcpyDeviceToDevice, s));
        APP_HIP(hipMemcpyAsync(Y_ref, L.Y, (size_t)T * d * sizeof(double), hipMemcpyDeviceToDevice, s));
        // P = |Xg||W1|, Q = |Ha_ref| + L P, R = Q |W2|, den_y = scatter(|g|, R)
        hipLaunchKernelGGL(app::abs_values, dim3(app::grid_for(A * d)), dim3(256), 0, s, L.Xg, aXg, A * d);
        hipLaunchKernelGGL(app::abs_values, dim3(app::grid_for((size_t)E * d * f)), dim3(256), 0, s, L.W1, aW1, (size_t)E * d * f);
        hipLaunchKernelGGL(app::abs_values, dim3(app::grid_for((size_t)E * f * d)), dim3(256), 0, s, L.W2, aW2, (size_t)E * f * d);
        build_descriptors(L, aXg, aW1, P, Q, aW2, R);
        int rc = ggemm_grouped_dgemm(h, GGEMM_PATH_NATIVE_LOOP, &cfg, L.up.data(), (int)L.up.size(), &st);
        hipLaunchKernelGGL(den_mix_kernel, dim3(app::grid_for(A * f)), dim3(256), 0, s, Ha_ref, P, Lact, Q, A * f);
        rc |= ggemm_grouped_dgemm(h, GGEMM_PATH_NATIVE_LOOP, &cfg, L.down.data(), (int)L.down.size(), &st);
        hipLaunchKernelGGL(scatter_kernel, dim3(app::grid_for((size_t)T * d)), dim3(256), 0, s, T, d, topk, R, L.expert,
                           L.slot, L.gate, L.off, L.counts, den_y, 1);
        APP_HIP(hipStreamSynchronize(s));
        ref_ok = rc == 0;
      }
      ggemm_destroy(h);
    }
    if (ref_ok) {
      load_max = *std::max_element(L.h_counts, L.h_counts + E);
      load_min = *std::min_element(L.h_counts, L.h_counts + E);
      for (int e = 0; e < E; ++e) active += L.h_counts[e] > 0;
    }
  }
  if (!ref_ok) std::fprintf(stderr, "warning: the NATIVE_LOOP reference failed; error columns are NaN\n");
  const double flops = 2.0 * 2.0 * (double)A * d * f;
  const double bnd_up = 2.0 * app::gamma(d), bnd_y = 2.0 * app::gamma((long long)std::max(d, f) + topk + 4);

  FILE* fo = std::fopen(csv.c_str(), append ? "a" : "w");
  if (!fo) { std::perror(csv.c_str()); return 1; }
  std::fseek(fo, 0, SEEK_END);
  if (std::ftell(fo) == 0)
    std::fprintf(fo, "app,path,T,E,topk,d_model,d_ff,zipf,phi,act,seed,num_moduli_cfg,experts_active,load_max,load_min,"
                     "gemm_flops,total_ms_median,total_ms_mean,wall_ms_median,route_ms,gather_ms,up_ms,act_ms,down_ms,"
                     "scatter_ms,gemm_pct,eff_GFLOPS,launches_up,launches_down,fallback_up,fallback_down,moduli_min,"
                     "moduli_max,err_up_cw,err_up_over_bound,err_y_cw,err_y_over_bound,rel_fro_y,nonfinite,reps,gpu,env,"
                     "status\n");
  std::fprintf(stderr, "device %s  T=%d E=%d topk=%d d=%d f=%d zipf=%.2f  loads max/min %d/%d active %d\n", gpu.c_str(), T,
               E, topk, d, f, zipf, load_max, load_min, active);
  static const char* stage[6] = {"route", "gather", "up", "act", "down", "scatter"};
  for (int p : paths) {
    const ggemm_config_t cfg = app::config_for(p, nmod);
    ggemm_handle_t h = nullptr;
    const char* status = "ok";
    if (ggemm_create(&h, E, maxA, maxB, maxC, s) != 0 || !h) status = "create_failed";
    ggemm_stats_t su{}, sd{};
    int rc = 0;
    for (int r = 0; h && rc == 0 && r < warmup; ++r) rc = forward(h, p, cfg, nullptr, &su, &sd);
    if (h) APP_HIP(hipStreamSynchronize(s));
    std::vector<double> tot, wall, st[6];
    for (int r = 0; h && rc == 0 && r < reps; ++r) {
      const double w = app::wall_ms([&] {
        rc = forward(h, p, cfg, ev, &su, &sd);
        APP_HIP(hipEventSynchronize(ev[6]));
      });
      if (rc != 0) break;
      float ms;
      APP_HIP(hipEventElapsedTime(&ms, ev[0], ev[6]));
      tot.push_back(ms);
      for (int k = 0; k < 6; ++k) {
        APP_HIP(hipEventElapsedTime(&ms, ev[k], ev[k + 1]));
        st[k].push_back(ms);
      }
      wall.push_back(w);
    }
    if (h && rc != 0) status = "call_failed";
    if (hipGetLastError() != hipSuccess) status = "hip_error";
    app::Err eu, ey;
    if (h && rc == 0 && ref_ok) {   // untimed check on outputs poisoned with NaN first
      hipLaunchKernelGGL(app::fill_value, dim3(app::grid_for(A * f)), dim3(256), 0, s, L.H, A * f, (double)NAN);
      hipLaunchKernelGGL(app::fill_value, dim3(app::grid_for(A * d)), dim3(256), 0, s, L.Yd, A * d, (double)NAN);
      hipLaunchKernelGGL(app::fill_value, dim3(app::grid_for((size_t)T * d)), dim3(256), 0, s, L.Y, (size_t)T * d, (double)NAN);
      if (forward(h, p, cfg, nullptr, &su, &sd) == 0) {
        eu = app::compare(L.H, H_ref, P, A * f, part, s);
        ey = app::compare(L.Y, Y_ref, den_y, (size_t)T * d, part, s);
      } else {
        status = "check_failed";
      }
    }
    const double tmed = app::median(tot), tmean = app::mean(tot);
    double sm[6];
    for (int k = 0; k < 6; ++k) sm[k] = app::mean(st[k]);
    std::fprintf(fo, "moe_ffn,%s,%d,%d,%d,%d,%d,%.3f,%.2f,%s,%llu,%d,%d,%d,%d,%.6e,%.6f,%.6f,%.6f", app::path_name(p), T, E,
                 topk, d, f, zipf, phi, act_s.c_str(), (unsigned long long)seed, nmod, active, load_max, load_min, flops,
                 tmed, tmean, app::median(wall));
    for (int k = 0; k < 6; ++k) std::fprintf(fo, ",%.6f", sm[k]);
    std::fprintf(fo, ",%.3f,%.3f,%d,%d,%d,%d,%d,%d,%.6e,%.6e,%.6e,%.6e,%.6e,%llu,%d,%s,%s,%s\n",
                 100.0 * (sm[2] + sm[4]) / tmean, flops / (tmed * 1e-3) / 1e9, su.kernel_launches, sd.kernel_launches,
                 su.num_fallback, sd.num_fallback, std::min(su.moduli_min, sd.moduli_min),
                 std::max(su.moduli_max, sd.moduli_max), eu.cw, eu.cw / bnd_up, ey.cw, ey.cw / bnd_y, ey.rel_fro,
                 eu.bad + ey.bad, (int)tot.size(), gpu.c_str(), envs.c_str(), status);
    std::fflush(fo);
    std::fprintf(stderr, "%-18s total %9.3f ms (%8.1f GFLOP/s)", app::path_name(p), tmed, flops / (tmed * 1e-3) / 1e9);
    for (int k = 0; k < 6; ++k) std::fprintf(stderr, " %s %4.1f%%", stage[k], 100.0 * sm[k] / tmean);
    std::fprintf(stderr, "  err_up %.2e err_y %.2e (%.2g x bound) %s\n", eu.cw, ey.cw, ey.cw / bnd_y, status);
    if (h) ggemm_destroy(h);
    if (!std::strcmp(status, "hip_error")) { std::fclose(fo); return 1; }
  }
  std::fclose(fo);
  return 0;
}
