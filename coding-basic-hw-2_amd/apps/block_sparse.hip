// block_sparse.hip -- application benchmark: FP64 block-sparse (BSR, variable block sizes) matrix
// times dense multi-vector, Y = A X, with every dense product a problem of ggemm_grouped_dgemm.
// Scenario and formulations of the reference's bench/app/block_sparse_fp64.cu: atom-blocked
// matrices of Gaussian-basis electronic-structure codes (one block per pair of atoms within a
// cutoff, block sizes from the elements' basis sets), where F C_occ-type products are many small
// non-uniform FP64 GEMMs plus a reduction.
//
// Instance (fixed seed): atoms uniform in a periodic cube of number density rho; elements 50 % H,
// 35 % C, 15 % O with basis sizes (dz: 5/14/14, tz: 14/30/30, qz: 30/55/55); block (I, J) stored iff
// the minimum-image distance r_IJ <= cutoff, its entries (U - 0.5) exp(phi Z) times exp(-r_IJ / 2);
// X is N x nrhs.  The pattern is static, so descriptors are built once outside the timed region.
//
// Formulations (--mode block|panel|both):
//   block  one problem per stored block, T_b = A_IJ X_J (X_J a row slice of X, ldb = N), then a
//          deterministic segmented sum Y_I = sum_J T_b.            stages: gemm, reduce
//   panel  one problem per block row: the row's blocks are one r_I x K_I column-major panel; the
//          X rows of its block columns are gathered into a packed K_I x nrhs panel and
//          Y_I = A_I Xp_I.                                         stages: gather, gemm
// Handles are created with ggemm_create_ex(min_k = the smallest block width), since residues of
// k < 32 are padded to 32 (the reference's workspace contract).
// Correctness against the same formulation through NATIVE_LOOP: err = max |Y - Y_ref| / (|A||X|)
// (the denominator through the same formulation on |A|, |X|), also as a multiple of 2 gamma_n,
// n = max_I K_I + max_I (blocks in row I) + 1.
//
// Usage: block_sparse [--atoms 1024] [--density 0.1] [--cutoff 6] [--basis dz|tz|qz] [--nrhs 128]
//                     [--mode both] [--phi 0.5] [--seed 4321] [--moduli 0] [--paths all] [--reps 5]
//                     [--warmup 2] [--csv block_sparse.csv] [--append]
#include "app_util.hpp"

namespace {

__global__ void block_scale_kernel(double* __restrict__ vals, const size_t* __restrict__ voff,
                                   const int* __restrict__ vlen, const double* __restrict__ sc, int nb) {
  for (int b = blockIdx.x; b < nb; b += gridDim.x)
    for (int i = threadIdx.x; i < vlen[b]; i += blockDim.x) vals[voff[b] + i] *= sc[b];
}
// block mode: Y(row, c) = sum over the blocks b of row I (ascending) of T_b(loc, c)
__global__ void reduce_kernel(int N, int nrhs, const int* __restrict__ row_block, const int* __restrict__ row_loc,
                              const int* __restrict__ bsz, const int* __restrict__ rowptr,
                              const size_t* __restrict__ toff, const double* __restrict__ Tb, double* __restrict__ Y) {
  const size_t n = (size_t)N * nrhs;
  for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < n; idx += (size_t)gridDim.x * blockDim.x) {
    const int row = (int)(idx % N);
    const size_t c = idx / N;
    const int I = row_block[row], loc = row_loc[row], r = bsz[I];
    double acc = 0.0;
    for (int b = rowptr[I]; b < rowptr[I + 1]; ++b) acc += Tb[toff[b] + loc + c * r];
    Y[idx] = acc;
  }
}
// panel mode: Xp_I(p, c) = X(src, c) for every packed row q = (I, p, src)
__global__ void gather_panel_kernel(int N, int nrhs, size_t rows, const int* __restrict__ q_block,
                                    const int* __restrict__ q_pos, const int* __restrict__ q_src,
                                    const size_t* __restrict__ poff, const int* __restrict__ Kr,
                                    const double* __restrict__ X, double* __restrict__ Xp) {
  const size_t n = rows * nrhs;
  for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < n; idx += (size_t)gridDim.x * blockDim.x) {
    const size_t q = idx % rows, c = idx / rows;
    const int I = q_block[q];
    Xp[poff[I] + q_pos[q] + c * (size_t)Kr[I]] = X[q_src[q] + c * (size_t)N];
  }
}

template <class T>
T* upload(const std::vector<T>& v) {
  T* p;
  APP_HIP(hipMalloc(&p, std::max<size_t>(v.size(), 1) * sizeof(T)));
  if (!v.empty()) APP_HIP(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice));
  return p;
}

}  // namespace

int main(int argc, char** argv) {
  int atoms = 1024, nrhs = 128, reps = 5, warmup = 2, nmod = 0;
  double rho = 0.1, cutoff = 6.0, phi = 0.5;
  uint64_t seed = 4321;
  std::string basis = "dz", mode_s = "both", paths_s = "all", csv = "block_sparse.csv";
  bool append = false;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    auto next = [&]() { return i + 1 < argc ? std::string(argv[++i]) : std::string(); };
    if (a == "--atoms") atoms = std::atoi(next().c_str());
    else if (a == "--density") rho = std::atof(next().c_str());
    else if (a == "--cutoff") cutoff = std::atof(next().c_str());
    else if (a == "--basis") basis = next();
    else if (a == "--nrhs") nrhs = std::atoi(next().c_str());
    else if (a == "--mode") mode_s = next();
    else if (a == "--phi") phi = std::atof(next().c_str());
    else if (a == "--seed") seed = std::strtoull(next().c_str(), nullptr, 10);
    else if (a == "--moduli") nmod = std::atoi(next().c_str());
    else if (a == "--paths") paths_s = next();
    else if (a == "--reps") reps = std::atoi(next().c_str());
    else if (a == "--warmup") warmup = std::atoi(next().c_str());
    else if (a == "--csv") csv = next();
    else if (a == "--append") append = true;
    else { std::fprintf(stderr, "unknown argument %s\n", a.c_str()); return 2; }
  }
  if (atoms <= 0 || nrhs <= 0 || !(rho > 0) || !(cutoff >= 0)) { std::fprintf(stderr, "bad sizes\n"); return 2; }
  int nbf[3];   // H, C, O
  if (basis == "dz") { nbf[0] = 5; nbf[1] = 14; nbf[2] = 14; }
  else if (basis == "tz") { nbf[0] = 14; nbf[1] = 30; nbf[2] = 30; }
  else if (basis == "qz") { nbf[0] = 30; nbf[1] = 55; nbf[2] = 55; }
  else { std::fprintf(stderr, "--basis dz|tz|qz\n"); return 2; }
  std::vector<std::string> modes;
  if (mode_s == "both" || mode_s == "block") modes.push_back("block");
  if (mode_s == "both" || mode_s == "panel") modes.push_back("panel");
  const std::vector<int> paths = app::parse_paths(paths_s);
  const std::string envs = app::env_string(), gpu = app::device_name();

  // ---- structure (host, deterministic)
  const double box = std::cbrt(atoms / rho);
  std::vector<double> pos(3 * (size_t)atoms);
  std::vector<int> bsz(atoms), rstart(atoms + 1, 0);
  for (int a = 0; a < atoms; ++a) {
    for (int k = 0; k < 3; ++k) pos[3 * a + k] = app::unit(seed, 4 * (uint64_t)a + k) * box;
    const double u = app::unit(seed, 4 * (uint64_t)a + 3);
    bsz[a] = nbf[u < 0.50 ? 0 : (u < 0.85 ? 1 : 2)];
    rstart[a + 1] = rstart[a] + bsz[a];
  }
  const int N = rstart[atoms];
  std::vector<int> rowptr(atoms + 1, 0), bcol, Kr(atoms, 0);
  std::vector<double> bscale;
  for (int I = 0; I < atoms; ++I) {
    for (int J = 0; J < atoms; ++J) {
      double r2 = 0.0;
      for (int k = 0; k < 3; ++k) {
        double dx = pos[3 * I + k] - pos[3 * J + k];
        dx -= box * std::nearbyint(dx / box);
        r2 += dx * dx;
      }
      const double r = std::sqrt(r2);
      if (r <= cutoff) {
        bcol.push_back(J);
        bscale.push_back(std::exp(-r / 2.0));
        Kr[I] += bsz[J];
      }
    }
    rowptr[I + 1] = (int)bcol.size();
  }
  const int nb = (int)bcol.size();
  std::vector<size_t> voff(nb + 1, 0), toff(nb + 1, 0), poff(atoms + 1, 0);
  std::vector<int> vlen(nb);
  int maxK = 0, maxRow = 0;
  for (int I = 0; I < atoms; ++I) {
    for (int b = rowptr[I]; b < rowptr[I + 1]; ++b) {
      vlen[b] = bsz[I] * bsz[bcol[b]];
      voff[b + 1] = voff[b] + vlen[b];
      toff[b + 1] = toff[b] + (size_t)bsz[I] * nrhs;
    }
    poff[I + 1] = poff[I] + (size_t)Kr[I] * nrhs;
    maxK = std::max(maxK, Kr[I]);
    maxRow = std::max(maxRow, rowptr[I + 1] - rowptr[I]);
  }
  const size_t nnz = voff[nb], nT = toff[nb], nXp = poff[atoms], prow = nXp / nrhs;
  std::vector<int> row_block(N), row_loc(N), q_block(prow), q_pos(prow), q_src(prow);
  for (int I = 0; I < atoms; ++I)
    for (int l = 0; l < bsz[I]; ++l) { row_block[rstart[I] + l] = I; row_loc[rstart[I] + l] = l; }
  for (size_t q = 0, I = 0; I < (size_t)atoms; ++I) {
    int p = 0;
    for (int b = rowptr[I]; b < rowptr[I + 1]; ++b)
      for (int l = 0; l < bsz[bcol[b]]; ++l, ++q, ++p) { q_block[q] = (int)I; q_pos[q] = p; q_src[q] = rstart[bcol[b]] + l; }
  }
  const double flops = 2.0 * (double)nnz * nrhs;
  std::fprintf(stderr, "device %s  atoms=%d basis=%s N=%d blocks=%d (%.1f per row) nnz=%zu (%.3f%%) maxK=%d nrhs=%d\n",
               gpu.c_str(), atoms, basis.c_str(), N, nb, (double)nb / atoms, nnz, 100.0 * nnz / ((double)N * N), maxK, nrhs);

  // ---- device data (outside every timed region)
  hipStream_t s;
  APP_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  auto dalloc = [](size_t n) { double* p; APP_HIP(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(double))); return p; };
  double *Av = dalloc(nnz), *X = dalloc((size_t)N * nrhs), *Y = dalloc((size_t)N * nrhs), *Tb = dalloc(nT), *Xp = dalloc(nXp);
  double *aAv = dalloc(nnz), *aX = dalloc((size_t)N * nrhs), *Yref = dalloc((size_t)N * nrhs), *den = dalloc((size_t)N * nrhs);
  size_t* d_voff = upload(voff);
  int* d_vlen = upload(vlen);
  double* d_bscale = upload(bscale);
  int *d_row_block = upload(row_block), *d_row_loc = upload(row_loc), *d_bsz = upload(bsz), *d_rowptr = upload(rowptr);
  size_t *d_toff = upload(toff), *d_poff = upload(poff);
  int *d_qb = upload(q_block), *d_qp = upload(q_pos), *d_qs = upload(q_src), *d_Kr = upload(Kr);
  APP_HIP(hipDeviceSynchronize());
  app::CmpPart* part;
  APP_HIP(hipMalloc(&part, sizeof(app::CmpPart) * app::kCmpBlocks));
  hipEvent_t ev[4];
  for (auto& e : ev) APP_HIP(hipEventCreate(&e));

  hipLaunchKernelGGL(app::fill_phi, dim3(app::grid_for(nnz)), dim3(256), 0, s, Av, nnz, phi, seed ^ 0xA1);
  hipLaunchKernelGGL(app::fill_phi, dim3(app::grid_for((size_t)N * nrhs)), dim3(256), 0, s, X, (size_t)N * nrhs, phi, seed ^ 0xB2);
  if (nb) hipLaunchKernelGGL(block_scale_kernel, dim3(std::min(nb, 65535)), dim3(128), 0, s, Av, d_voff, d_vlen, d_bscale, nb);
  hipLaunchKernelGGL(app::abs_values, dim3(app::grid_for(nnz)), dim3(256), 0, s, Av, aAv, nnz);
  hipLaunchKernelGGL(app::abs_values, dim3(app::grid_for((size_t)N * nrhs)), dim3(256), 0, s, X, aX, (size_t)N * nrhs);
  APP_HIP(hipStreamSynchronize(s));

  // descriptors of one formulation over (A values, X, outputs)
  auto make_problems = [&](bool blk, const double* Ap, const double* Xs, double* Tout, double* Yout) {
    std::vector<ggemm_problem_t> v;
    if (blk) {
      v.reserve(nb);
      for (int I = 0; I < atoms; ++I)
        for (int b = rowptr[I]; b < rowptr[I + 1]; ++b)
          v.push_back(ggemm_problem_t{bsz[I], nrhs, bsz[bcol[b]], Ap + voff[b], bsz[I], Xs + rstart[bcol[b]], N,
                                      Tout + toff[b], bsz[I], 1.0, 0.0});
    } else {
      v.reserve(atoms);
      for (int I = 0; I < atoms; ++I)
        v.push_back(ggemm_problem_t{bsz[I], nrhs, Kr[I], Ap + voff[rowptr[I]], bsz[I], Xp + poff[I], std::max(Kr[I], 1),
                                    Yout + rstart[I], N, 1.0, 0.0});
    }
    return v;
  };

  FILE* fo = std::fopen(csv.c_str(), append ? "a" : "w");
  if (!fo) { std::perror(csv.c_str()); return 1; }
  std::fseek(fo, 0, SEEK_END);
  if (std::ftell(fo) == 0)
    std::fprintf(fo, "app,mode,path,atoms,basis,N,nrhs,blocks,G,nnz,max_K,cutoff,density,phi,seed,num_moduli_cfg,flops,"
                     "total_ms_median,total_ms_mean,wall_ms_median,pre_ms,gemm_ms,post_ms,gemm_pct,eff_GFLOPS,launches,"
                     "num_fallback,moduli_min,moduli_max,err_cw,err_over_bound,rel_fro,nonfinite,reps,gpu,env,status\n");
  const double bnd = 2.0 * app::gamma((long long)maxK + maxRow + 1);

  for (const auto& mode : modes) {
    const bool blk = mode == "block";
    // the panel gather reads X for the values and |X| for the denominator: one source per step
    auto step = [&](ggemm_handle_t h, int p, const ggemm_config_t& cfg, const std::vector<ggemm_problem_t>& pr,
                    const double* Xs, double* Yout, hipEvent_t* e, ggemm_stats_t* st) -> int {
      if (e) APP_HIP(hipEventRecord(e[0], s));
      if (!blk && prow)
        hipLaunchKernelGGL(gather_panel_kernel, dim3(app::grid_for(nXp)), dim3(256), 0, s, N, nrhs, prow, d_qb, d_qp,
                           d_qs, d_poff, d_Kr, Xs, Xp);
      if (e) APP_HIP(hipEventRecord(e[1], s));
      const int rc = ggemm_grouped_dgemm(h, (ggemm_path_t)p, &cfg, pr.data(), (int)pr.size(), st);
      if (e) APP_HIP(hipEventRecord(e[2], s));
      if (blk)
        hipLaunchKernelGGL(reduce_kernel, dim3(app::grid_for((size_t)N * nrhs)), dim3(256), 0, s, N, nrhs, d_row_block,
                           d_row_loc, d_bsz, d_rowptr, d_toff, Tb, Yout);
      if (e) APP_HIP(hipEventRecord(e[3], s));
      return rc;
    };
    const auto probs = make_problems(blk, Av, X, Tb, Y);
    const auto aprobs = make_problems(blk, aAv, aX, Tb, den);
    const int G = (int)probs.size();
    const size_t mA = nnz + 1, mB = nXp + 1, mC = (blk ? nT : (size_t)N * nrhs) + 1;
    // the workspace is sized for the smallest k (Kp = round_up(k, 32) inflates small blocks)
    int min_k = 32;
    for (const auto& pr : probs) min_k = std::max(1, std::min(min_k, pr.k));
    auto create = [&](ggemm_handle_t* h) { return ggemm_create_ex(h, std::max(G, 1), mA, mB, mC, s, min_k); };

    int ref_ok = 0;
    {
      ggemm_handle_t h = nullptr;
      ggemm_stats_t st;
      const ggemm_config_t cfg = app::config_for(GGEMM_PATH_NATIVE_LOOP, 0);
      if (create(&h) == 0 && h) {
        int rc = step(h, GGEMM_PATH_NATIVE_LOOP, cfg, probs, X, Y, nullptr, &st);
        APP_HIP(hipMemcpyAsync(Yref, Y, (size_t)N * nrhs * sizeof(double), hipMemcpyDeviceToDevice, s));
        rc |= step(h, GGEMM_PATH_NATIVE_LOOP, cfg, aprobs, aX, den, nullptr, &st);
        APP_HIP(hipStreamSynchronize(s));
        ref_ok = rc == 0;
        ggemm_destroy(h);
      }
    }
    if (!ref_ok) std::fprintf(stderr, "warning: [%s] the NATIVE_LOOP reference failed; error columns are NaN\n", mode.c_str());

    for (int p : paths) {
      const ggemm_config_t cfg = app::config_for(p, nmod);
      ggemm_handle_t h = nullptr;
      ggemm_stats_t st{};
      const char* status = "ok";
      if (create(&h) != 0 || !h) status = "create_failed";
      int rc = 0;
      for (int r = 0; h && rc == 0 && r < warmup; ++r) rc = step(h, p, cfg, probs, X, Y, nullptr, &st);
      if (h) APP_HIP(hipStreamSynchronize(s));
      std::vector<double> tot, wall, sp[3];
      for (int r = 0; h && rc == 0 && r < reps; ++r) {
        const double w = app::wall_ms([&] {
          rc = step(h, p, cfg, probs, X, Y, ev, &st);
          APP_HIP(hipEventSynchronize(ev[3]));
        });
        if (rc != 0) break;
        float ms;
        APP_HIP(hipEventElapsedTime(&ms, ev[0], ev[3]));
        tot.push_back(ms);
        for (int k = 0; k < 3; ++k) {
          APP_HIP(hipEventElapsedTime(&ms, ev[k], ev[k + 1]));
          sp[k].push_back(ms);
        }
        wall.push_back(w);
      }
      if (h && rc != 0) status = "call_failed";
      if (hipGetLastError() != hipSuccess) status = "hip_error";
      app::Err er;
      if (h && rc == 0 && ref_ok) {
        hipLaunchKernelGGL(app::fill_value, dim3(app::grid_for((size_t)N * nrhs)), dim3(256), 0, s, Y, (size_t)N * nrhs, (double)NAN);
        if (blk) hipLaunchKernelGGL(app::fill_value, dim3(app::grid_for(nT)), dim3(256), 0, s, Tb, nT, (double)NAN);
        if (step(h, p, cfg, probs, X, Y, nullptr, &st) == 0) er = app::compare(Y, Yref, den, (size_t)N * nrhs, part, s);
        else status = "check_failed";
      }
      const double tmed = app::median(tot), tmean = app::mean(tot);
      double sm[3];
      for (int k = 0; k < 3; ++k) sm[k] = app::mean(sp[k]);
      std::fprintf(fo, "block_sparse,%s,%s,%d,%s,%d,%d,%d,%d,%zu,%d,%.2f,%.3f,%.2f,%llu,%d,%.6e,%.6f,%.6f,%.6f,%.6f,%.6f,"
                       "%.6f,%.3f,%.3f,%d,%d,%d,%d,%.6e,%.6e,%.6e,%llu,%d,%s,%s,%s\n",
                   mode.c_str(), app::path_name(p), atoms, basis.c_str(), N, nrhs, nb, G, nnz, maxK, cutoff, rho, phi,
                   (unsigned long long)seed, nmod, flops, tmed, tmean, app::median(wall), sm[0], sm[1], sm[2],
                   100.0 * sm[1] / tmean, flops / (tmed * 1e-3) / 1e9, st.kernel_launches, st.num_fallback,
                   st.moduli_min, st.moduli_max, er.cw, er.cw / bnd, er.rel_fro, er.bad, (int)tot.size(), gpu.c_str(),
                   envs.c_str(), status);
      std::fflush(fo);
      std::fprintf(stderr, "[%s] %-18s G=%-6d total %9.3f ms (%8.1f GFLOP/s) gemm %4.1f%% launches %d fb %d "
                           "err %.2e (%.2g x bound) %s\n",
                   mode.c_str(), app::path_name(p), G, tmed, flops / (tmed * 1e-3) / 1e9, 100.0 * sm[1] / tmean,
                   st.kernel_launches, st.num_fallback, er.cw, er.cw / bnd, status);
      if (h) ggemm_destroy(h);
      if (!std::strcmp(status, "hip_error")) { std::fclose(fo); return 1; }
    }
  }
  std::fclose(fo);
  return 0;
}
