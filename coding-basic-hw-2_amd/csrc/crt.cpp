// crt.cpp -- CRT constants (host), per-device context, a-priori error bound and moduli choice,
// device counters.
//
// The quantities follow the reference's src/moduli.h:8-21 and :124-181 (moduli set, M_l split
// into s1 + s2 2^-18 against u1 = 2^sh, P1/P2, T_N) and src/ozaki2_numerics.cu:639-693 (bound,
// choice of N, counters).  The big-integer arithmetic here is this library's own 64-bit-limb
// code; only the conversion of P to double keeps the reference's exact operation order (Horner
// over 32-bit limbs in 80-bit long double) because T_N, and with it every shift, depends on it
// to the last bit.
#include <cmath>
#include <cstring>
#include <mutex>

#include "common.hpp"

namespace ggemm {
namespace {

// src/moduli.h:39-41
constexpr int kModuli[kMaxModuli] = {256, 255, 253, 251, 247, 239, 233, 229, 227, 223,
                                     217, 211, 199, 197, 193, 191, 181, 179, 173, 167};

// Unsigned integer below 2^192 as three 64-bit limbs (P_20 < 2^155).
struct U192 {
  uint64_t w[3] = {0, 0, 0};
};
U192 mul_small(U192 a, uint32_t m) {
  unsigned __int128 c = 0;
  for (auto& x : a.w) {
    c += (unsigned __int128)x * m;
    x = (uint64_t)c;
    c >>= 64;
  }
  return a;
}
uint32_t divmod_small(U192 a, uint32_t d, U192* q) {
  unsigned __int128 r = 0;
  U192 out;
  for (int i = 2; i >= 0; --i) {
    unsigned __int128 cur = (r << 64) | a.w[i];
    out.w[i] = (uint64_t)(cur / d);
    r = cur % d;
  }
  if (q) *q = out;
  return (uint32_t)r;
}
int bit_length(const U192& a) {
  for (int i = 2; i >= 0; --i)
    if (a.w[i]) return 64 * i + 64 - __builtin_clzll(a.w[i]);
  return 0;
}
int test_bit(const U192& a, int i) { return (i < 0 || i >= 192) ? 0 : (int)((a.w[i / 64] >> (i % 64)) & 1); }
// a >> s for s >= 0, a << -s for s < 0 (bits beyond 192 dropped)
U192 shift(const U192& a, int s) {
  U192 r;
  for (int i = 0; i < 192; ++i)
    if (test_bit(a, i)) {
      const int j = i - s;
      if (j >= 0 && j < 192) r.w[j / 64] |= 1ull << (j % 64);
    }
  return r;
}
U192 low_bits(const U192& a, int s) {
  U192 r;
  for (int i = 0; i < s && i < 192; ++i)
    if (test_bit(a, i)) r.w[i / 64] |= 1ull << (i % 64);
  return r;
}
// P as a double: Horner over 32-bit limbs, most significant first, in long double.
double to_double(const U192& a) {
  long double v = 0.0L;
  for (int i = 5; i >= 0; --i) {
    const uint32_t limb = (uint32_t)(a.w[i / 2] >> (32 * (i % 2)));
    v = v * 4294967296.0L + (long double)limb;
  }
  return (double)v;
}

// r in [0, p) as the byte of its symmetric representative in [-floor(p/2), p - 1 - floor(p/2)]
uint32_t sym_byte(uint32_t r, uint32_t p) {
  const int v = (int)r > (int)(p - 1 - p / 2) ? (int)r - (int)p : (int)r;
  return (uint32_t)v & 0xffu;
}

// the four weight words of CrtTables::wb for modulus p and multiplier q
void digit_weights(uint32_t p, uint32_t q, uint32_t* w) {
  uint32_t e[12];   // q 2^(8 i) mod p
  e[0] = q % p;
  for (int i = 1; i < 12; ++i) e[i] = (e[i - 1] * 256u) % p;
  for (int b = 0; b < 4; ++b) {
    w[0] |= e[b] << (8 * b);
    w[1] |= e[4 + b] << (8 * b);
    w[2] |= sym_byte(e[4 + b], p) << (8 * b);
    w[3] |= sym_byte(e[8 + b], p) << (8 * b);
  }
}

int build(CrtTables* t) {
  std::memset(t, 0, sizeof *t);
  for (int a = 0; a < kMaxModuli; ++a)
    for (int b = a + 1; b < kMaxModuli; ++b) {
      int x = kModuli[a], y = kModuli[b];
      while (y) { const int r = x % y; x = y; y = r; }
      if (x != 1) return 1;
    }
  for (int l = 0; l < kMaxModuli; ++l) {
    const uint32_t p = (uint32_t)kModuli[l];
    t->p[l] = (int32_t)p;
    t->magic[l] = (uint32_t)((1ull << 32) / p);
    t->ipf[l] = (float)(1.0 / (double)p);
    t->cf[l] = (float)(((double)(p / 2) + 0.5) / (double)p + 2048.0);
    digit_weights(p, 1u, t->wb[0][l]);
  }
  for (int N = 1; N <= kMaxModuli; ++N) {
    U192 P;
    P.w[0] = 1;
    for (int l = 0; l < N; ++l) P = mul_small(P, (uint32_t)kModuli[l]);
    U192 M[kMaxModuli];
    int top = 0;
    for (int l = 0; l < N; ++l) {
      const uint32_t p = (uint32_t)kModuli[l];
      if (divmod_small(P, p, &M[l]) != 0) return 3;
      const uint32_t mr = divmod_small(M[l], p, nullptr);
      int inv = -1;
      for (uint32_t x = 0; x < p; ++x)
        if ((mr * x) % p == 1 % p) { inv = (int)x; break; }
      if (inv < 0) return 4;
      t->qinv[N][l] = inv;
      digit_weights(p, (uint32_t)inv, t->wb[N][l]);
      top = std::max(top, bit_length(M[l]));
    }
    const int sh = top - 49;   // u1 = 2^sh keeps every M_l / u1 below 2^49
    t->log2_u1[N] = sh;
    for (int l = 0; l < N; ++l) {
      t->s1[N][l] = shift(M[l], sh).w[0];
      uint64_t s2 = 0;
      if (sh > 0) {
        const U192 frac = low_bits(M[l], sh);
        if (sh >= kS2Bits)   // round half up to 18 fractional bits
          s2 = shift(frac, sh - kS2Bits).w[0] + (uint64_t)test_bit(frac, sh - kS2Bits - 1);
        else
          s2 = frac.w[0] << (kS2Bits - sh);
      }
      if (s2 > (1u << kS2Bits) || t->s1[N][l] >= (1ull << 49)) return 5;
      t->s2[N][l] = (uint32_t)s2;
    }
    const U192 P1 = shift(P, sh);
    if (bit_length(P1) > 57) return 7;
    t->P1[N] = (int64_t)P1.w[0];
    t->P2[N] = sh > 0 ? std::ldexp(to_double(low_bits(P, sh)), -sh) : 0.0;
    t->inv_Pu[N] = 1.0 / ((double)t->P1[N] + t->P2[N]);
    const double Pd = to_double(P);
    t->log2P[N] = std::log2(Pd);
    t->T[N] = std::sqrt(Pd * 0.5 * (1.0 - std::ldexp(1.0, -20))) * (1.0 - std::ldexp(1.0, -40));
  }
  return 0;
}

std::mutex g_ctx_mu;
DevCtx g_ctx_store[64];
bool g_ctx_ready[64] = {};

}  // namespace

const CrtTables* host_tables() {
  static CrtTables tab;
  static const int st = build(&tab);
  return st == 0 ? &tab : nullptr;
}

// The tables and counters are device globals (device_state); the first use on a device copies the
// host-built tables there (a plain copy: nothing is allocated on the device).
DevCtx* dev_ctx() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lk(g_ctx_mu);
  DevCtx* c = &g_ctx_store[dev];
  if (g_ctx_ready[dev]) return c;
  const CrtTables* h = host_tables();
  if (!h) return nullptr;
  c->device = dev;
  if (hipDeviceGetAttribute(&c->num_cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      c->num_cus <= 0)
    c->num_cus = 256;
  void* tab = nullptr;
  void* cnt = nullptr;
  if (device_state(&tab, &cnt) != 0 || hipMemcpy(tab, h, sizeof(CrtTables), hipMemcpyHostToDevice) != hipSuccess)
    return nullptr;
  c->tab = static_cast<const CrtTables*>(tab);
  c->counters = static_cast<unsigned long long*>(cnt);
  g_ctx_ready[dev] = true;
  return c;
}

}  // namespace ggemm

using namespace ggemm;

extern "C" int oz2_init_constants(void) { return dev_ctx() ? 0 : 1; }

// src/ozaki2_numerics.cu:639-650: eps_N(k) = 4 sqrt(k)/T + 4k/T^2 + 4 u1 (N 255 2^-19 + 2^-10)/T^2 + u
extern "C" double oz2_error_bound(int k, int num_moduli) {
  const CrtTables* t = host_tables();
  if (!t || num_moduli < 1 || num_moduli > kMaxModuli || k < 0) return INFINITY;
  const double T = t->T[num_moduli];
  const double T2 = T * T;
  const double kk = (double)k;
  const double u = std::ldexp(1.0, -53);
  const double u1 = std::ldexp(1.0, t->log2_u1[num_moduli]);
  return 4.0 * std::sqrt(kk) / T + 4.0 * kk / T2 +
         4.0 * u1 * (num_moduli * 255.0 * std::ldexp(1.0, -19) + std::ldexp(1.0, -10)) / T2 + u;
}

// src/ozaki2_numerics.cu:652-657
extern "C" int oz2_choose_num_moduli(int k, double target_rel_err) {
  if (k < 0 || k > OZ2_MAX_K) return -1;
  for (int N = 2; N <= kMaxModuli; ++N)
    if (oz2_error_bound(k, N) <= target_rel_err) return N;
  return -1;
}

// src/ozaki2_numerics.cu:665-673
extern "C" int oz2_choose_num_moduli_cw(int k, double rho_budget) {
  if (k < 0 || k > OZ2_MAX_K) return -1;
  if (rho_budget < 1.0) rho_budget = 1.0;
  const double u = std::ldexp(1.0, -53);
  const double budget = 0.5 * (k > 2 ? (double)(k - 2) : 1.0) * u;
  for (int N = 2; N <= kMaxModuli; ++N)
    if ((oz2_error_bound(k, N) - u) * rho_budget <= budget) return N;
  return kMaxModuli;
}

// src/ozaki2_numerics.cu:675-693
extern "C" int oz2_read_counters(oz2_counters* out, int reset, hipStream_t s) {
  DevCtx* c = dev_ctx();
  if (!c) return 1;
  // the slots of every counter, summed (the kernels spread their atomics over them)
  static thread_local unsigned long long h[kCounterSlots * kCounterStride];
  if (out && hipMemcpyAsync(h, c->counters, sizeof h, hipMemcpyDeviceToHost, s) != hipSuccess) return 2;
  if (reset && hipMemsetAsync(c->counters, 0, sizeof h, s) != hipSuccess) return 4;
  if (out) {
    if (hipStreamSynchronize(s) != hipSuccess) return 3;
    unsigned long long v[4] = {0, 0, 0, 0};
    for (int sl = 0; sl < kCounterSlots; ++sl)
      for (int q = 0; q < 4; ++q) v[q] += h[sl * kCounterStride + q];
    out->nonfinite_vectors = v[0];
    out->uncertified = v[1];
    out->repaired = v[2];
    out->safety_fallback = v[3];
  }
  return 0;
}
