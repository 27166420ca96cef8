/* oz2_i8dot.c -- exact int8 dot products for the oracle's integer GEMM (test infrastructure only).
 *
 * Plain integer arithmetic with AVX2 (the x86-64-v3 floor of the hosts this runs on): int8 values
 * widened to int16, products summed pairwise into int32 lanes (vpmaddwd: |a b + c d| <= 2^15).
 * Every sum of kp <= 131040 products is exact in any order; chunks of at most 65536 products are
 * summed in int32 lanes (|lane| <= 2^15 * 65536 / 16 = 2^27), the chunks in int64. */
#include <immintrin.h>
#include <stdint.h>

#include "oz2_oracle.h"

static inline __m256i widen16(const int8_t* p) { return _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)p)); }

static inline int64_t hsum(__m256i v) {
  __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4e));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xb1));
  return (int64_t)_mm_cvtsi128_si32(s);
}

/* dots of row a with rows b[0..R-1] over n products (n <= 65536), added to out */
static inline void dots_chunk(const int8_t* a, const int8_t* const* b, int R, int n, int64_t* out) {
  __m256i acc[4] = {_mm256_setzero_si256(), _mm256_setzero_si256(), _mm256_setzero_si256(), _mm256_setzero_si256()};
  int q = 0;
  for (; q + 16 <= n; q += 16) {
    const __m256i va = widen16(a + q);
    for (int r = 0; r < R; ++r) acc[r] = _mm256_add_epi32(acc[r], _mm256_madd_epi16(va, widen16(b[r] + q)));
  }
  for (int r = 0; r < R; ++r) {
    int64_t s = hsum(acc[r]);
    for (int t = q; t < n; ++t) s += (int32_t)a[t] * (int32_t)b[r][t];
    out[r] += s;
  }
}

int64_t oz2o_dot_i8(const int8_t* a, const int8_t* b, int n) {
  int64_t s = 0;
  for (int q0 = 0; q0 < n; q0 += 65536) {
    const int8_t* bb[1] = {b + q0};
    dots_chunk(a + q0, bb, 1, n - q0 < 65536 ? n - q0 : 65536, &s);
  }
  return s;
}

void oz2o_dot4_i8(const int8_t* a, const int8_t* b0, const int8_t* b1, const int8_t* b2, const int8_t* b3, int n,
                  int64_t* out) {
  out[0] = out[1] = out[2] = out[3] = 0;
  for (int q0 = 0; q0 < n; q0 += 65536) {
    const int8_t* bb[4] = {b0 + q0, b1 + q0, b2 + q0, b3 + q0};
    dots_chunk(a + q0, bb, 4, n - q0 < 65536 ? n - q0 : 65536, out);
  }
}
