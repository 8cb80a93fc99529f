/* The reference's AVX2 kernels for the CPU baseline (test infrastructure
 * and the reported CPU baseline only; nothing in c2slm_amd/ links it).
 *
 * A C restatement, with x86 intrinsics, of the AVX2 branches of
 * internal/simd that the reference runs on an AVX2 host:
 *   Q4_K x Q8_K  c2_tensor_dot_q4_k_q8_k_gen.go:54-90 (per pair, the low and
 *                high nibbles VPMADDUBSW the 32 Q8_K quants, VPMADDWD by 1,
 *                eight int32 lanes summed; the float fold of :85);
 *   Q6_K x Q8_K  c2_tensor_gemv2_q6_k_q8_k_gen.go:89-214 (per half and
 *                quarter, the 6-bit quants built from ql / qh with byte
 *                masks and 16-bit shifts, VPMADDUBSW, VPMADDWD by 1, lanes
 *                0-3 and 4-7 the two 16-element sums; isum in int32);
 *   Q8_0 x f32   c2_tensor_dot_q8_0_gen.go:80-103 (four 8-lane products of
 *                the sign-extended quants by x, (p0+p1)+(p2+p3), times d,
 *                added to an 8-lane accumulator; lanes summed left to right).
 * Every integer is the scalar oracle's and every float operation is in the
 * same order, so results equal orc_dot_q4k_q8k / orc_dot_q6k_q8k /
 * orc_dot_q8_0 bit for bit (tests/test_oracle.py checks it); only the
 * speed differs.  Compiled with the oracle (-mavx2, -ffp-contract=off). */
#include <immintrin.h>
#include <stdint.h>
#include <string.h>

float orc_fp16_simd(uint16_t h);

#define QK_K 256
#define BS_Q4K 144
#define BS_Q6K 210
#define BS_Q8K 292
#define BS_Q8_0 34

static inline float rdf32(const uint8_t* p) { float f; memcpy(&f, p, 4); return f; }
static inline uint16_t rdu16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline int16_t rdi16(const uint8_t* p) { return (int16_t)rdu16(p); }

/* eight int32 lanes summed (integer: any order) */
static inline int32_t hsum8(__m256i v) {
  __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4e));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xb1));
  return _mm_cvtsi128_si32(s);
}
static inline int32_t hsum4(__m128i s) {
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4e));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xb1));
  return _mm_cvtsi128_si32(s);
}

float orc_avx2_dot_q4k_q8k(const uint8_t* w, const uint8_t* q8k, int cols) {
  const int nb = cols / QK_K;
  const __m256i m4 = _mm256_set1_epi8(15), ones = _mm256_set1_epi16(1);
  float acc = 0.0f;
  for (int b = 0; b < nb; ++b) {
    const uint8_t* wb = w + (long)b * BS_Q4K;
    const uint8_t* qb = q8k + (long)b * BS_Q8K;
    const float q8d = rdf32(qb);
    const float dW = orc_fp16_simd(rdu16(wb)) * q8d;
    const float mW = orc_fp16_simd(rdu16(wb + 2)) * q8d;
    const uint8_t* s = wb + 4;
    uint8_t sc[8], m[8];
    for (int j = 0; j < 4; ++j) { /* c2_tensor_dot_q4_k_q8_k_gen.go:47-61 */
      sc[j] = s[j] & 63;
      m[j] = s[j + 4] & 63;
      sc[j + 4] = (uint8_t)((s[j + 8] & 15) | ((s[j] >> 6) << 4));
      m[j + 4] = (uint8_t)((s[j + 8] >> 4) | ((s[j + 4] >> 6) << 4));
    }
    const uint8_t* bs = qb + 260;
    for (int p = 0; p < 4; ++p) {
      const __m256i qs = _mm256_loadu_si256((const __m256i*)(wb + 16 + 32 * p));
      const __m256i x_lo = _mm256_loadu_si256((const __m256i*)(qb + 4 + 64 * p));
      const __m256i x_hi = _mm256_loadu_si256((const __m256i*)(qb + 4 + 64 * p + 32));
      const __m256i lo = _mm256_and_si256(qs, m4);
      const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(qs, 4), m4);
      const int32_t s_lo = hsum8(_mm256_madd_epi16(_mm256_maddubs_epi16(lo, x_lo), ones));
      const int32_t s_hi = hsum8(_mm256_madd_epi16(_mm256_maddubs_epi16(hi, x_hi), ones));
      const float bA = (float)((int32_t)rdi16(bs + 2 * (4 * p)) + (int32_t)rdi16(bs + 2 * (4 * p + 1)));
      const float bB = (float)((int32_t)rdi16(bs + 2 * (4 * p + 2)) + (int32_t)rdi16(bs + 2 * (4 * p + 3)));
      const float t = (((float)s_lo * (dW * (float)sc[2 * p])) - (bA * (mW * (float)m[2 * p]))) +
                      (((float)s_hi * (dW * (float)sc[2 * p + 1])) - (bB * (mW * (float)m[2 * p + 1])));
      acc += t;
    }
  }
  return acc;
}

int32_t orc_avx2_q6k_block_isum(const uint8_t* wb, const uint8_t* qb) {
  const __m256i m4 = _mm256_set1_epi8(15), m2 = _mm256_set1_epi8(3), ones = _mm256_set1_epi16(1);
  const int8_t* sc = (const int8_t*)(wb + 192);
  const uint8_t* bs = qb + 260;
  int32_t isum = 0;
  for (int n = 0; n < 2; ++n) {
    const __m256i qh = _mm256_loadu_si256((const __m256i*)(wb + 128 + 32 * n));
    const __m256i ql0 = _mm256_loadu_si256((const __m256i*)(wb + 64 * n));
    const __m256i ql1 = _mm256_loadu_si256((const __m256i*)(wb + 64 * n + 32));
    for (int k = 0; k < 4; ++k) {
      const __m256i ql = (k & 1) ? ql1 : ql0;
      const __m256i lo = (k < 2) ? _mm256_and_si256(ql, m4) : _mm256_and_si256(_mm256_srli_epi16(ql, 4), m4);
      __m256i h = qh;
      if (k == 1) h = _mm256_srli_epi16(qh, 2);
      if (k == 2) h = _mm256_srli_epi16(qh, 4);
      if (k == 3) h = _mm256_srli_epi16(qh, 6);
      const __m256i q6 = _mm256_or_si256(lo, _mm256_slli_epi16(_mm256_and_si256(h, m2), 4));
      const __m256i x = _mm256_loadu_si256((const __m256i*)(qb + 4 + 128 * n + 32 * k));
      const __m256i d = _mm256_madd_epi16(_mm256_maddubs_epi16(q6, x), ones);
      const int32_t sa = hsum4(_mm256_castsi256_si128(d));
      const int32_t sb = hsum4(_mm256_extracti128_si256(d, 1));
      const int32_t ba = 32 * (int32_t)rdi16(bs + 2 * (8 * n + 2 * k));
      const int32_t bb = 32 * (int32_t)rdi16(bs + 2 * (8 * n + 2 * k + 1));
      isum += ((sa - ba) * (int32_t)sc[8 * n + 2 * k]) + ((sb - bb) * (int32_t)sc[8 * n + 2 * k + 1]);
    }
  }
  return isum;
}

float orc_avx2_dot_q6k_q8k(const uint8_t* w, const uint8_t* q8k, int cols) {
  const int nb = cols / QK_K;
  float acc = 0.0f;
  for (int b = 0; b < nb; ++b) {
    const uint8_t* wb = w + (long)b * BS_Q6K;
    const uint8_t* qb = q8k + (long)b * BS_Q8K;
    const float q8d = rdf32(qb);
    const float d = orc_fp16_simd(rdu16(wb + 208));
    acc += (float)orc_avx2_q6k_block_isum(wb, qb) * (d * q8d);
  }
  return acc;
}

float orc_avx2_dot_q8_0(const uint8_t* w, const float* x, int cols) {
  const int nb = cols / 32;
  __m256 acc = _mm256_setzero_ps();
  for (int b = 0; b < nb; ++b) {
    const uint8_t* blk = w + (long)b * BS_Q8_0;
    const float* xb = x + 32 * b;
    const __m256 d = _mm256_set1_ps(orc_fp16_simd(rdu16(blk)));
    const __m128i a = _mm_loadu_si128((const __m128i*)(blk + 2));
    const __m128i c = _mm_loadu_si128((const __m128i*)(blk + 18));
    const __m256 p0 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(a)), _mm256_loadu_ps(xb));
    const __m256 p1 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(a, 8))), _mm256_loadu_ps(xb + 8));
    const __m256 p2 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(c)), _mm256_loadu_ps(xb + 16));
    const __m256 p3 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(c, 8))), _mm256_loadu_ps(xb + 24));
    acc = _mm256_add_ps(acc, _mm256_mul_ps(_mm256_add_ps(_mm256_add_ps(p0, p1), _mm256_add_ps(p2, p3)), d));
  }
  float l[8];
  _mm256_storeu_ps(l, acc);
  return ((((((l[0] + l[1]) + l[2]) + l[3]) + l[4]) + l[5]) + l[6]) + l[7];
}
