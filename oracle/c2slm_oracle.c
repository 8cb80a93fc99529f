/*
 * c2slm decode-path oracle: a plain-C restatement of the reference's CPU
 * arithmetic, statement by statement, with the float operation order kept.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or the reported CPU baseline.  The product (c2slm_amd/) never links it.
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off: every a*b+c below is
 * two roundings unless written as fmaf(), exactly like the reference's
 * GOAMD64=v1 Go build; fmaf() appears only where the reference calls
 * archsimd MulAdd).
 *
 * Each function names the reference file:line it restates.  What pins it
 * (tests/test_oracle.py):
 *   fp16 decode        exhaustive 65,536 values vs IEEE; tensor/ops_test.go cases
 *   Q8_K quantiser     known-answer fixture (c2_tensor_dot_q4_k_q8_k_test.go:92-94),
 *                      invariants, floor/zero-block, Go NaN conversion
 *   Q4_K/Q6_K sums     the reference's own C dequant oracles (oracle/_ref),
 *                      brute force over unpacked nibbles
 *   Q6_K dot           golden values c2_tensor_gemv2_q6_k_q8_k_test.go:55-56
 *   Q4_K/Q8_0 fold     float64 dequant, order known answers, unit vectors
 *   RMSNorm/RoPE/      reference cases, float64, invariants
 *   Softmax
 *   attention          textbook float64 attention, FMA-order known answers
 *   SwiGLU             c2_tensor_swiglu_test.go:34 precision, extremes
 *   penalty/argmax     brute force, ties, NaN at id 0
 *   forward / ingest / float64 Qwen2 decoder written from the model's
 *   logits / generate  mathematics (tests/qwen2_f64.py, tests/test_oracle_model.py):
 *                      normX, K/V and logits within 1e-3 (seen: 1e-6), the
 *                      greedy stream wherever decided; planted mistakes are
 *                      caught (tests/test_oracle_mutants.py)
 *   f64 exp / pow /    every input whose f32 result two <=1-ulp libraries could
 *   cos / sin          round differently is listed (tests/golden/f32_stability.json):
 *                      one exp input of 1.1e9; RoPE entries only from position 2,387
 * Parity unpinned (needs the Go toolchain, absent here): the f32 results of
 * Go's math.Exp at t = -14.56709 (0xc16912cd) and of Go's Pow/Cos/Sin at the
 * listed RoPE entries (positions >= 2,387), archsimd ConvertToInt32 in SwiGLU
 * (truncation assumed; the reference pins it to 1e-4), and the reference's
 * own bits of the end-to-end stream beyond these pins.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK_K 256
#define BS_Q4K 144
#define BS_Q6K 210
#define BS_Q8K 292
#define QK8_0 32
#define BS_Q8_0 34
#define QK5_0 32
#define BS_Q5_0 22

enum { T_F32 = 0, T_Q5_0 = 6, T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14 };

static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline int16_t rd_i16(const uint8_t* p) { return (int16_t)(uint16_t)(p[0] | (p[1] << 8)); }
static inline uint16_t rd_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline float rd_f32(const uint8_t* p) {
  return bits_f32((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24));
}

/* ---------------------------------------------------------------- A6 fp16 */

/* internal/simd/c2_tensor_dot_q8_0_gen.go:24-66 (LUT used by every simd
 * kernel): +0 for both zeros, subnormals normalised, Inf/NaN keep payload.
 * The exponent is uint32 and wraps while normalising, as in Go. */
float orc_fp16_simd(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t e = (h >> 10) & 31u;
  uint32_t m = h & 0x3ffu;
  if (e == 0) {
    if (m == 0) return 0.0f;
    for (;;) {
      if (m & 0x400u) break;
      m <<= 1;
      e--;
    }
    e++;
    m &= 0x3ffu;
    e = (e + 0x70u) << 23;
    m <<= 13;
    return bits_f32(sign | e | m);
  }
  if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
  return bits_f32(sign | ((e + 0x70u) << 23) | (m << 13));
}

/* tensor/fp16.go:16-50 (tensor.FP16ToF32, used by DequantizeRowQ8_0 and so by
 * EmbedToken): identical except that -0 keeps its sign (fp16.go:26-28). */
float orc_fp16_tensor(uint16_t h) {
  if ((h & 0x7fffu) == 0) return bits_f32((uint32_t)(h >> 15) << 31);
  return orc_fp16_simd(h);
}

/* bit patterns, for callers whose float return path would quiet a NaN */
uint32_t orc_fp16_simd_bits(uint16_t h) { return f32_bits(orc_fp16_simd(h)); }
uint32_t orc_fp16_tensor_bits(uint16_t h) { return f32_bits(orc_fp16_tensor(h)); }

/* Go's int(float32) on amd64 is CVTTSS2SQ: truncation toward zero, and
 * 0x8000000000000000 for NaN or out-of-range values. */
static inline int64_t go_f32_to_int(float t) {
  if (!(t >= -9223372036854775808.0f && t < 9223372036854775808.0f)) return INT64_MIN;
  return (int64_t)t;
}

/* archsimd Float32x8.ConvertToInt32 is VCVTTPS2DQ: truncation, and
 * 0x80000000 for NaN or out-of-range lanes. */
static inline int32_t x86_cvtt_i32(float t) {
  if (!(t >= -2147483648.0f && t < 2147483648.0f)) return INT32_MIN;
  return (int32_t)t;
}

/* ------------------------------------------------------------ A1 Q8_K */

/* internal/simd/c2_quantize_q8_k_gen.go:11-91 (tensor/ops.go:170-172).
 * cols/256 blocks (floor).  y_len is the length of the destination slice:
 * an all-zero block clears y from that block's qs to the end of the slice
 * (gen.go:43-44); later blocks are rewritten afterwards. */
void orc_quantize_row_q8k(const float* x, uint8_t* y, int cols, long y_len) {
  int nb = cols / QK_K;
  for (int b = 0; b < nb; ++b) {
    const float* xb = x + b * QK_K;
    long yo = (long)b * BS_Q8K;
    float amax = 0.0f;
    for (int i = 0; i < QK_K; ++i) {
      float v = xb[i];
      float a = (v < 0.0f) ? -v : v;
      if (a > amax) amax = a;
    }
    if (amax == 0.0f) {
      y[yo] = y[yo + 1] = y[yo + 2] = y[yo + 3] = 0;
      if (y_len > yo + 4) memset(y + yo + 4, 0, (size_t)(y_len - yo - 4));
      continue;
    }
    uint32_t db = f32_bits(amax / 127.0f);
    y[yo] = (uint8_t)(db & 0xff);
    y[yo + 1] = (uint8_t)((db >> 8) & 0xff);
    y[yo + 2] = (uint8_t)((db >> 16) & 0xff);
    y[yo + 3] = (uint8_t)((db >> 24) & 0xff);
    float iscale = 127.0f / amax;
    for (int i = 0; i < QK_K; ++i) {
      float v = xb[i] * iscale;
      float t = (v >= 0.0f) ? (v + 0.5f) : (v - 0.5f);
      int64_t q = go_f32_to_int(t);
      if (q > 127) q = 127;
      if (q < -127) q = -127;
      y[yo + 4 + i] = (uint8_t)(int8_t)q;
    }
    for (int j = 0; j < 16; ++j) {
      int s = 0;
      for (int k = 0; k < 16; ++k) s += (int8_t)y[yo + 4 + j * 16 + k];
      y[yo + 260 + 2 * j] = (uint8_t)(s & 255);
      y[yo + 260 + 2 * j + 1] = (uint8_t)((s >> 8) & 255);
    }
  }
}

/* ------------------------------------------------------- A2 Q4_K x Q8_K */

static inline void q4k_unpack_scales(const uint8_t* s, uint8_t sc[8], uint8_t m[8]) {
  /* c2_tensor_dot_q4_k_q8_k_gen.go:47-61 */
  for (int j = 0; j < 4; ++j) {
    sc[j] = s[j] & 63;
    m[j] = s[j + 4] & 63;
    sc[j + 4] = (uint8_t)((s[j + 8] & 15) | ((s[j] >> 6) << 4));
    m[j + 4] = (uint8_t)((s[j + 8] >> 4) | ((s[j + 4] >> 6) << 4));
  }
}

/* Integer part of one Q4_K super-block against one Q8_K block: the eight
 * 32-element sums s[2p] (low nibbles, q8[64p..]) and s[2p+1] (high nibbles,
 * q8[64p+32..]).  gen.go:62-83 (VPMADDUBSW/VPMADDWD cannot saturate here). */
void orc_q4k_block_isums(const uint8_t* wb, const uint8_t* qb, int32_t s[8]) {
  const uint8_t* qs = wb + 16;
  const int8_t* q8 = (const int8_t*)(qb + 4);
  for (int p = 0; p < 4; ++p) {
    int32_t lo = 0, hi = 0;
    for (int l = 0; l < 32; ++l) {
      uint8_t q = qs[32 * p + l];
      lo += (int32_t)(q & 15) * (int32_t)q8[64 * p + l];
      hi += (int32_t)(q >> 4) * (int32_t)q8[64 * p + 32 + l];
    }
    s[2 * p] = lo;
    s[2 * p + 1] = hi;
  }
}

/* internal/simd/c2_tensor_dot_q4_k_q8_k_gen.go:17-142 (AVX2 and scalar
 * branches accumulate identically); the 2-row kernel
 * c2_tensor_gemv2_q4_k_q8_k_gen.go:9-216 computes each row with the same
 * expression, so one row function serves GEMVQ4_K_Q8_KRange
 * (tensor/ops.go:182-198). */
float orc_dot_q4k_q8k(const uint8_t* w, const uint8_t* q8k, int cols) {
  int nb = cols / QK_K;
  float acc = 0.0f;
  for (int b = 0; b < nb; ++b) {
    const uint8_t* wb = w + (long)b * BS_Q4K;
    const uint8_t* qb = q8k + (long)b * BS_Q8K;
    float q8d = rd_f32(qb);
    float dW = orc_fp16_simd(rd_u16(wb)) * q8d;
    float mW = orc_fp16_simd(rd_u16(wb + 2)) * q8d;
    uint8_t sc[8], m[8];
    q4k_unpack_scales(wb + 4, sc, m);
    int32_t s[8];
    orc_q4k_block_isums(wb, qb, s);
    const uint8_t* bs = qb + 260;
    for (int p = 0; p < 4; ++p) {
      float bA = (float)((int32_t)rd_i16(bs + 2 * (4 * p)) + (int32_t)rd_i16(bs + 2 * (4 * p + 1)));
      float bB = (float)((int32_t)rd_i16(bs + 2 * (4 * p + 2)) + (int32_t)rd_i16(bs + 2 * (4 * p + 3)));
      float t = (((float)s[2 * p] * (dW * (float)sc[2 * p])) - (bA * (mW * (float)m[2 * p]))) +
                (((float)s[2 * p + 1] * (dW * (float)sc[2 * p + 1])) - (bB * (mW * (float)m[2 * p + 1])));
      acc += t;
    }
  }
  return acc;
}

/* ------------------------------------------------------- A3 Q6_K x Q8_K */

static inline uint8_t q6k_quant(const uint8_t* wb, int n, int k, int l) {
  /* c2_tensor_gemv2_q6_k_q8_k_gen.go:243-289 (scalar), :123-139 (AVX2) */
  const uint8_t* ql = wb + 64 * n;
  uint8_t h = wb[128 + 32 * n + l];
  switch (k) {
    case 0: return (uint8_t)((ql[l] & 15) | ((h & 3) << 4));
    case 1: return (uint8_t)((ql[32 + l] & 15) | (((h >> 2) & 3) << 4));
    case 2: return (uint8_t)((ql[l] >> 4) | (((h >> 4) & 3) << 4));
    default: return (uint8_t)((ql[32 + l] >> 4) | (((h >> 6) & 3) << 4));
  }
}

/* Integer super-block sum of gen.go:104-207: Σ_{n,k} (s_a-32·bsum)·sc +
 * (s_b-32·bsum)·sc, with the stored Q8_K bsums. */
int32_t orc_q6k_block_isum(const uint8_t* wb, const uint8_t* qb) {
  const int8_t* q8 = (const int8_t*)(qb + 4);
  const uint8_t* bs = qb + 260;
  const int8_t* sc = (const int8_t*)(wb + 192);
  int32_t isum = 0;
  for (int n = 0; n < 2; ++n) {
    for (int k = 0; k < 4; ++k) {
      int32_t sa = 0, sb = 0;
      for (int l = 0; l < 16; ++l) sa += (int32_t)q6k_quant(wb, n, k, l) * (int32_t)q8[128 * n + 32 * k + l];
      for (int l = 16; l < 32; ++l) sb += (int32_t)q6k_quant(wb, n, k, l) * (int32_t)q8[128 * n + 32 * k + l];
      int32_t ba = 32 * (int32_t)rd_i16(bs + 2 * (8 * n + 2 * k));
      int32_t bb = 32 * (int32_t)rd_i16(bs + 2 * (8 * n + 2 * k + 1));
      isum += ((sa - ba) * (int32_t)sc[8 * n + 2 * k]) + ((sb - bb) * (int32_t)sc[8 * n + 2 * k + 1]);
    }
  }
  return isum;
}

/* One row of internal/simd/c2_tensor_gemv2_q6_k_q8_k_gen.go:14-395:
 * acc += f32(isum)·(f16(d)·q8.d) per super-block (:208-209, :390-391).
 * GEMVQ6_K_Q8_KRange (tensor/ops.go:120-141) pairs rows, or a row with
 * itself at an odd tail; each output is this row function. */
float orc_dot_q6k_q8k(const uint8_t* w, const uint8_t* q8k, int cols) {
  int nb = cols / QK_K;
  float acc = 0.0f;
  for (int b = 0; b < nb; ++b) {
    const uint8_t* wb = w + (long)b * BS_Q6K;
    const uint8_t* qb = q8k + (long)b * BS_Q8K;
    float q8d = rd_f32(qb);
    float d = orc_fp16_simd(rd_u16(wb + 208));
    int32_t isum = orc_q6k_block_isum(wb, qb);
    acc += (float)isum * (d * q8d);
  }
  return acc;
}

/* --------------------------------------------------------- A4 Q8_0 x f32 */

/* internal/simd/c2_tensor_dot_q8_0_gen.go:72-122: eight lane accumulators,
 * acc[j] += ((w[j]x[j] + w[j+8]x[j+8]) + (w[j+16]x[j+16] + w[j+24]x[j+24]))·d
 * (no FMA), then (((((((a0+a1)+a2)+a3)+a4)+a5)+a6)+a7). */
float orc_dot_q8_0(const uint8_t* w, const float* x, int cols) {
  int nb = cols / QK8_0;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int b = 0; b < nb; ++b) {
    const uint8_t* blk = w + (long)b * BS_Q8_0;
    float d = orc_fp16_simd(rd_u16(blk));
    const int8_t* q = (const int8_t*)(blk + 2);
    const float* xb = x + b * QK8_0;
    for (int j = 0; j < 8; ++j) {
      float p0 = (float)q[j] * xb[j];
      float p1 = (float)q[j + 8] * xb[j + 8];
      float p2 = (float)q[j + 16] * xb[j + 16];
      float p3 = (float)q[j + 24] * xb[j + 24];
      acc[j] = acc[j] + ((p0 + p1) + (p2 + p3)) * d;
    }
  }
  return ((((((acc[0] + acc[1]) + acc[2]) + acc[3]) + acc[4]) + acc[5]) + acc[6]) + acc[7];
}

/* Q4_K scales and mins of one super-block (get_scale_min_k4), as the float
 * dot unpacks them: internal/simd/c2_tensor_dot_q4_k_gen.go:28-44. */
static void q4k_scales(const uint8_t* s, uint8_t sc[8], uint8_t mn[8]) {
  for (int i = 0; i < 4; ++i) {
    sc[i] = s[i] & 63;
    mn[i] = s[i + 4] & 63;
    sc[i + 4] = (uint8_t)((s[i + 8] & 15) | ((s[i] >> 6) << 4));
    mn[i + 4] = (uint8_t)((s[i + 8] >> 4) | ((s[i + 4] >> 6) << 4));
  }
}

/* The float-x Q4_K dot (tensor/ops.go:165 DotQ4_K ->
 * internal/simd/c2_tensor_dot_q4_k_gen.go:9-100, AVX2 path): eight lane
 * accumulators; per 32-element sub-block with scale pair (sc, m), lane l
 * forms a = (q[l]x[l] + q[l+8]x[l+8]) + (q[l+16]x[l+16] + q[l+24]x[l+24]),
 * s = (x[l] + x[l+8]) + (x[l+16] + x[l+24]) and adds
 * a·(d·sc) − s·(dmin·m) (products and the difference rounded separately);
 * the low nibbles of the pair's 32 bytes are sub-block 2j, the high ones
 * 2j+1; then (((((((a0+a1)+a2)+a3)+a4)+a5)+a6)+a7). */
float orc_dot_q4k_f32(const uint8_t* w, const float* x, int cols) {
  int nb = cols / QK_K;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int b = 0; b < nb; ++b) {
    const uint8_t* blk = w + (long)b * BS_Q4K;
    float d = orc_fp16_simd(rd_u16(blk));
    float dmin = orc_fp16_simd(rd_u16(blk + 2));
    uint8_t sc[8], mn[8];
    q4k_scales(blk + 4, sc, mn);
    for (int j = 0; j < 4; ++j) {
      const uint8_t* q = blk + 16 + 32 * j;
      for (int half = 0; half < 2; ++half) {
        const int is = 2 * j + half;
        const float* xb = x + b * QK_K + 64 * j + 32 * half;
        const float dsc = d * (float)sc[is];
        const float dmm = dmin * (float)mn[is];
        for (int l = 0; l < 8; ++l) {
          const int sh = 4 * half;
          float p0 = (float)((q[l] >> sh) & 15) * xb[l];
          float p1 = (float)((q[l + 8] >> sh) & 15) * xb[l + 8];
          float p2 = (float)((q[l + 16] >> sh) & 15) * xb[l + 16];
          float p3 = (float)((q[l + 24] >> sh) & 15) * xb[l + 24];
          float a = (p0 + p1) + (p2 + p3);
          float sx = (xb[l] + xb[l + 8]) + (xb[l + 16] + xb[l + 24]);
          float t = sx * dmm;
          float v = a * dsc - t;
          acc[l] = acc[l] + v;
        }
      }
    }
  }
  return ((((((acc[0] + acc[1]) + acc[2]) + acc[3]) + acc[4]) + acc[5]) + acc[6]) + acc[7];
}

/* The float-x Q6_K dot (tensor/ops.go:114 DotQ6_K ->
 * internal/simd/c2_tensor_dot_q6_k_gen.go:9-81, AVX2 path): per half h of a
 * super-block, four 8-lane partial vectors s0..s3 (quants of x offsets
 * 0, 32, 64, 96 within the half) each take, for k = 0, 1, the pair sum
 * (q[16k+l]·dk·x[16k+l]) + (q[16k+8+l]·dk·x[16k+8+l]) with
 * dk = d·scale[k + 2i] for partial i, products in that order; then
 * acc += (s0 + s1) + (s2 + s3), and the lanes are summed left to right. */
float orc_dot_q6k_f32(const uint8_t* w, const float* x, int cols) {
  int nb = cols / QK_K;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int b = 0; b < nb; ++b) {
    const uint8_t* blk = w + (long)b * BS_Q6K;
    float d = orc_fp16_simd(rd_u16(blk + 208));
    for (int h = 0; h < 2; ++h) {
      const uint8_t* ql = blk + 64 * h;
      const uint8_t* qh = blk + 128 + 32 * h;
      const int8_t* scl = (const int8_t*)(blk + 192 + 8 * h);
      const float* xb = x + b * QK_K + 128 * h;
      float s[4][8];
      for (int i = 0; i < 4; ++i)
        for (int l = 0; l < 8; ++l) s[i][l] = 0.0f;
      for (int k = 0; k < 2; ++k) {
        float dk[4];
        for (int i = 0; i < 4; ++i) dk[i] = d * (float)scl[k + 2 * i];
        for (int i = 0; i < 4; ++i) {
          for (int l = 0; l < 8; ++l) {
            float pr[2];
            for (int t = 0; t < 2; ++t) {
              const int o = 16 * k + 8 * t + l;
              const uint8_t a = ql[o], c = ql[32 + o], hb = qh[o];
              int v;
              switch (i) {
                case 0: v = (a & 15) | ((hb & 3) << 4); break;
                case 1: v = (c & 15) | (((hb >> 2) & 3) << 4); break;
                case 2: v = (a >> 4) | (((hb >> 4) & 3) << 4); break;
                default: v = (c >> 4) | (((hb >> 6) & 3) << 4); break;
              }
              const float qv = (float)(v - 32);
              pr[t] = (qv * dk[i]) * xb[32 * i + o];
            }
            s[i][l] = s[i][l] + (pr[0] + pr[1]);
          }
        }
      }
      for (int l = 0; l < 8; ++l) acc[l] = acc[l] + ((s[0][l] + s[1][l]) + (s[2][l] + s[3][l]));
    }
  }
  return ((((((acc[0] + acc[1]) + acc[2]) + acc[3]) + acc[4]) + acc[5]) + acc[6]) + acc[7];
}

/* tensor/ops.go:40-74 (DotQ5_0, plain float loop; real-model format). */
float orc_dot_q5_0(const uint8_t* w, const float* x, int cols) {
  float total = 0.0f;
  int nb = cols / QK5_0;
  for (int b = 0; b < nb; ++b) {
    const uint8_t* blk = w + (long)b * BS_Q5_0;
    float d = orc_fp16_tensor(rd_u16(blk));
    uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) | ((uint32_t)blk[5] << 24);
    const uint8_t* qs = blk + 6;
    const float* xb = x + b * QK5_0;
    float sum = 0.0f;
    for (int i = 0; i < 16; ++i) {
      uint8_t x0 = qs[i] & 15, x1 = qs[i] >> 4;
      uint8_t h0 = (uint8_t)((qh >> i) & 1), h1 = (uint8_t)((qh >> (i + 16)) & 1);
      float q0 = (float)((int32_t)(x0 | (h0 << 4)) - 16);
      float q1 = (float)((int32_t)(x1 | (h1 << 4)) - 16);
      sum += q0 * xb[i];
      sum += q1 * xb[i + 16];
    }
    total += d * sum;
  }
  return total;
}

/* ------------------------------------------------------ A7 embedding */

/* tensor/ops.go:412-424 */
void orc_dequant_row_q8_0(float* dst, const uint8_t* data, int cols) {
  int nb = cols / QK8_0;
  for (int b = 0; b < nb; ++b) {
    const uint8_t* blk = data + (long)b * BS_Q8_0;
    float d = orc_fp16_tensor(rd_u16(blk));
    for (int i = 0; i < 32; ++i) dst[b * 32 + i] = d * (float)(int8_t)blk[2 + i];
  }
}

/* --------------------------------------------------------- A8/A9 norm */

/* tensor/ops.go:207-218 */
void orc_rmsnorm(float* out, const float* x, const float* w, int n, float eps) {
  float sumsq = 0.0f;
  for (int i = 0; i < n; ++i) {
    float p = x[i] * x[i];
    sumsq = sumsq + p;
  }
  float inv = (float)(1.0 / sqrt((double)(sumsq / (float)n + eps)));
  for (int i = 0; i < n; ++i) out[i] = (x[i] * inv) * w[i];
}

/* tensor/ops.go:221-225 */
void orc_add_bias(float* x, const float* bias, int n) {
  for (int i = 0; i < n; ++i) x[i] = x[i] + bias[i];
}

/* ------------------------------------------------------------ A10 RoPE */

/* tensor/ops.go:237-257: float64 pow/cos/sin, rounded to f32. */
void orc_rope_table(float* cosb, float* sinb, int max_len, int head_dim, float theta) {
  int half = head_dim / 2;
  for (int p = 0; p < max_len; ++p) {
    for (int i = 0; i < half; ++i) {
      double freq = 1.0 / pow((double)theta, (double)(2 * i) / (double)head_dim);
      double val = (double)p * freq;
      cosb[(long)p * half + i] = (float)cos(val);
      sinb[(long)p * half + i] = (float)sin(val);
    }
  }
}

/* tensor/ops.go:262-286: a position outside the table is a no-op. */
void orc_rope_apply(float* vec, int vec_len, int n_heads, int pos, const float* cosb, const float* sinb,
                    int max_len, int head_dim) {
  if (pos < 0 || pos >= max_len) return;
  if (n_heads <= 0 || n_heads * head_dim > vec_len) return;
  int half = head_dim / 2;
  const float* c = cosb + (long)pos * half;
  const float* s = sinb + (long)pos * half;
  for (int h = 0; h < n_heads; ++h) {
    float* v = vec + h * head_dim;
    for (int i = 0; i < half; ++i) {
      float x0 = v[i], x1 = v[i + half];
      v[i] = (x0 * c[i]) - (x1 * s[i]);
      v[i + half] = (x0 * s[i]) + (x1 * c[i]);
    }
  }
}

/* --------------------------------------------------------- A12 softmax */

/* tensor/ops.go:317-339: f32 max (strict >, x[0] first), e =
 * f32(exp(f64(x-max))), sequential f32 sum, multiply by f32(1/sum). */
void orc_softmax(float* x, int n) {
  if (n <= 0) return;
  float mx = x[0];
  for (int i = 1; i < n; ++i)
    if (x[i] > mx) mx = x[i];
  float sum = 0.0f;
  for (int i = 0; i < n; ++i) {
    float e = (float)exp((double)(x[i] - mx));
    x[i] = e;
    sum = sum + e;
  }
  float inv = 1.0f / sum;
  for (int i = 0; i < n; ++i) x[i] = x[i] * inv;
}

/* ------------------------------------------------------- A12 attention */

/* internal/simd/c2_tensor_attn_gen.go:9-66, AVX2/FMA branch: two 8-lane FMA
 * accumulators over 16-wide chunks, an 8-wide chunk into acc0, horizontal
 * ((l0+l1)+(l2+l3))+((l4+l5)+(l6+l7)) of acc0+acc1, scalar non-FMA tail. */
void orc_attn_qk(const float* q, const float* kbase, int pos, int stride, float scale, float* scores, int hd) {
  for (int p = 0; p <= pos; ++p) {
    const float* k = kbase + (long)p * stride;
    float a0[8] = {0, 0, 0, 0, 0, 0, 0, 0}, a1[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int d = 0;
    for (; d + 16 <= hd; d += 16) {
      for (int l = 0; l < 8; ++l) {
        a0[l] = fmaf(q[d + l], k[d + l], a0[l]);
        a1[l] = fmaf(q[d + 8 + l], k[d + 8 + l], a1[l]);
      }
    }
    for (; d + 8 <= hd; d += 8)
      for (int l = 0; l < 8; ++l) a0[l] = fmaf(q[d + l], k[d + l], a0[l]);
    float v[8];
    for (int l = 0; l < 8; ++l) v[l] = a0[l] + a1[l];
    float s = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    for (; d < hd; ++d) s = s + q[d] * k[d];
    scores[p] = s * scale;
  }
}

/* internal/simd/c2_tensor_attn_gen.go:68-153, AVX2/FMA branch: one FMA chain
 * over p = 0..pos per output dimension (hd%64==0 and the 8-wide path alike),
 * scalar non-FMA tail for hd%8 dims. */
void orc_attn_av(const float* scores, const float* vbase, int pos, int stride, float* out, int hd) {
  int d8 = hd - (hd % 8);
  for (int d = 0; d < d8; ++d) {
    float acc = 0.0f;
    for (int p = 0; p <= pos; ++p) acc = fmaf(scores[p], vbase[(long)p * stride + d], acc);
    out[d] = acc;
  }
  for (int d = d8; d < hd; ++d) {
    float acc = 0.0f;
    for (int p = 0; p <= pos; ++p) acc = acc + scores[p] * vbase[(long)p * stride + d];
    out[d] = acc;
  }
}

/* ---------------------------------------------------------- A13 SwiGLU */

/* internal/simd/c2_tensor_swiglu_gen.go:11-58: 8-wide exp(-x) by range
 * reduction and a degree-5 Taylor polynomial, sig = 1/(1+e), (x·sig)·up;
 * the n%8 tail uses f64 exp. */
void orc_swiglu(float* out, const float* gate, const float* up, int n) {
  const float half = bits_f32(0x3f000000u), one = bits_f32(0x3f800000u);
  const float inv_ln2 = bits_f32(0x3fb8aa3bu), ln2 = bits_f32(0x3f317218u);
  const float c5 = bits_f32(0x3c088888u), c4 = bits_f32(0x3d2aaaabu), c3 = bits_f32(0x3e2aaaabu);
  int i = 0;
  for (; i + 8 <= n; i += 8) {
    for (int l = 0; l < 8; ++l) {
      float xv = gate[i + l];
      float nx = -xv;
      float nf = nx * inv_ln2;
      int32_t np = x86_cvtt_i32(nf + half);
      int32_t nn = x86_cvtt_i32(nf - half);
      int32_t ni = (nf >= 0.0f) ? np : nn;
      if (ni < -126) ni = -126;
      if (ni > 127) ni = 127;
      float nif = (float)ni;
      float r = nx - (nif * ln2);
      float p = c5 * r;
      p = p + c4;
      p = p * r;
      p = p + c3;
      p = p * r;
      p = p + half;
      p = p * r;
      p = p + one;
      p = p * r;
      p = p + one;
      float sc = bits_f32((uint32_t)(ni + 127) << 23);
      float ev = p * sc;
      float den = one + ev;
      float sig = one / den;
      float silu = xv * sig;
      out[i + l] = silu * up[i + l];
    }
  }
  for (; i < n; ++i) {
    double g = (double)gate[i];
    float silu = (float)(g / (1.0 + exp(-g)));
    out[i] = silu * up[i];
  }
}

/* ------------------------------------------------- A5 penalty + argmax */

/* c2slm.go:157-180: per-occurrence penalty over TokenIDs[max(0,pos-64),pos),
 * skipping ids outside [0,V), im_end and eos; strict '>' argmax from id 0. */
int32_t orc_penalty_argmax(float* logits, int vocab, const int32_t* token_ids, int pos, int32_t im_end,
                           int32_t eos, float penalty) {
  int start = pos - 64;
  if (start < 0) start = 0;
  for (int p = start; p < pos; ++p) {
    int32_t t = token_ids[p];
    if (t >= 0 && t < vocab && t != im_end && t != eos) {
      if (logits[t] > 0.0f)
        logits[t] = logits[t] / penalty;
      else
        logits[t] = logits[t] * penalty;
    }
  }
  int32_t best = 0;
  float bl = logits[0];
  for (int id = 1; id < vocab; ++id) {
    if (logits[id] > bl) {
      bl = logits[id];
      best = id;
    }
  }
  return best;
}

/* ------------------------------------------------------------ model */

typedef struct {
  const float *attn_norm, *bq, *bk, *bv, *ffn_norm;
  const uint8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
  int32_t tq, tk, tv, to, tg, tu, td;
  const float *q_norm, *k_norm; /* Qwen3 attn_q_norm / attn_k_norm (head_dim), NULL when absent */
} orc_layer;

typedef struct {
  int32_t n_layers, n_embd, n_heads, n_kv_heads, head_dim, n_ff, n_vocab, max_ctx;
  float eps, theta;
  const uint8_t* token_embd;
  int32_t embd_type;
  const uint8_t* output;
  int32_t output_type;
  const float* output_norm;
  const orc_layer* layers;
  int32_t n_threads;
  /* 1: the GEMVs run the reference's AVX2 kernels as restated in
   * c2slm_avx2.c (the CPU baseline); 0: the scalar restatement.  The results
   * are identical. */
  int32_t simd_avx2;
} orc_model;

float orc_avx2_dot_q4k_q8k(const uint8_t* w, const uint8_t* q8k, int cols);
float orc_avx2_dot_q6k_q8k(const uint8_t* w, const uint8_t* q8k, int cols);
int32_t orc_avx2_q6k_block_isum(const uint8_t* wb, const uint8_t* qb);
float orc_avx2_dot_q8_0(const uint8_t* w, const float* x, int cols);

typedef struct {
  orc_model m;
  float *x, *normx, *q, *k, *v, *scores, *attn, *gate, *up, *down, *logits;
  uint8_t* q8k;
  float *cosb, *sinb;
  float* kv; /* [2][L][KVH][max_ctx][HD], engine/kvcache.go:31 */
  int32_t* token_ids;
  int32_t seq_len;
  /* test hook: every Q8_K row dispatch_gemv produces, appended in call
     order (tests/qwen2_f64.py checks each against its own activation) */
  uint8_t* trace;
  long trace_cap, trace_len;
} orc_state;

static long kv_off(const orc_state* s, int is_v, int layer, int head, int pos) {
  /* engine/kvcache.go:127-140 */
  long hd = s->m.head_dim, mt = s->m.max_ctx;
  long head_group = mt * hd, layer_stride = s->m.n_kv_heads * head_group;
  long kv_stride = s->m.n_layers * layer_stride;
  return (is_v ? kv_stride : 0) + layer * layer_stride + head * head_group + pos * hd;
}

orc_state* orc_state_new(const orc_model* m) {
  orc_state* s = (orc_state*)calloc(1, sizeof(orc_state));
  if (!s) return NULL;
  s->m = *m;
  int E = m->n_embd, KV = m->n_kv_heads * m->head_dim, F = m->n_ff;
  s->x = (float*)calloc(E, 4);
  s->normx = (float*)calloc(E, 4);
  s->q = (float*)calloc(E, 4);
  s->k = (float*)calloc(KV, 4);
  s->v = (float*)calloc(KV, 4);
  s->scores = (float*)calloc((size_t)m->max_ctx * (m->n_heads > 0 ? m->n_heads : 1), 4);
  s->attn = (float*)calloc(E, 4);
  s->gate = (float*)calloc(F, 4);
  s->up = (float*)calloc(F, 4);
  s->down = (float*)calloc(E, 4);
  s->logits = (float*)calloc(m->n_vocab, 4);
  s->q8k = (uint8_t*)calloc((16384 / 256) * BS_Q8K, 1); /* engine/pool.go:59 */
  s->cosb = (float*)calloc((size_t)m->max_ctx * (m->head_dim / 2), 4);
  s->sinb = (float*)calloc((size_t)m->max_ctx * (m->head_dim / 2), 4);
  s->kv = (float*)calloc((size_t)2 * m->n_layers * m->n_kv_heads * m->max_ctx * m->head_dim, 4);
  s->token_ids = (int32_t*)calloc(m->max_ctx, 4);
  if (!s->x || !s->kv || !s->cosb || !s->token_ids || !s->logits) return NULL;
  orc_rope_table(s->cosb, s->sinb, m->max_ctx, m->head_dim, m->theta);
  return s;
}

void orc_state_free(orc_state* s) {
  if (!s) return;
  free(s->x); free(s->normx); free(s->q); free(s->k); free(s->v); free(s->scores); free(s->attn);
  free(s->gate); free(s->up); free(s->down); free(s->logits); free(s->q8k); free(s->cosb); free(s->sinb);
  free(s->kv); free(s->token_ids);
  free(s);
}

static int n_workers(const orc_state* s) {
  int nw = s->m.n_threads;
  if (nw < 1) nw = 1;
  if (nw > 32) nw = 32; /* engine/pool.go:47-53 */
  return nw;
}

/* engine/model.go:250-270 → engine/pool.go:122-154: Q4_K/Q6_K quantize x to
 * Q8_K once per call; rows are split over the workers, inline below 256
 * rows.  The split does not change any row's arithmetic. */
static void dispatch_gemv(orc_state* s, float* y, const uint8_t* w, int type, const float* x, int rows, int cols) {
  if (type == T_Q4_K || type == T_Q6_K) {
    orc_quantize_row_q8k(x, s->q8k, cols, (16384 / 256) * BS_Q8K);
    long nbytes = (long)(cols / QK_K) * BS_Q8K;
    if (s->trace && s->trace_len + nbytes <= s->trace_cap) memcpy(s->trace + s->trace_len, s->q8k, (size_t)nbytes);
    s->trace_len += nbytes;
  }
  int nw = (rows < 256) ? 1 : n_workers(s);
  const uint8_t* q8k = s->q8k;
  const int avx2 = s->m.simd_avx2;
  float (*dot_q8k)(const uint8_t*, const uint8_t*, int);
  long rb;
  switch (type) {
    case T_Q4_K:
      rb = (long)(cols / QK_K) * BS_Q4K;
      dot_q8k = avx2 ? orc_avx2_dot_q4k_q8k : orc_dot_q4k_q8k;
#pragma omp parallel for num_threads(nw) schedule(static)
      for (int r = 0; r < rows; ++r) y[r] = dot_q8k(w + r * rb, q8k, cols);
      break;
    case T_Q6_K:
      rb = (long)(cols / QK_K) * BS_Q6K;
      dot_q8k = avx2 ? orc_avx2_dot_q6k_q8k : orc_dot_q6k_q8k;
#pragma omp parallel for num_threads(nw) schedule(static)
      for (int r = 0; r < rows; ++r) y[r] = dot_q8k(w + r * rb, q8k, cols);
      break;
    case T_Q8_0: {
      float (*dot_x)(const uint8_t*, const float*, int) = avx2 ? orc_avx2_dot_q8_0 : orc_dot_q8_0;
      rb = (long)(cols / QK8_0) * BS_Q8_0;
#pragma omp parallel for num_threads(nw) schedule(static)
      for (int r = 0; r < rows; ++r) y[r] = dot_x(w + r * rb, x, cols);
      break;
    }
    case T_Q5_0:
      rb = (long)(cols / QK5_0) * BS_Q5_0;
#pragma omp parallel for num_threads(nw) schedule(static)
      for (int r = 0; r < rows; ++r) y[r] = orc_dot_q5_0(w + r * rb, x, cols);
      break;
    default:
      /* pooled path leaves y untouched for other types (engine/pool.go:105-114) */
      break;
  }
}

/* engine/model.go:221-247 */
static void embed_token(orc_state* s, float* out, int32_t tok) {
  const orc_model* m = &s->m;
  if (tok >= m->n_vocab || tok < 0) tok = 0;
  int E = m->n_embd;
  if (m->embd_type == T_Q8_0) {
    long rb = (long)(E / QK8_0) * BS_Q8_0;
    orc_dequant_row_q8_0(out, m->token_embd + tok * rb, E);
  } else if (m->embd_type == T_F32) {
    memcpy(out, m->token_embd + (long)tok * E * 4, (size_t)E * 4);
  }
}

/* engine/forward.go:143-155 */
static void attention_head(orc_state* s, int layer, int pos, int h, float scale, float* scores) {
  const orc_model* m = &s->m;
  int hd = m->head_dim, qpkv = m->n_heads / m->n_kv_heads;
  int kvh = h / qpkv;
  long ko = kv_off(s, 0, layer, kvh, 0), vo = kv_off(s, 1, layer, kvh, 0);
  orc_attn_qk(s->q + h * hd, s->kv + ko, pos, hd, scale, scores, hd);
  orc_softmax(scores, pos + 1);
  orc_attn_av(scores, s->kv + vo, pos, hd, s->attn + h * hd, hd);
}

/* engine/forward.go:54-138 */
void orc_forward(orc_state* s, int32_t tok, int pos, float* normx_out) {
  const orc_model* m = &s->m;
  int E = m->n_embd, hd = m->head_dim, KV = m->n_kv_heads * hd, F = m->n_ff;
  float scale = (float)(1.0 / sqrt((double)hd));
  embed_token(s, s->x, tok);
  for (int l = 0; l < m->n_layers; ++l) {
    const orc_layer* L = &m->layers[l];
    orc_rmsnorm(s->normx, s->x, L->attn_norm, E, m->eps);
    dispatch_gemv(s, s->q, L->wq, L->tq, s->normx, E, E);
    if (L->bq) orc_add_bias(s->q, L->bq, E);
    dispatch_gemv(s, s->k, L->wk, L->tk, s->normx, KV, E);
    if (L->bk) orc_add_bias(s->k, L->bk, KV);
    dispatch_gemv(s, s->v, L->wv, L->tv, s->normx, KV, E);
    if (L->bv) orc_add_bias(s->v, L->bv, KV);
    /* engine/forward.go:80-91: per-head QK-RMSNorm (Qwen3), before RoPE */
    if (L->q_norm)
      for (int h = 0; h < m->n_heads; ++h) orc_rmsnorm(s->q + h * hd, s->q + h * hd, L->q_norm, hd, m->eps);
    if (L->k_norm)
      for (int h = 0; h < m->n_kv_heads; ++h) orc_rmsnorm(s->k + h * hd, s->k + h * hd, L->k_norm, hd, m->eps);
    orc_rope_apply(s->q, E, m->n_heads, pos, s->cosb, s->sinb, m->max_ctx, hd);
    orc_rope_apply(s->k, KV, m->n_kv_heads, pos, s->cosb, s->sinb, m->max_ctx, hd);
    if (pos >= 0 && pos < m->max_ctx) { /* engine/kvcache.go:143-157 */
      for (int h = 0; h < m->n_kv_heads; ++h) {
        memcpy(s->kv + kv_off(s, 0, l, h, pos), s->k + h * hd, (size_t)hd * 4);
        memcpy(s->kv + kv_off(s, 1, l, h, pos), s->v + h * hd, (size_t)hd * 4);
      }
    }
    /* engine/pool.go:180-208: heads split over workers from pos 256 on */
    int nw = (pos < 256) ? 1 : n_workers(s);
#pragma omp parallel for num_threads(nw) schedule(static)
    for (int h = 0; h < m->n_heads; ++h) attention_head(s, l, pos, h, scale, s->scores + (long)h * m->max_ctx);
    dispatch_gemv(s, s->down, L->wo, L->to, s->attn, E, E);
    for (int i = 0; i < E; ++i) s->x[i] = s->x[i] + s->down[i];
    orc_rmsnorm(s->normx, s->x, L->ffn_norm, E, m->eps);
    dispatch_gemv(s, s->gate, L->wg, L->tg, s->normx, F, E);
    dispatch_gemv(s, s->up, L->wu, L->tu, s->normx, F, E);
    orc_swiglu(s->gate, s->gate, s->up, F);
    dispatch_gemv(s, s->down, L->wd, L->td, s->gate, E, F);
    for (int i = 0; i < E; ++i) s->x[i] = s->x[i] + s->down[i];
  }
  orc_rmsnorm(s->normx, s->x, m->output_norm, E, m->eps);
  if (normx_out) memcpy(normx_out, s->normx, (size_t)E * 4);
}

/* engine/forward.go:171-191 (full-vocabulary path) */
void orc_compute_logits(orc_state* s, const float* normx, float* logits_out) {
  const orc_model* m = &s->m;
  dispatch_gemv(s, s->logits, m->output, m->output_type, normx, m->n_vocab, m->n_embd);
  if (logits_out) memcpy(logits_out, s->logits, (size_t)m->n_vocab * 4);
}

/* c2slm.go:92-117 */
int orc_ingest_from(orc_state* s, int pos, const int32_t* tokens, int n, float* normx_out) {
  if (n == 0) return 0;
  if (pos < 0) pos = 0;
  if (pos > s->seq_len) pos = s->seq_len;
  if (pos < s->seq_len) s->seq_len = pos; /* Rewind, engine/kvcache.go:109-117 */
  int done = 0;
  for (int i = 0; i < n; ++i) {
    int p = pos + i;
    if (p >= s->m.max_ctx) break;
    orc_forward(s, tokens[i], p, NULL);
    s->token_ids[p] = tokens[i];
    s->seq_len = p + 1;
    done++;
  }
  if (normx_out) memcpy(normx_out, s->normx, (size_t)s->m.n_embd * 4);
  return done;
}

/* c2slm.go:144-226 without the text side (no Decode, callback or stop
 * strings): logits → penalty → argmax → EOS check → Forward(best, pos).
 * Returns the number of tokens written to out_tokens. */
int orc_generate(orc_state* s, int max_new, int32_t im_end, int32_t eos, float penalty, int32_t* out_tokens) {
  int cur = s->seq_len, n = 0;
  for (int step = 0; step < max_new; ++step) {
    if (cur >= s->m.max_ctx) break;
    orc_compute_logits(s, s->normx, NULL);
    int32_t best = orc_penalty_argmax(s->logits, s->m.n_vocab, s->token_ids, cur, im_end, eos, penalty);
    out_tokens[n++] = best;
    orc_forward(s, best, cur, NULL);
    s->token_ids[cur] = best;
    cur++;
    s->seq_len = cur;
    if (best == im_end || best == eos) break;
  }
  return n;
}

/* accessors for tests */
float* orc_state_logits(orc_state* s) { return s->logits; }
float* orc_state_normx(orc_state* s) { return s->normx; }
float* orc_state_kv(orc_state* s) { return s->kv; }
int32_t* orc_state_token_ids(orc_state* s) { return s->token_ids; }
int32_t orc_state_seq_len(orc_state* s) { return s->seq_len; }
void orc_state_set_seq_len(orc_state* s, int32_t n) { s->seq_len = n; }
/* test hook: record the Q8_K rows into buf (cap bytes); the length counts
   every byte produced since the last call, so len > cap means truncation */
void orc_state_trace(orc_state* s, uint8_t* buf, long cap) { s->trace = buf; s->trace_cap = cap; s->trace_len = 0; }
long orc_state_trace_len(orc_state* s) { return s->trace_len; }
