// gfx950 kernels for c2slm's per-token decode step.
//
// Structure of one decode step (one HIP graph, one stream):
//   vocab      Q8_0 x f32 projection of the previous normX, repetition
//              penalty, per-workgroup argmax partials       (A4, A5)
//   per layer:
//     attn_in  [argmax reduce + embed on layer 0] RMSNorm -> Q8_K in LDS ->
//              q|k|v integer GEMV + bias                    (A7, A8, A1, A2, A3, A9)
//     attn     RoPE, KV store, exact-order softmax attention (A10, A11, A12)
//     attn_out Q8_K(attnOut) in LDS -> o GEMV -> X += o      (A1, A2, A9)
//     ffn_in   RMSNorm -> Q8_K -> gate|up GEMV -> SwiGLU     (A8, A1, A2, A13)
//     ffn_out  Q8_K(h) in LDS -> down GEMV -> X += down      (A1, A3, A9)
//   final      RMSNorm -> normX                               (A8)
//
// Every float operation follows the reference's order (see each kernel), so
// the device results are bit-identical to the CPU path; integer dot products
// use v_dot4_i32_i8 and are exact in any order.
#include "c2h_device.h"
#include "c2h_kernels.h"

namespace c2h {

// ---------------------------------------------------------------- helpers

__device__ __forceinline__ float wave_max_nonneg(float m) {
  // all inputs are >= 0 (or -0) and not NaN; '>' keeps the reference's
  // comparison semantics (a -0 never replaces +0).
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    float t = __shfl_xor(m, o);
    m = (t > m) ? t : m;
  }
  return m;
}

struct ArgCand {
  float v;
  int i;
};

// Candidate order of the reference's greedy scan (c2slm.go:173-180): larger
// key wins, ties go to the lower index.  Keys are never NaN (see vocab).
__device__ __forceinline__ ArgCand arg_better(ArgCand a, ArgCand b) {
  bool take_b = (b.v > a.v) || (b.v == a.v && b.i < a.i);
  return take_b ? b : a;
}

__device__ __forceinline__ ArgCand wave_argmax(ArgCand c) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    ArgCand t;
    t.v = __shfl_xor(c.v, o);
    t.i = __shfl_xor(c.i, o);
    c = arg_better(c, t);
  }
  return c;
}

// Q8_K block (A1) quantised by one wave from 256 floats; lane l owns
// elements 4l..4l+3.  Writes the LDS form used by the GEMVs.
// internal/simd/c2_quantize_q8_k_gen.go:22-90.
__device__ __forceinline__ void quantize_block_wave(const float* xb, Q8KLds& s, int blk, int lane) {
  float4 v = *reinterpret_cast<const float4*>(xb + 4 * lane);
  float e[4] = {v.x, v.y, v.z, v.w};
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float a = (e[i] < 0.0f) ? -e[i] : e[i];
    m = (a > m) ? a : m;
  }
  m = wave_max_nonneg(m);
  uint32_t packed = 0;
  int qsum = 0;
  float d = 0.0f;
  if (m != 0.0f) {
    d = m / 127.0f;
    float iscale = 127.0f / m;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float t = e[i] * iscale;
      float r = (t >= 0.0f) ? (t + 0.5f) : (t - 0.5f);
      int q = go_f32_to_int_clamped127(r);
      qsum += q;
      packed |= ((uint32_t)(q & 0xff)) << (8 * i);
    }
  }
  s.q[blk][lane] = packed;
  qsum += __shfl_xor(qsum, 1);
  qsum += __shfl_xor(qsum, 2);
  if ((lane & 3) == 0) s.bs[blk][lane >> 2] = qsum;
  if (lane == 0) s.d[blk] = d;
}

// Same quantiser writing the reference's 292-byte Q8_K block.
__global__ void k_quantize_q8k(const float* __restrict__ x, int nb, uint8_t* __restrict__ y) {
  int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  int lane = threadIdx.x & 63;
  if (wave >= nb) return;
  const float* xb = x + (size_t)wave * QK_K;
  float4 v = *reinterpret_cast<const float4*>(xb + 4 * lane);
  float e[4] = {v.x, v.y, v.z, v.w};
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float a = (e[i] < 0.0f) ? -e[i] : e[i];
    m = (a > m) ? a : m;
  }
  m = wave_max_nonneg(m);
  uint8_t* yb = y + (size_t)wave * BS_Q8K;
  uint32_t packed = 0;
  int qsum = 0;
  float d = 0.0f;
  if (m != 0.0f) {
    d = m / 127.0f;
    float iscale = 127.0f / m;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float t = e[i] * iscale;
      float r = (t >= 0.0f) ? (t + 0.5f) : (t - 0.5f);
      int q = go_f32_to_int_clamped127(r);
      qsum += q;
      packed |= ((uint32_t)(q & 0xff)) << (8 * i);
    }
  }
  reinterpret_cast<uint32_t*>(yb + 4)[lane] = packed;
  qsum += __shfl_xor(qsum, 1);
  qsum += __shfl_xor(qsum, 2);
  if ((lane & 3) == 0) reinterpret_cast<int16_t*>(yb + 260)[lane >> 2] = (int16_t)qsum;
  if (lane == 0) *reinterpret_cast<float*>(yb) = d;
}

// Reference Q8_K bytes -> LDS form (for GEMVs fed an external Q8_K row).
__device__ __forceinline__ void load_q8k_block(const uint8_t* qb, Q8KLds& s, int blk, int lane) {
  s.q[blk][lane] = reinterpret_cast<const uint32_t*>(qb + 4)[lane];
  if (lane < 16) s.bs[blk][lane] = (int)reinterpret_cast<const int16_t*>(qb + 260)[lane];
  if (lane == 0) s.d[blk] = *reinterpret_cast<const float*>(qb);
}

// Sequential f32 sum of n values in LDS, read ahead in float4 chunks so the
// chain runs at add latency (tensor/ops.go:210-212 order).
__device__ __forceinline__ float seq_sum_lds(const float* a, int n) {
  float s = 0.0f;
  int n4 = n >> 2;
  const float4* a4 = reinterpret_cast<const float4*>(a);
  int i = 0;
  if (n4 > 0) {
    float4 nxt0 = a4[0];
    float4 nxt1 = (n4 > 1) ? a4[1] : nxt0;
    for (; i < n4; ++i) {
      float4 cur = nxt0;
      nxt0 = nxt1;
      if (i + 2 < n4) nxt1 = a4[i + 2];
      s = s + cur.x;
      s = s + cur.y;
      s = s + cur.z;
      s = s + cur.w;
    }
  }
  for (int j = n4 * 4; j < n; ++j) s = s + a[j];
  return s;
}

// RMSNorm of xs (LDS, n floats) into xs, tensor/ops.go:207-218:
// sequential f32 sum of x*x, inv = f32(1/sqrt(f64(sum/n + eps))),
// out = (x*inv)*w.  sq is LDS scratch of n floats.
__device__ void rmsnorm_lds(float* xs, float* sq, const float* __restrict__ w, int n, float eps, float* inv_slot) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) sq[i] = xs[i] * xs[i];
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = seq_sum_lds(sq, n);
    *inv_slot = (float)(1.0 / sqrt((double)(s / (float)n + eps)));
  }
  __syncthreads();
  float inv = *inv_slot;
  for (int i = threadIdx.x; i < n; i += blockDim.x) xs[i] = (xs[i] * inv) * w[i];
  __syncthreads();
}

// -------------------------------------------------------------- GEMV units

// Four pair terms of one Q4_K super-block against Q8_K block b
// (c2_tensor_dot_q4_k_q8_k_gen.go:38-85).  isums (optional) receives the
// eight 32-element integer sums.
__device__ __forceinline__ void q4k_unit(const uint8_t* __restrict__ wblk, const Q8KLds& s, int b, float t[4],
                                         int32_t* isums) {
  const uint4* wp = reinterpret_cast<const uint4*>(wblk);
  uint4 w[9];
#pragma unroll
  for (int i = 0; i < 9; ++i) w[i] = ld_nt(wp + i);
  float q8d = s.d[b];
  float dW = fp16_simd(w[0].x & 0xffffu) * q8d;
  float mW = fp16_simd(w[0].x >> 16) * q8d;
  uint32_t sw[3] = {w[0].y, w[0].z, w[0].w};
  uint8_t sb[12];
#pragma unroll
  for (int i = 0; i < 12; ++i) sb[i] = (uint8_t)(sw[i >> 2] >> (8 * (i & 3)));
  uint8_t sc[8], mn[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    sc[j] = sb[j] & 63;
    mn[j] = sb[j + 4] & 63;
    sc[j + 4] = (uint8_t)((sb[j + 8] & 15) | ((sb[j] >> 6) << 4));
    mn[j + 4] = (uint8_t)((sb[j + 8] >> 4) | ((sb[j + 4] >> 6) << 4));
  }
  uint32_t qs[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    qs[4 * i] = w[1 + i].x;
    qs[4 * i + 1] = w[1 + i].y;
    qs[4 * i + 2] = w[1 + i].z;
    qs[4 * i + 3] = w[1 + i].w;
  }
  const uint32_t* q8 = s.q[b];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    int lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t q = qs[8 * p + i];
      lo = sdot4((int)(q & 0x0f0f0f0fu), (int)q8[16 * p + i], lo);
      hi = sdot4((int)((q >> 4) & 0x0f0f0f0fu), (int)q8[16 * p + 8 + i], hi);
    }
    if (isums) {
      isums[2 * p] = lo;
      isums[2 * p + 1] = hi;
    }
    float bA = (float)(s.bs[b][4 * p] + s.bs[b][4 * p + 1]);
    float bB = (float)(s.bs[b][4 * p + 2] + s.bs[b][4 * p + 3]);
    t[p] = (((float)lo * (dW * (float)sc[2 * p])) - (bA * (mW * (float)mn[2 * p]))) +
           (((float)hi * (dW * (float)sc[2 * p + 1])) - (bB * (mW * (float)mn[2 * p + 1])));
  }
}

// Integer super-block sum of one Q6_K block (packed as ql|qh|scales, 208 B)
// against Q8_K block b (c2_tensor_gemv2_q6_k_q8_k_gen.go:104-207).
__device__ __forceinline__ int32_t q6k_unit(const uint8_t* __restrict__ wblk, const Q8KLds& s, int b) {
  const uint4* wp = reinterpret_cast<const uint4*>(wblk);
  uint4 w[13];
#pragma unroll
  for (int i = 0; i < 13; ++i) w[i] = ld_nt(wp + i);
  uint32_t qlw[32], qhw[16];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    qlw[4 * i] = w[i].x;
    qlw[4 * i + 1] = w[i].y;
    qlw[4 * i + 2] = w[i].z;
    qlw[4 * i + 3] = w[i].w;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    qhw[4 * i] = w[8 + i].x;
    qhw[4 * i + 1] = w[8 + i].y;
    qhw[4 * i + 2] = w[8 + i].z;
    qhw[4 * i + 3] = w[8 + i].w;
  }
  uint32_t scw[4] = {w[12].x, w[12].y, w[12].z, w[12].w};
  const uint32_t* q8 = s.q[b];
  int32_t isum = 0;
#pragma unroll
  for (int n = 0; n < 2; ++n) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      int sa = 0, sbv = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t qlv = qlw[16 * n + 8 * (k & 1) + i];
        uint32_t lo = (k < 2) ? (qlv & 0x0f0f0f0fu) : ((qlv >> 4) & 0x0f0f0f0fu);
        uint32_t hi = ((qhw[8 * n + i] >> (2 * k)) & 0x03030303u) << 4;
        int q6 = (int)(lo | hi);
        int q8v = (int)q8[32 * n + 8 * k + i];
        if (i < 4)
          sa = sdot4(q6, q8v, sa);
        else
          sbv = sdot4(q6, q8v, sbv);
      }
      int j0 = 8 * n + 2 * k;
      int sc0 = (int)(int8_t)(scw[j0 >> 2] >> (8 * (j0 & 3)));
      int sc1 = (int)(int8_t)(scw[(j0 + 1) >> 2] >> (8 * ((j0 + 1) & 3)));
      isum += ((sa - 32 * s.bs[b][j0]) * sc0) + ((sbv - 32 * s.bs[b][j0 + 1]) * sc1);
    }
  }
  return isum;
}

// One row-block unit of a job; returns the row's value in the lane that owns
// block 0 of the row (other lanes return garbage).  The per-row fold is the
// reference's sequential order over super-blocks (and pairs for Q4_K).
__device__ __forceinline__ float gemv_row_fold(const WeightRef& W, int type, int nb, int row, int r_local, int b,
                                               bool active, const Q8KLds& s, int lane, int32_t* isums_out) {
  if (type == T_Q4_K) {
    float t[4] = {0.f, 0.f, 0.f, 0.f};
    int32_t is[8];
    if (active) {
      q4k_unit(W.q + ((size_t)row * nb + b) * BS_Q4K, s, b, t, isums_out ? is : nullptr);
      if (isums_out) {
#pragma unroll
        for (int i = 0; i < 8; ++i) isums_out[((size_t)row * nb + b) * 8 + i] = is[i];
      }
    }
    float acc = 0.0f;
    int base = r_local * nb;
    for (int bb = 0; bb < nb; ++bb) {
      int src = (base + bb) & 63;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        float v = __shfl(t[p], src);
        acc = acc + v;
      }
    }
    return acc;
  } else {
    float term = 0.0f;
    if (active) {
      int32_t isum = q6k_unit(W.q + ((size_t)row * nb + b) * BS_Q6K_PACKED, s, b);
      if (isums_out) isums_out[(size_t)row * nb + b] = isum;
      float d = fp16_simd(W.d[(size_t)row * nb + b]);
      term = (float)isum * (d * s.d[b]);
    }
    float acc = 0.0f;
    int base = r_local * nb;
    for (int bb = 0; bb < nb; ++bb) {
      float v = __shfl(term, (base + bb) & 63);
      acc = acc + v;
    }
    return acc;
  }
}

// ------------------------------------------------------------- prologues

// Argmax over the vocab kernel's per-workgroup candidates.
__device__ int reduce_argmax_partials(const float* __restrict__ pv, const int* __restrict__ pi, int n, ArgCand* red) {
  ArgCand c;
  c.v = -__builtin_inff();
  c.i = 0x7fffffff;
  for (int k = threadIdx.x; k < n; k += blockDim.x) {
    ArgCand t;
    t.v = pv[k];
    t.i = pi[k];
    c = arg_better(c, t);
  }
  c = wave_argmax(c);
  int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[wave] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    ArgCand r = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = arg_better(r, red[w]);
    red[0] = r;
  }
  __syncthreads();
  int tok = red[0].i;
  __syncthreads();
  return tok;
}

// Token embedding (engine/model.go:221-247 → tensor/ops.go:412-424) from the
// packed Q8_0 table into LDS.
__device__ void embed_lds(const WeightRef& emb, int n_vocab, int E, int tok, float* xs) {
  if (tok >= n_vocab || tok < 0) tok = 0;
  int nb8 = E / QK8_0;
  int nq = (nb8 + 3) >> 2;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int b = e >> 5, k = e & 31;
    int j = k & 7, i = k >> 3;  // element k of block b is byte i of lane j's dword
    int bq = b >> 2, bb = b & 3;
    const uint8_t* qsrow = emb.q + (size_t)tok * nq * 128;
    int8_t q = (int8_t)qsrow[(bq * 8 + j) * 16 + bb * 4 + i];
    float d = fp16_tensor(emb.d[(size_t)tok * nb8 + b]);
    xs[e] = d * (float)q;
  }
  __syncthreads();
}

// ------------------------------------------------------------ GEMV kernel

__global__ void __launch_bounds__(256) k_gemv(GemvParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  Q8KLds& s = *reinterpret_cast<Q8KLds*>(smem);
  float* xs = reinterpret_cast<float*>(smem + sizeof(Q8KLds));
  float* sq = xs + P.n_x_lds;
  __shared__ float inv_slot;
  __shared__ ArgCand red[4];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;

  // ---- prologue: produce the Q8_K input row in LDS
  if (P.prologue == PRO_Q8K) {
    for (int b = wave; b < P.nb_in; b += 4) load_q8k_block(P.q8k_in + (size_t)b * BS_Q8K, s, b, lane);
    __syncthreads();
  } else if (P.prologue == PRO_QUANT) {
    for (int b = wave; b < P.nb_in; b += 4) quantize_block_wave(P.x + (size_t)b * QK_K, s, b, lane);
    __syncthreads();
  } else {
    // PRO_NORM / PRO_EMBED_NORM / PRO_ARGMAX_EMBED_NORM
    const int E = P.n_x;
    if (P.prologue == PRO_NORM) {
      for (int i = threadIdx.x; i < E; i += blockDim.x) xs[i] = P.x[i];
      __syncthreads();
    } else {
      int tok;
      if (P.prologue == PRO_ARGMAX_EMBED_NORM) {
        tok = reduce_argmax_partials(P.part_v, P.part_i, P.n_part, red);
      } else {
        tok = P.state->token;
      }
      embed_lds(P.emb, P.n_vocab, E, tok, xs);
      if (blockIdx.x == 0) {
        for (int i = threadIdx.x; i < E; i += blockDim.x) P.x_out[i] = xs[i];
        if (threadIdx.x == 0) {
          int pos = P.state->pos;
          P.state->token = tok;
          if (pos >= 0 && pos < P.max_ctx) P.token_ids[pos] = tok;
        }
      }
    }
    rmsnorm_lds(xs, sq, P.norm_w, E, P.eps, &inv_slot);
    for (int b = wave; b < P.nb_in; b += 4) quantize_block_wave(xs + b * QK_K, s, b, lane);
    __syncthreads();
  }

  // ---- wave tasks
  int task = blockIdx.x * 4 + wave;
  int ji = 0;
  while (ji < P.n_jobs - 1 && task >= P.jobs[ji + 1].task_begin) ++ji;
  const GemvJob& J = P.jobs[ji];
  int t_local = task - J.task_begin;
  if (t_local < 0 || t_local >= J.n_tasks) return;
  const int nb = J.nb;
  const int r_local = lane / nb;
  const int b = lane - r_local * nb;
  const int row = t_local * J.rpt + r_local;
  const bool active = (r_local < J.rpt) && (row < J.rows);
  const bool owner = active && (b == 0);

  float acc = gemv_row_fold(J.w, J.type, nb, row, r_local, b, active, s, lane, J.isums);
  if (J.mode == MODE_SWIGLU) {
    float up = gemv_row_fold(J.w2, J.type2, nb, row, r_local, b, active, s, lane, nullptr);
    if (owner) {
      int n8 = J.rows - (J.rows % 8);
      J.y[row] = (row < n8) ? swiglu_poly(acc, up) : swiglu_tail(acc, up);
    }
  } else if (owner) {
    if (J.mode == MODE_STORE)
      J.y[row] = acc;
    else if (J.mode == MODE_BIAS)
      J.y[row] = acc + J.bias[row];
    else  // MODE_RESID
      J.y[row] = J.y[row] + acc;
  }
}

// ------------------------------------------------------------- final norm

__global__ void __launch_bounds__(256) k_rmsnorm(NormParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  float* xs = reinterpret_cast<float*>(smem);
  float* sq = xs + P.n;
  __shared__ float inv_slot;
  for (int i = threadIdx.x; i < P.n; i += blockDim.x) xs[i] = P.x[i];
  __syncthreads();
  rmsnorm_lds(xs, sq, P.w, P.n, P.eps, &inv_slot);
  float* out = P.out_sel ? P.out_buf[P.state->nx_out] : P.out;
  for (int i = threadIdx.x; i < P.n; i += blockDim.x) out[i] = xs[i];
}

// -------------------------------------------------------------- attention

// Exact-order decode attention for one query head per workgroup
// (engine/forward.go:143-155 with the AVX2 kernels of
// internal/simd/c2_tensor_attn_gen.go and tensor.Softmax):
//   RoPE (tensor/ops.go:262-286) on q_h and on k of its KV head,
//   KV store (engine/kvcache.go:143-157) by the first head of each group,
//   scores by the two-accumulator FMA order, softmax with f64 exp and a
//   sequential f32 sum, and one FMA chain over positions per output dim.
__global__ void __launch_bounds__(256) k_attention(AttnParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  float* sc = reinterpret_cast<float*>(smem);  // [max_ctx] scores / probabilities
  __shared__ __align__(16) float q_s[64];
  __shared__ __align__(16) float k_s[64];
  __shared__ __align__(16) float v_s[64];
  __shared__ float red_m[4];
  __shared__ float inv_slot;

  const int h = blockIdx.x;
  const int qpkv = P.n_heads / P.n_kv_heads;
  const int g = h / qpkv;
  const int tid = threadIdx.x;
  const int pos = P.state->pos;
  const int T = pos + 1;
  const int HD = 64;

  if (tid < HD) {
    q_s[tid] = P.q[h * HD + tid];
    k_s[tid] = P.k[g * HD + tid];
    v_s[tid] = P.v[g * HD + tid];
  }
  __syncthreads();
  if (pos >= 0 && pos < P.rope_len && tid < HD / 2) {
    const float c = P.rope_cos[(size_t)pos * (HD / 2) + tid];
    const float sn = P.rope_sin[(size_t)pos * (HD / 2) + tid];
    float x0 = q_s[tid], x1 = q_s[tid + 32];
    q_s[tid] = (x0 * c) - (x1 * sn);
    q_s[tid + 32] = (x0 * sn) + (x1 * c);
    x0 = k_s[tid];
    x1 = k_s[tid + 32];
    k_s[tid] = (x0 * c) - (x1 * sn);
    k_s[tid + 32] = (x0 * sn) + (x1 * c);
  }
  __syncthreads();

  const size_t head_stride = (size_t)P.max_ctx * HD;
  float* kcache = P.kv + ((size_t)P.layer * P.n_kv_heads + g) * head_stride;
  float* vcache = P.kv + (((size_t)P.n_layers + P.layer) * P.n_kv_heads + g) * head_stride;
  if ((h % qpkv) == 0 && tid < HD && pos < P.max_ctx) {
    kcache[(size_t)pos * HD + tid] = k_s[tid];
    vcache[(size_t)pos * HD + tid] = v_s[tid];
  }
  if (T > P.max_ctx) return;  // rejected on the host; kept as a guard

  // scores: score[p] = (Σ q·k in the two-accumulator FMA order) * scale
  float lmax = -__builtin_inff();
  for (int p = tid; p < T; p += blockDim.x) {
    const float* kr = (p == pos) ? k_s : (kcache + (size_t)p * HD);
    float a0[8], a1[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      a0[l] = 0.0f;
      a1[l] = 0.0f;
    }
#pragma unroll
    for (int d = 0; d < HD; d += 16) {
      float4 k0 = *reinterpret_cast<const float4*>(kr + d);
      float4 k1 = *reinterpret_cast<const float4*>(kr + d + 4);
      float4 k2 = *reinterpret_cast<const float4*>(kr + d + 8);
      float4 k3 = *reinterpret_cast<const float4*>(kr + d + 12);
      float kk[16] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w, k2.x, k2.y, k2.z, k2.w, k3.x, k3.y, k3.z, k3.w};
#pragma unroll
      for (int l = 0; l < 8; ++l) {
        a0[l] = __builtin_fmaf(q_s[d + l], kk[l], a0[l]);
        a1[l] = __builtin_fmaf(q_s[d + 8 + l], kk[8 + l], a1[l]);
      }
    }
    float v[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) v[l] = a0[l] + a1[l];
    float s = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    s = s * P.scale;
    sc[p] = s;
    lmax = (s > lmax) ? s : lmax;
  }
  // max: x[0] first, strict '>' (tensor/ops.go:321-326): the max of the
  // non-NaN scores, or NaN when score[0] is NaN.
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    float t = __shfl_xor(lmax, o);
    lmax = (t > lmax) ? t : lmax;
  }
  if ((tid & 63) == 0) red_m[tid >> 6] = lmax;
  __syncthreads();
  float mx = red_m[0];
  for (int w = 1; w < 4; ++w) mx = (red_m[w] > mx) ? red_m[w] : mx;
  if (sc[0] != sc[0]) mx = sc[0];
  for (int p = tid; p < T; p += blockDim.x) sc[p] = (float)exp((double)(sc[p] - mx));
  __syncthreads();
  if (tid == 0) inv_slot = 1.0f / seq_sum_lds(sc, T);
  __syncthreads();
  const float inv = inv_slot;
  for (int p = tid; p < T; p += blockDim.x) sc[p] = sc[p] * inv;
  __syncthreads();

  // AV: out[d] = fma chain over p of (prob[p], V[p][d])
  if (tid < HD) {
    const int d = tid;
    float acc = 0.0f;
    const int npre = pos;  // positions read from the cache; pos itself uses v_s
    int p = 0;
    for (; p + 8 <= npre; p += 8) {
      float vv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) vv[u] = vcache[(size_t)(p + u) * HD + d];
      float4 s0 = *reinterpret_cast<const float4*>(sc + p);
      float4 s1 = *reinterpret_cast<const float4*>(sc + p + 4);
      float ss[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = __builtin_fmaf(ss[u], vv[u], acc);
    }
    for (; p < npre; ++p) acc = __builtin_fmaf(sc[p], vcache[(size_t)p * HD + d], acc);
    acc = __builtin_fmaf(sc[pos], v_s[d], acc);
    P.out[h * HD + d] = acc;
  }
}

// ------------------------------------------------------------------ vocab

// Vocabulary projection with the 8-lane order of
// internal/simd/c2_tensor_dot_q8_0_gen.go:79-102 (lane j of a row owns
// acc[j]), repetition penalty (c2slm.go:157-170) and per-workgroup argmax
// candidates (c2slm.go:173-180).  256 threads = 32 rows x 8 lanes; each
// workgroup covers VOCAB_TILES consecutive 32-row tiles.
__global__ void __launch_bounds__(256) k_vocab(VocabParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  float* xp = reinterpret_cast<float*>(smem);  // x permuted: [b][j][i] = x[32b + j + 8i]
  __shared__ int win[64];
  __shared__ int nwin_s;
  __shared__ ArgCand red[4];

  const int tid = threadIdx.x;
  const int j = tid & 7;
  const int rl = tid >> 3;
  const int E = P.n_embd;
  const int nb8 = E / QK8_0;
  const int nq = (nb8 + 3) >> 2;
  const float* x = P.x_sel ? P.x_buf[P.state->nx_in] : P.x;

  for (int e = tid; e < nb8 * 32; e += blockDim.x) {
    int b = e >> 5, k = e & 31;
    int jj = k & 7, ii = k >> 3;
    xp[(b * 8 + jj) * 4 + ii] = x[e];
  }
  if (tid == 0) {
    int pos = P.state->pos;
    int start = pos - 64;
    if (start < 0) start = 0;
    int n = (P.apply_penalty && pos > 0) ? (pos - start) : 0;
    nwin_s = n;
  }
  __syncthreads();
  const int nwin = nwin_s;
  if (tid < nwin) {
    int pos = P.state->pos;
    int start = pos - 64;
    if (start < 0) start = 0;
    win[tid] = P.token_ids[start + tid];
  }
  __syncthreads();

  ArgCand best;
  best.v = -__builtin_inff();
  best.i = 0x7fffffff;
  const int im_end = P.state->im_end, eos = P.state->eos;
  const float penalty = P.state->penalty;

  for (int tile = 0; tile < VOCAB_TILES; ++tile) {
    const int row = (blockIdx.x * VOCAB_TILES + tile) * 32 + rl;
    const bool valid = row < P.n_vocab;
    float acc = 0.0f;
    if (valid) {
      const uint4* qrow = reinterpret_cast<const uint4*>(P.w.q + (size_t)row * nq * 128);
      const uint16_t* drow = P.w.d + (size_t)row * nb8;
      for (int bq = 0; bq < nq; ++bq) {
        uint4 wv = ld_nt(qrow + bq * 8 + j);
        uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
          int b = bq * 4 + bb;
          if (b < nb8) {
            float d = fp16_simd(drow[b]);
            float4 xv = *reinterpret_cast<const float4*>(xp + (b * 8 + j) * 4);
            uint32_t q = ww[bb];
            float p0 = (float)(int8_t)(q & 0xff) * xv.x;
            float p1 = (float)(int8_t)((q >> 8) & 0xff) * xv.y;
            float p2 = (float)(int8_t)((q >> 16) & 0xff) * xv.z;
            float p3 = (float)(int8_t)(q >> 24) * xv.w;
            acc = acc + ((p0 + p1) + (p2 + p3)) * d;
          }
        }
      }
    }
    // (((((((a0+a1)+a2)+a3)+a4)+a5)+a6)+a7) into lane j == 0
    const int base = tid & ~7;
    float tot = __shfl(acc, base);
#pragma unroll
    for (int k = 1; k < 8; ++k) tot = tot + __shfl(acc, base + k);
    // occurrences of this row id in the penalty window
    int cnt = 0;
    for (int e = j; e < nwin; e += 8) cnt += (win[e] == row) ? 1 : 0;
    cnt += __shfl_xor(cnt, 1);
    cnt += __shfl_xor(cnt, 2);
    cnt += __shfl_xor(cnt, 4);
    if (valid && j == 0) {
      if (P.logits_out) P.logits_out[row] = tot;
      if (row != im_end && row != eos) {
        for (int c = 0; c < cnt; ++c) tot = (tot > 0.0f) ? (tot / penalty) : (tot * penalty);
      }
      ArgCand c;
      // NaN never wins the scan except at id 0, where it ends it
      c.v = (tot != tot) ? ((row == 0) ? __builtin_inff() : -__builtin_inff()) : tot;
      c.i = row;
      best = arg_better(best, c);
    }
  }
  best = wave_argmax(best);
  if ((tid & 63) == 0) red[tid >> 6] = best;
  __syncthreads();
  if (tid == 0) {
    ArgCand r = red[0];
    for (int w = 1; w < 4; ++w) r = arg_better(r, red[w]);
    P.part_v[blockIdx.x] = r.v;
    P.part_i[blockIdx.x] = r.i;
  }
}

// Final reduction for standalone argmax calls (no following layer kernel).
__global__ void __launch_bounds__(256) k_argmax_final(const float* pv, const int* pi, int n, C2hState* state) {
  __shared__ ArgCand red[4];
  int tok = reduce_argmax_partials(pv, pi, n, red);
  if (threadIdx.x == 0) state->token = tok;
}

}  // namespace c2h
