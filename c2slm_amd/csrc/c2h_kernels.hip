// gfx950 kernels for c2slm's per-token decode step.
//
// One decode step (one HIP graph on one stream):
//   vocab      Q8_0 x f32 projection of the previous normX, repetition
//              penalty, per-workgroup argmax candidates      (A4, A5)
//   per layer:
//     attn     [argmax reduce + embed on layer 0] RMSNorm -> Q8_K ->
//              q|k|v integer GEMV + bias -> RoPE -> KV store ->
//              exact-order softmax attention, one workgroup
//              per query head                                (A7-A12, A1-A3)
//     attn_out Q8_K(attnOut) -> o GEMV -> X += o              (A1, A2, A9)
//     ffn_in   RMSNorm -> Q8_K -> gate|up GEMV -> SwiGLU      (A8, A1, A2, A13)
//     ffn_out  Q8_K(h) -> down GEMV -> X += down              (A1, A3, A9)
//   final      RMSNorm -> normX                               (A8)
//
// Every float operation follows the reference's order (see each kernel), so
// device results are bit-identical to the CPU path; integer dot products use
// v_dot4_i32_i8 and are exact in any order.  Weight loads are issued at
// kernel entry so HBM latency overlaps the dependent prologue work.
#include "c2h_device.h"
#include "c2h_kernels.h"

namespace c2h {

// ---------------------------------------------------------------- helpers

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

__device__ __forceinline__ float abs_branch(float v) { return (v < 0.0f) ? -v : v; }

// Q8_K quantisation (A1) of nb blocks of x (global or LDS) into LDS by all
// 256 threads: thread t owns element t of every block, so the per-block
// reductions of all blocks run side by side.
// internal/simd/c2_quantize_q8_k_gen.go:22-90: amax of branch-|x| (NaN never
// wins), d = amax/127, q = int(x*(127/amax) ± 0.5) clamped to ±127, zero
// block when amax == 0, bsums over 16 quants.
// red: LDS float[4*64]; scl: LDS float[3*64] (amax, d, 127/amax per block).
constexpr int QCHUNK = 20;

// Element t of blocks b0 .. b0+QCHUNK-1 of x (zero past nb).  Issued before
// the weight prefetch: loads retire in order, so the quantiser then waits
// only for these.
__device__ __forceinline__ void load_row_elems(const float* x, int b0, int nb, float v[QCHUNK]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int k = 0; k < QCHUNK; ++k) v[k] = (b0 + k < nb) ? x[(size_t)(b0 + k) * QK_K + t] : 0.0f;
}

// Quantises blocks b0 .. min(b0+QCHUNK, nb)-1 from registers.
__device__ __forceinline__ void quantize_chunk(const float v[QCHUNK], int b0, int nb, Q8KLds& s, float* red, float* scl) {
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  {
    const int cnt = min(QCHUNK, nb - b0);
#pragma unroll
    for (int k = 0; k < QCHUNK; ++k) {
      if (k < cnt) {
        float m = wave_max_dpp(abs_branch(v[k]));
        if (lane == 0) red[wave * 64 + b0 + k] = m;
      }
    }
    __syncthreads();
    if (t < cnt) {
      const int b = b0 + t;
      float m = red[b];
      m = fmax_gt(m, red[64 + b]);
      m = fmax_gt(m, red[128 + b]);
      m = fmax_gt(m, red[192 + b]);
      scl[b] = m;
      float d = 0.0f, isc = 0.0f;
      if (m != 0.0f) {
        d = m / 127.0f;
        isc = 127.0f / m;
      }
      scl[64 + b] = d;
      scl[128 + b] = isc;
      s.d[b] = d;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < QCHUNK; ++k) {
      if (k < cnt) {
        const int b = b0 + k;
        int q = 0;
        if (scl[b] != 0.0f) {
          float tq = v[k] * scl[128 + b];
          float r = (tq >= 0.0f) ? (tq + 0.5f) : (tq - 0.5f);
          q = go_f32_to_int_clamped127(r);
        }
        reinterpret_cast<int8_t*>(s.q[b])[t] = (int8_t)q;
        int bsum = row16_sum_dpp(q);
        if ((t & 15) == 0) s.bs[b][t >> 4] = bsum;
      }
    }
  }
  __syncthreads();
}

// Whole row: loads chunk by chunk, then quantises.
__device__ void quantize_row_par(const float* x, int nb, Q8KLds& s, float* red, float* scl) {
  for (int b0 = 0; b0 < nb; b0 += QCHUNK) {
    float v[QCHUNK];
    load_row_elems(x, b0, nb, v);
    quantize_chunk(v, b0, nb, s, red, scl);
  }
}

// Same quantiser writing the reference's 292-byte Q8_K block: one
// workgroup (256 threads) per block.
__global__ void __launch_bounds__(256) k_quantize_q8k(const float* __restrict__ x, int nb, uint8_t* __restrict__ y) {
  __shared__ float red[4];
  const int b = blockIdx.x;
  if (b >= nb) return;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const float v = x[(size_t)b * QK_K + t];
  float m = wave_max_dpp(abs_branch(v));
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = fmax_gt(fmax_gt(fmax_gt(red[0], red[1]), red[2]), red[3]);
  uint8_t* yb = y + (size_t)b * BS_Q8K;
  int q = 0;
  float d = 0.0f;
  if (m != 0.0f) {
    d = m / 127.0f;
    float tq = v * (127.0f / m);
    float r = (tq >= 0.0f) ? (tq + 0.5f) : (tq - 0.5f);
    q = go_f32_to_int_clamped127(r);
  }
  yb[4 + t] = (uint8_t)(int8_t)q;
  int bsum = row16_sum_dpp(q);
  if ((t & 15) == 0) reinterpret_cast<int16_t*>(yb + 260)[t >> 4] = (int16_t)bsum;
  if (t == 0) *reinterpret_cast<float*>(yb) = d;
}

// Reference Q8_K bytes -> LDS form (GEMVs fed an external Q8_K row).
__device__ __forceinline__ void load_q8k_block(const uint8_t* qb, Q8KLds& s, int blk, int lane) {
  s.q[blk][lane] = reinterpret_cast<const uint32_t*>(qb + 4)[lane];
  if (lane < 16) s.bs[blk][lane] = (int)reinterpret_cast<const int16_t*>(qb + 260)[lane];
  if (lane == 0) s.d[blk] = *reinterpret_cast<const float*>(qb);
}

// Sequential f32 sum a[0] + a[1] + ... + a[n-1] (one dependent add per
// element, the reference's order) of an LDS buffer that stays readable
// CHAIN_PAD floats past round_up(n, CHAIN_PAD).  The next 32 values are
// loaded before the current 32 are added, so the chain runs at add latency.
constexpr int CHAIN_PAD = 32;
__device__ __forceinline__ float seq_sum_lds(const float* a, int n) {
  const float4* a4 = reinterpret_cast<const float4*>(a);
  float s = 0.0f;
  float4 c[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) c[k] = a4[k];
  const int nc = n >> 5;
  for (int i = 0; i < nc; ++i) {
    float4 nx[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) nx[k] = a4[8 * i + 8 + k];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      s = s + c[k].x;
      s = s + c[k].y;
      s = s + c[k].z;
      s = s + c[k].w;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) c[k] = nx[k];
  }
  const int r = n & 31;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (4 * k + 0 < r) s = s + c[k].x;
    if (4 * k + 1 < r) s = s + c[k].y;
    if (4 * k + 2 < r) s = s + c[k].z;
    if (4 * k + 3 < r) s = s + c[k].w;
  }
  return s;
}

// RMSNorm of xs (LDS, n floats) in place, tensor/ops.go:207-218:
// sequential f32 sum of x*x, inv = f32(1/sqrt(f64(sum/n + eps))),
// out = (x*inv)*w.  sq: LDS scratch readable to round_up(n,32)+32.
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

// ------------------------------------------------------------- GEMV items

// One item = one quarter of one super-block of one row.  The loads are
// issued at kernel entry (prefetch), the arithmetic runs once the Q8_K row
// is in LDS.
struct ItemW {
  uint4 a, b, c, e;  // Q4_K: header, qs lo, qs hi; Q6_K: qlA, qlB, qh, scales
  uint32_t d;        // Q6_K fp16 d
};

// Four 16-byte loads and one fp16 load per item, issued unconditionally with
// the format chosen by address arithmetic (no branch): a loaded register
// that crossed a branch merge would make the compiler wait for it right
// there, defeating the prefetch.  `row` must be a valid row (callers clamp).
//   Q4_K: header, qs[32u..32u+16), qs[32u+16..32u+32), header again;
//   Q6_K: ql[64n+16c..), ql[64n+32+16c..), qh[32n+16c..), scales, d
//         with n = u>>1, c = u&1.
__device__ __forceinline__ ItemW load_item(const WeightRef& W, int type, int nb, int row, int b, int u) {
  const bool q4 = (type == T_Q4_K);
  const size_t blk_idx = (size_t)row * nb + b;
  const int n = u >> 1, c = u & 1;
  const uint8_t* base = W.q + blk_idx * (q4 ? BS_Q4K : BS_Q6K_PACKED);
  const uint4* p = reinterpret_cast<const uint4*>(base);
  const int ia = q4 ? 0 : 4 * n + c;
  const int ib = q4 ? 1 + 2 * u : 4 * n + 2 + c;
  const int ic = q4 ? 2 + 2 * u : 8 + 2 * n + c;
  const int ie = q4 ? 0 : 12;
  const uint16_t* dp = q4 ? reinterpret_cast<const uint16_t*>(base) : (W.d + blk_idx);
  ItemW it;
  it.a = ld_nt(p + ia);
  it.b = ld_nt(p + ib);
  it.c = ld_nt(p + ic);
  it.e = ld_nt(p + ie);
  it.d = *dp;
  return it;
}

__device__ __forceinline__ uint32_t u4get(const uint4& v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

__device__ __forceinline__ uint32_t byte_of(const uint4& v, int i) { return (u4get(v, i >> 2) >> (8 * (i & 3))) & 0xffu; }

// Q4_K pair term (c2_tensor_dot_q4_k_q8_k_gen.go:38-85): s_lo, s_hi of pair u
// of super-block b, folded with the block scales exactly as the reference.
__device__ __forceinline__ float q4k_item(const ItemW& it, const Q8KLds& s, int b, int u, int32_t* lo_out,
                                          int32_t* hi_out) {
  const float q8d = s.d[b];
  const float dW = fp16_simd(it.a.x & 0xffffu) * q8d;
  const float mW = fp16_simd(it.a.x >> 16) * q8d;
  // scale/min pairs 2u, 2u+1 (gen.go:47-61); scale bytes sit at 4..15
  auto sb = [&](int i) { return byte_of(it.a, 4 + i); };
  uint32_t sc0, sc1, m0, m1;
  if (u < 2) {
    sc0 = sb(2 * u) & 63;
    m0 = sb(2 * u + 4) & 63;
    sc1 = sb(2 * u + 1) & 63;
    m1 = sb(2 * u + 5) & 63;
  } else {
    const int k0 = 2 * u - 4, k1 = 2 * u - 3;
    sc0 = (sb(k0 + 8) & 15) | ((sb(k0) >> 6) << 4);
    m0 = (sb(k0 + 8) >> 4) | ((sb(k0 + 4) >> 6) << 4);
    sc1 = (sb(k1 + 8) & 15) | ((sb(k1) >> 6) << 4);
    m1 = (sb(k1 + 8) >> 4) | ((sb(k1 + 4) >> 6) << 4);
  }
  const uint32_t* q8 = s.q[b] + 16 * u;
  int lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t q = u4get(it.b, i);
    lo = sdot4((int)(q & 0x0f0f0f0fu), (int)q8[i], lo);
    hi = sdot4((int)((q >> 4) & 0x0f0f0f0fu), (int)q8[8 + i], hi);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t q = u4get(it.c, i);
    lo = sdot4((int)(q & 0x0f0f0f0fu), (int)q8[4 + i], lo);
    hi = sdot4((int)((q >> 4) & 0x0f0f0f0fu), (int)q8[12 + i], hi);
  }
  *lo_out = lo;
  *hi_out = hi;
  const float bA = (float)(s.bs[b][4 * u] + s.bs[b][4 * u + 1]);
  const float bB = (float)(s.bs[b][4 * u + 2] + s.bs[b][4 * u + 3]);
  return (((float)lo * (dW * (float)sc0)) - (bA * (mW * (float)m0))) +
         (((float)hi * (dW * (float)sc1)) - (bB * (mW * (float)m1)));
}

// Q6_K partial super-block sum for half n = u>>1, lanes l in [16c, 16c+16)
// with c = u&1 (c2_tensor_gemv2_q6_k_q8_k_gen.go:104-207): four (n,k) sums
// s, each contributing (s - 32*bsum)*scale.  The four partials of a block
// add up (exactly) to the reference's isum.
__device__ __forceinline__ int32_t q6k_item(const ItemW& it, const Q8KLds& s, int b, int u) {
  const int n = u >> 1, c = u & 1;
  int32_t part = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint4& ql = (k & 1) ? it.b : it.a;
    const uint32_t* q8 = s.q[b] + 32 * n + 8 * k + 4 * c;
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t qlv = u4get(ql, i);
      uint32_t lo = (k < 2) ? (qlv & 0x0f0f0f0fu) : ((qlv >> 4) & 0x0f0f0f0fu);
      uint32_t hi = ((u4get(it.c, i) >> (2 * k)) & 0x03030303u) << 4;
      sum = sdot4((int)(lo | hi), (int)q8[i], sum);
    }
    const int j = 8 * n + 2 * k + c;
    const int sc = (int)(int8_t)byte_of(it.e, j);
    part += (sum - 32 * s.bs[b][j]) * sc;
  }
  return part;
}

// Item result into LDS: Q4_K a float term, Q6_K an int partial plus (u==0)
// the block's d*q8d.
__device__ __forceinline__ void run_item(const ItemW& it, int type, const Q8KLds& s, int b, int u, float* term_slot,
                                         float* dq_slot, int32_t* isums, size_t isum_base) {
  if (type == T_Q4_K) {
    int32_t lo, hi;
    *term_slot = q4k_item(it, s, b, u, &lo, &hi);
    if (isums) {
      isums[isum_base + 2 * u] = lo;
      isums[isum_base + 2 * u + 1] = hi;
    }
  } else {
    *reinterpret_cast<int32_t*>(term_slot) = q6k_item(it, s, b, u);
    if (u == 0) *dq_slot = fp16_simd(it.d) * s.d[b];
  }
}

// Per-row fold in the reference's order: Q4_K acc += term over (block, pair);
// Q6_K acc += f32(isum)*(d*q8d) over blocks.
__device__ __forceinline__ float fold_row(int type, const float* terms, const float* dq, int nb, int32_t* isums,
                                          size_t isum_base) {
  float acc = 0.0f;
  if (type == T_Q4_K) {
    for (int i = 0; i < 4 * nb; ++i) acc = acc + terms[i];
  } else {
    const int32_t* p = reinterpret_cast<const int32_t*>(terms);
    for (int bb = 0; bb < nb; ++bb) {
      int32_t isum = p[4 * bb] + p[4 * bb + 1] + p[4 * bb + 2] + p[4 * bb + 3];
      if (isums) isums[isum_base + bb] = isum;
      acc = acc + (float)isum * dq[bb];
    }
  }
  return acc;
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

// fp16 block scale of the Q8_0 table as the simd kernels decode it: hardware
// conversion (exact for every finite half), +0.0f maps -0 to +0 like the
// reference's lookup table.  NaN scales stay NaN (payload bits may differ).
__device__ __forceinline__ float q8_0_scale(uint32_t h16) {
  float f = (float)__builtin_bit_cast(_Float16, (unsigned short)h16);
  return f + 0.0f;
}

// Token embedding (engine/model.go:221-247 -> tensor/ops.go:412-424) from the
// packed Q8_0 table into LDS; fp16 decoded like tensor.FP16ToF32 (-0 kept).
__device__ __forceinline__ void embed_lds(const WeightRef& emb, int n_vocab, int E, int tok, float* xs) {
  if (tok >= n_vocab || tok < 0) tok = 0;
  const int nb8 = E / QK8_0;
  const uint8_t* row = emb.q + (size_t)tok * q8_0_row_stride(nb8);
  const uint16_t* drow = reinterpret_cast<const uint16_t*>(row);
  const uint8_t* qsrow = row + (size_t)q8_0_dpad(nb8) * 2;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int b = e >> 5, k = e & 31;
    int j = k & 7, i = k >> 3;  // element k of block b is byte i of lane j's dword
    int bq = b >> 2, bb = b & 3;
    int8_t q = (int8_t)qsrow[(bq * 8 + j) * 16 + bb * 4 + i];
    float d = fp16_tensor(drow[b]);
    xs[e] = d * (float)q;
  }
  __syncthreads();
}

// X into LDS (optionally from the embedding), RMSNorm, Q8_K of the first nb
// blocks.  Shared by the attention block and ffn_in.
struct NormArgs {
  int prologue;
  const float* x;
  float* x_out;
  const float* norm_w;
  float eps;
  int E;
  const WeightRef* emb;
  int n_vocab;
  const float* part_v;
  const int* part_i;
  int n_part;
  int32_t* token_ids;
  int max_ctx;
  C2hState* state;
};

// X elements tid + 256k (k < 4, n_embd <= 1024) for the PRO_NORM prologue,
// loaded before the weight prefetch so the prologue does not wait on it.
constexpr int XREG = 4;
__device__ __forceinline__ void load_x_regs(const float* x, int E, float xr[XREG]) {
#pragma unroll
  for (int k = 0; k < XREG; ++k) {
    const int i = threadIdx.x + 256 * k;
    xr[k] = (i < E) ? x[i] : 0.0f;
  }
}

__device__ __forceinline__ void norm_quant_prologue(const NormArgs& A, int nb, float* xs, float* sq, Q8KLds& s,
                                                    float* red, float* scl, float* inv_slot, ArgCand* ared,
                                                    const float xr[XREG]) {
  const int tid = threadIdx.x;
  if (A.prologue == PRO_NORM) {
#pragma unroll
    for (int k = 0; k < XREG; ++k) {
      const int i = tid + 256 * k;
      if (i < A.E) xs[i] = xr[k];
    }
    __syncthreads();
  } else {
    int tok;
    if (A.prologue == PRO_ARGMAX_EMBED_NORM)
      tok = reduce_argmax_partials(A.part_v, A.part_i, A.n_part, ared);
    else
      tok = A.state->token;
    embed_lds(*A.emb, A.n_vocab, A.E, tok, xs);
    if (blockIdx.x == 0) {
      for (int i = tid; i < A.E; i += blockDim.x) A.x_out[i] = xs[i];
      if (tid == 0) {
        int pos = A.state->pos;
        A.state->token = tok;
        if (pos >= 0 && pos < A.max_ctx) A.token_ids[pos] = tok;
      }
    }
  }
  rmsnorm_lds(xs, sq, A.norm_w, A.E, A.eps, inv_slot);
  quantize_row_par(xs, nb, s, red, scl);
}

// ------------------------------------------------------------ GEMV kernel

// GEMV launch: a workgroup owns rpw rows of one job; thread t owns item
// (row t / (4nb), block, quarter).  LDS: Q8_K row | 512 term slots |
// 256 scale slots | red[256] | scl[192] | x | x*x.
__global__ void __launch_bounds__(256) k_gemv(GemvParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  Q8KLds& s = *reinterpret_cast<Q8KLds*>(smem);
  float* terms = reinterpret_cast<float*>(smem + sizeof(Q8KLds));  // [2][256]
  float* dq = terms + 512;                                          // [2][128]
  float* red = dq + 256;                                            // [256]
  float* scl = red + 256;                                           // [192]
  float* xs = scl + 192;                                            // [n_x_lds]
  float* sq = xs + P.n_x_lds;                                       // [n_x_lds]
  __shared__ float inv_slot;
  __shared__ ArgCand ared[4];

  const int tid = threadIdx.x;

  // ---- which job and rows this workgroup owns
  int ji = 0;
  while (ji < P.n_jobs - 1 && (int)blockIdx.x >= P.jobs[ji + 1].wg_begin) ++ji;
  const GemvJob& J = P.jobs[ji];
  const int nb = J.nb;
  const int ipr = 4 * nb;  // items per row
  const int r_local = tid / ipr;
  const int rem = tid - r_local * ipr;
  const int b = rem >> 2, u = rem & 3;
  const int row0 = ((int)blockIdx.x - J.wg_begin) * J.rpw;
  const int row = row0 + r_local;
  const bool active = (r_local < J.rpw) && (row < J.rows);
  const bool paired = (J.mode == MODE_SWIGLU);

  // ---- activation loads first (loads retire in order)
  const bool quant_regs = (P.prologue == PRO_QUANT) && (P.nb_in <= QCHUNK);
  float xq[QCHUNK];
  float xr[XREG];
  if (quant_regs) load_row_elems(P.x, 0, P.nb_in, xq);
  if (P.prologue == PRO_NORM) load_x_regs(P.x, P.n_x, xr);

  // ---- weight prefetch (independent of the activation row)
  ItemW w1, w2;
  if (active) {
    w1 = load_item(J.w, J.type, nb, row, b, u);
    if (paired) w2 = load_item(J.w2, J.type2, nb, row, b, u);
  }

  // ---- prologue: the Q8_K input row in LDS
  if (P.prologue == PRO_Q8K) {
    const int wave = tid >> 6, lane = tid & 63;
    for (int bb = wave; bb < P.nb_in; bb += 4) load_q8k_block(P.q8k_in + (size_t)bb * BS_Q8K, s, bb, lane);
    __syncthreads();
  } else if (P.prologue == PRO_QUANT) {
    if (quant_regs)
      quantize_chunk(xq, 0, P.nb_in, s, red, scl);
    else
      quantize_row_par(P.x, P.nb_in, s, red, scl);
  } else {
    NormArgs A{P.prologue, P.x, P.x_out, P.norm_w, P.eps, P.n_x, &P.emb, P.n_vocab, P.part_v, P.part_i, P.n_part,
               P.token_ids, P.max_ctx, P.state};
    norm_quant_prologue(A, P.nb_in, xs, sq, s, red, scl, &inv_slot, ared, xr);
  }

  // ---- items
  if (active) {
    const size_t ib = ((size_t)row * nb + b) * 8;
    run_item(w1, J.type, s, b, u, terms + tid, dq + r_local * nb + b, J.isums, ib);
    if (paired) run_item(w2, J.type2, s, b, u, terms + 256 + tid, dq + 128 + r_local * nb + b, nullptr, 0);
  }
  __syncthreads();

  // ---- per-row fold in the reference's order, then the epilogue
  if (tid < J.rpw) {
    const int r = row0 + tid;
    if (r < J.rows) {
      float acc = fold_row(J.type, terms + tid * ipr, dq + tid * nb, nb, J.isums, (size_t)r * nb);
      if (paired) {
        float up = fold_row(J.type2, terms + 256 + tid * ipr, dq + 128 + tid * nb, nb, nullptr, 0);
        int n8 = J.rows - (J.rows % 8);
        J.y[r] = (r < n8) ? swiglu_poly(acc, up) : swiglu_tail(acc, up);
      } else if (J.mode == MODE_STORE) {
        J.y[r] = acc;
      } else if (J.mode == MODE_BIAS) {
        J.y[r] = acc + J.bias[r];
      } else {  // MODE_RESID
        J.y[r] = J.y[r] + acc;
      }
    }
  }
}

// ------------------------------------------------------------- final norm

__global__ void __launch_bounds__(256) k_rmsnorm(NormParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  float* xs = reinterpret_cast<float*>(smem);
  float* sq = xs + P.n_lds;
  __shared__ float inv_slot;
  for (int i = threadIdx.x; i < P.n; i += blockDim.x) xs[i] = P.x[i];
  __syncthreads();
  rmsnorm_lds(xs, sq, P.w, P.n, P.eps, &inv_slot);
  float* out = P.out_sel ? P.out_buf[P.state->nx_out] : P.out;
  for (int i = threadIdx.x; i < P.n; i += blockDim.x) out[i] = xs[i];
}

// ------------------------------------------------------- attention block

// One query head h per workgroup (engine/forward.go:66-106 for that head):
//   [embed] RMSNorm -> Q8_K, q rows [64h, 64h+64), k and v rows of KV head
//   g = h/qpkv (+ bias, tensor/ops.go:221-225), RoPE (tensor/ops.go:262-286)
//   on q_h and k_g, KV store (engine/kvcache.go:143-157) by the group's
//   first head, then attention (engine/forward.go:143-155 with
//   internal/simd/c2_tensor_attn_gen.go and tensor.Softmax): scores in the
//   two-accumulator FMA order, softmax with f64 exp and a sequential f32 sum,
//   one FMA chain over positions per output dim with V staged through LDS.
// Heads of one group recompute their shared k/v rows (64+64 rows of 3
// super-blocks), which costs less than a launch and a global round trip.
template <int NB>
__global__ void __launch_bounds__(256) k_attn_fused(AttnFusedParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  // region A: Q8_K | red | scl | dq | x | x*x     (reused for staged V)
  Q8KLds& s = *reinterpret_cast<Q8KLds*>(smem);
  float* red = reinterpret_cast<float*>(smem + sizeof(Q8KLds));  // [256]
  float* scl = red + 256;                                         // [192]
  float* dq = scl + 192;                                          // [3][64*FUSED_MAX_NB]
  float* xs = dq + 3 * 64 * FUSED_MAX_NB;                         // [n_x_lds]
  float* sq = xs + P.n_x_lds;                                     // [n_x_lds]
  float* vs = reinterpret_cast<float*>(smem);                     // [vchunk][64], after the GEMV
  // region B: GEMV terms [3][64][4nb], then scores
  float* regb = reinterpret_cast<float*>(smem) + P.a_lds;
  float* terms = regb;
  float* sc = regb;
  __shared__ __align__(16) float qkv_s[3][64];
  __shared__ float red_m[4];
  __shared__ float inv_slot;
  __shared__ ArgCand ared[4];

  const int tid = threadIdx.x;
  const int h = blockIdx.x;
  const int qpkv = P.n_heads / P.n_kv_heads;
  const int g = h / qpkv;
  constexpr int nb = NB;
  constexpr int ipr = 4 * nb;
  constexpr int HD = 64;
  constexpr int ipm = HD * ipr;  // items per matrix (= 256*nb)

  // ---- activation loads first (loads retire in order)
  float xr[XREG];
  if (P.prologue == PRO_NORM) load_x_regs(P.x, P.n_embd, xr);

  // ---- weight prefetch: thread t owns items t + 256*j of each matrix
  ItemW w[3][NB];
  const WeightRef* W[3] = {&P.wq, &P.wk, &P.wv};
  const int T3[3] = {P.tq, P.tk, P.tv};
  const int rbase[3] = {h * HD, g * HD, g * HD};
#pragma unroll
  for (int m = 0; m < 3; ++m) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int i = tid + 256 * j;
      const int r = i / ipr, rem = i - r * ipr;
      w[m][j] = load_item(*W[m], T3[m], nb, rbase[m] + r, rem >> 2, rem & 3);
    }
  }

  // ---- prologue
  NormArgs A{P.prologue, P.x, P.x_out, P.norm_w, P.eps, P.n_embd, &P.emb, P.n_vocab, P.part_v, P.part_i, P.n_part,
             P.token_ids, P.max_ctx, P.state};
  norm_quant_prologue(A, nb, xs, sq, s, red, scl, &inv_slot, ared, xr);

  // ---- items -> terms [m][r][4nb]
#pragma unroll
  for (int m = 0; m < 3; ++m) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int i = tid + 256 * j;
      const int r = i / ipr, rem = i - r * ipr;
      const int b = rem >> 2, u = rem & 3;
      run_item(w[m][j], T3[m], s, b, u, terms + m * ipm + i, dq + m * HD * FUSED_MAX_NB + r * nb + b, nullptr, 0);
    }
  }
  __syncthreads();

  // ---- fold + bias: thread t < 192 owns row t%64 of matrix t/64
  if (tid < 3 * HD) {
    const int m = tid / HD, r = tid - m * HD;
    float acc = fold_row(T3[m], terms + m * ipm + r * ipr, dq + m * HD * FUSED_MAX_NB + r * nb, nb, nullptr, 0);
    const float* bias = (m == 0) ? P.bq : (m == 1 ? P.bk : P.bv);
    if (bias) acc = acc + bias[rbase[m] + r];
    qkv_s[m][r] = acc;
  }
  __syncthreads();

  float* q_s = qkv_s[0];
  float* k_s = qkv_s[1];
  float* v_s = qkv_s[2];
  const int pos = P.state->pos;
  const int T = pos + 1;
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

  // ---- scores: (Σ q·k in the two-accumulator FMA order) * scale
  float lmax = -__builtin_inff();
  for (int p = tid; p < T; p += blockDim.x) {
    const float* kr = (p == pos) ? k_s : (kcache + (size_t)p * HD);
    float4 kk4[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) kk4[i] = *reinterpret_cast<const float4*>(kr + 4 * i);
    float a0[8], a1[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      a0[l] = 0.0f;
      a1[l] = 0.0f;
    }
#pragma unroll
    for (int d = 0; d < HD; d += 16) {
      const float kk[16] = {kk4[d / 4].x,     kk4[d / 4].y,     kk4[d / 4].z,     kk4[d / 4].w,
                            kk4[d / 4 + 1].x, kk4[d / 4 + 1].y, kk4[d / 4 + 1].z, kk4[d / 4 + 1].w,
                            kk4[d / 4 + 2].x, kk4[d / 4 + 2].y, kk4[d / 4 + 2].z, kk4[d / 4 + 2].w,
                            kk4[d / 4 + 3].x, kk4[d / 4 + 3].y, kk4[d / 4 + 3].z, kk4[d / 4 + 3].w};
#pragma unroll
      for (int l = 0; l < 8; ++l) {
        a0[l] = __builtin_fmaf(q_s[d + l], kk[l], a0[l]);
        a1[l] = __builtin_fmaf(q_s[d + 8 + l], kk[8 + l], a1[l]);
      }
    }
    float v[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) v[l] = a0[l] + a1[l];
    float sco = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    sco = sco * P.scale;
    sc[p] = sco;
    lmax = (sco > lmax) ? sco : lmax;
  }
  // max: x[0] first, strict '>' (tensor/ops.go:321-326): the max of the
  // non-NaN scores, or NaN when score[0] is NaN.
  lmax = wave_max_dpp(lmax);
  if ((tid & 63) == 0) red_m[tid >> 6] = lmax;
  __syncthreads();
  float mx = fmax_gt(fmax_gt(fmax_gt(red_m[0], red_m[1]), red_m[2]), red_m[3]);
  if (sc[0] != sc[0]) mx = sc[0];
  for (int p = tid; p < T; p += blockDim.x) sc[p] = (float)exp((double)(sc[p] - mx));
  __syncthreads();
  if (tid == 0) inv_slot = 1.0f / seq_sum_lds(sc, T);
  __syncthreads();
  const float inv = inv_slot;
  for (int p = tid; p < T; p += blockDim.x) sc[p] = sc[p] * inv;

  // ---- AV: out[d] = fma chain over p of (prob[p], V[p][d]); V[pos] is v_s
  float acc = 0.0f;
  const int d = tid & 63;
  for (int p0 = 0; p0 < pos; p0 += P.vchunk) {
    const int np = min(P.vchunk, pos - p0);
    __syncthreads();  // previous chunk consumed (and probabilities written)
    const float4* src = reinterpret_cast<const float4*>(vcache + (size_t)p0 * HD);
    float4* dst = reinterpret_cast<float4*>(vs);
    for (int i = tid; i < np * (HD / 4); i += blockDim.x) dst[i] = src[i];
    __syncthreads();
    if (tid < HD) {
      int p = 0;
      for (; p + 16 <= np; p += 16) {
        float vv[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) vv[k] = vs[(p + k) * HD + d];
        float4 s0 = *reinterpret_cast<const float4*>(sc + p0 + p);
        float4 s1 = *reinterpret_cast<const float4*>(sc + p0 + p + 4);
        float4 s2 = *reinterpret_cast<const float4*>(sc + p0 + p + 8);
        float4 s3 = *reinterpret_cast<const float4*>(sc + p0 + p + 12);
        const float ss[16] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w,
                              s2.x, s2.y, s2.z, s2.w, s3.x, s3.y, s3.z, s3.w};
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = __builtin_fmaf(ss[k], vv[k], acc);
      }
      for (; p < np; ++p) acc = __builtin_fmaf(sc[p0 + p], vs[p * HD + d], acc);
    }
  }
  __syncthreads();
  if (tid < HD) {
    acc = __builtin_fmaf(sc[pos], v_s[d], acc);
    P.out[h * HD + d] = acc;
  }
}

template __global__ void k_attn_fused<1>(AttnFusedParams);
template __global__ void k_attn_fused<2>(AttnFusedParams);
template __global__ void k_attn_fused<3>(AttnFusedParams);
template __global__ void k_attn_fused<4>(AttnFusedParams);

// ------------------------------------------------------------------ vocab

// Vocabulary projection with the 8-lane order of
// internal/simd/c2_tensor_dot_q8_0_gen.go:79-102 (lane j of a row owns
// acc[j]), repetition penalty (c2slm.go:157-170) and per-workgroup argmax
// candidates (c2slm.go:173-180).  256 threads = 32 rows x 8 lanes; each
// workgroup covers VOCAB_TILES consecutive 32-row tiles, loading tile t+1
// while computing tile t.  Rows of up to VOCAB_NQ*4 blocks (1024 columns).
constexpr int VOCAB_NQ = 8;

struct VocabRow {
  uint4 q[VOCAB_NQ];
  uint4 d[VOCAB_NQ / 2];
};

__device__ __forceinline__ void vocab_load(const VocabParams& P, int row, int j, int nq, size_t stride, int dpad,
                                           VocabRow& R) {
  if (row < P.n_vocab) {
    const uint8_t* rowp = P.w.q + (size_t)row * stride;
    const uint4* dvec = reinterpret_cast<const uint4*>(rowp);
    const uint4* qrow = reinterpret_cast<const uint4*>(rowp + (size_t)dpad * 2);
#pragma unroll
    for (int bq = 0; bq < VOCAB_NQ; ++bq)
      if (bq < nq) R.q[bq] = ld_nt(qrow + bq * 8 + j);
#pragma unroll
    for (int k = 0; k < VOCAB_NQ / 2; ++k)
      if (2 * k < nq) R.d[k] = dvec[k];
  }
}

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
  const int nq = q8_0_nq(nb8);
  const int dpad = q8_0_dpad(nb8);
  const size_t stride = q8_0_row_stride(nb8);
  const int row_base = blockIdx.x * VOCAB_TILES * 32 + rl;

  // x first (loads retire in order), then the weights of the first tile
  const float* x = P.x_sel ? P.x_buf[P.state->nx_in] : P.x;
  float xr[VOCAB_NQ / 2];
#pragma unroll
  for (int k = 0; k < VOCAB_NQ / 2; ++k) {
    const int e = tid + 256 * k;
    xr[k] = (e < nb8 * 32) ? x[e] : 0.0f;
  }
  VocabRow cur, nxt;
  vocab_load(P, row_base, j, nq, stride, dpad, cur);
#pragma unroll
  for (int k = 0; k < VOCAB_NQ / 2; ++k) {
    const int e = tid + 256 * k;
    if (e < nb8 * 32) {
      int b = e >> 5, kk = e & 31;
      int jj = kk & 7, ii = kk >> 3;
      xp[(b * 8 + jj) * 4 + ii] = xr[k];
    }
  }
  if (tid == 0) {
    int pos = P.state->pos;
    int start = pos - 64;
    if (start < 0) start = 0;
    nwin_s = (P.apply_penalty && pos > 0) ? (pos - start) : 0;
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

#pragma unroll
  for (int tile = 0; tile < VOCAB_TILES; ++tile) {
    const int row = row_base + tile * 32;
    if (tile + 1 < VOCAB_TILES) vocab_load(P, row + 32, j, nq, stride, dpad, nxt);
    const bool valid = row < P.n_vocab;
    float acc = 0.0f;
    if (valid) {
#pragma unroll
      for (int bq = 0; bq < VOCAB_NQ; ++bq) {
        if (bq < nq) {
          const uint4 dv = cur.d[bq >> 1];
          const uint32_t dlo = (bq & 1) ? dv.z : dv.x;
          const uint32_t dhi = (bq & 1) ? dv.w : dv.y;
          const uint32_t dd[4] = {dlo & 0xffffu, dlo >> 16, dhi & 0xffffu, dhi >> 16};
          const uint32_t ww[4] = {cur.q[bq].x, cur.q[bq].y, cur.q[bq].z, cur.q[bq].w};
#pragma unroll
          for (int bb = 0; bb < 4; ++bb) {
            const int b = bq * 4 + bb;
            if (b < nb8) {
              const float dsc = q8_0_scale(dd[bb]);
              const float4 xv = *reinterpret_cast<const float4*>(xp + (b * 8 + j) * 4);
              const uint32_t q = ww[bb];
              const float p0 = (float)(int8_t)(q & 0xff) * xv.x;
              const float p1 = (float)(int8_t)((q >> 8) & 0xff) * xv.y;
              const float p2 = (float)(int8_t)((q >> 16) & 0xff) * xv.z;
              const float p3 = (float)(int8_t)(q >> 24) * xv.w;
              acc = acc + ((p0 + p1) + (p2 + p3)) * dsc;
            }
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
    cur = nxt;
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
