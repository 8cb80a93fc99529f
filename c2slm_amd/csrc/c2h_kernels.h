// Kernel parameter blocks shared by the device code and the host launcher.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace c2h {

// Device-resident per-step state.  The host rewrites it (one small copy)
// before each graph launch, so captured graphs replay unchanged.
struct C2hState {
  int32_t pos;      // position of the token being forwarded
  int32_t token;    // forward: token to embed; step: argmax result
  int32_t im_end;   // ids exempt from the penalty (c2slm.go:163)
  int32_t eos;
  float penalty;    // 1.15 in the reference (c2slm.go:165,167)
  int32_t nx_in;    // normX buffer read by the vocab projection
  int32_t nx_out;   // normX buffer written by the final RMSNorm
  int32_t pad;
};

// Q8_K row as the GEMVs keep it in LDS: quants packed four per dword, the
// f32 scale and the sixteen 16-element sums widened to int32.
constexpr int LDS_Q8K_BLOCKS = 64;
struct Q8KLds {
  uint32_t q[LDS_Q8K_BLOCKS][64];
  float d[LDS_Q8K_BLOCKS];
  int32_t bs[LDS_Q8K_BLOCKS][16];
};

// A weight tensor in its device layout:
//   Q4_K: the reference's rows back to back, row stride (cols/256)*144;
//   Q6_K: per super-block 208 bytes ql|qh|scales in q, the fp16 d in d;
//   Q8_0: per row ceil(nb/4) groups of 8 lanes x 16 bytes (lane j holds
//         bytes j, j+8, j+16, j+24 of four consecutive blocks) in q, the
//         per-block fp16 d in d.
struct WeightRef {
  const uint8_t* q;
  const uint16_t* d;
};

enum Prologue : int {
  PRO_Q8K = 0,                // copy an external Q8_K row
  PRO_QUANT = 1,              // quantise the f32 input x
  PRO_NORM = 2,               // RMSNorm(x) then quantise
  PRO_EMBED_NORM = 3,         // embed state->token, RMSNorm, quantise
  PRO_ARGMAX_EMBED_NORM = 4,  // reduce vocab argmax candidates, embed, RMSNorm, quantise
};

enum GemvMode : int {
  MODE_STORE = 0,   // y = acc
  MODE_BIAS = 1,    // y = acc + bias       (tensor/ops.go:221-225)
  MODE_RESID = 2,   // y = y + acc          (engine/forward.go:112-114,129-131)
  MODE_SWIGLU = 3,  // y = SwiGLU(acc(w), acc(w2))
};

struct GemvJob {
  WeightRef w;
  WeightRef w2;
  int type;
  int type2;
  int rows;
  int nb;          // super-blocks per row (floor(cols/256))
  int rpt;         // rows per wave task = floor(64/nb)
  int task_begin;  // first wave task of this job
  int n_tasks;
  int mode;
  float* y;
  const float* bias;
  int32_t* isums;  // optional integer sums (Q4_K: 8 per row-block; Q6_K: 1)
};

constexpr int MAX_JOBS = 4;

struct GemvParams {
  int prologue;
  int nb_in;
  int n_x;      // length of x for the norm prologues
  int n_x_lds;  // LDS floats reserved for x (multiple of 4)
  float eps;
  const float* x;
  const float* norm_w;
  const uint8_t* q8k_in;
  float* x_out;
  WeightRef emb;
  int n_vocab;
  int max_ctx;
  int32_t* token_ids;
  const float* part_v;
  const int* part_i;
  int n_part;
  C2hState* state;
  int n_jobs;
  GemvJob jobs[MAX_JOBS];
};

struct NormParams {
  const float* x;
  const float* w;
  float eps;
  int n;
  int out_sel;  // 1: write out_buf[state->nx_out]
  float* out;
  float* out_buf[2];
  C2hState* state;
};

struct AttnParams {
  const float* q;
  const float* k;
  const float* v;
  float* out;
  float* kv;
  const float* rope_cos;
  const float* rope_sin;
  int rope_len;
  int layer;
  int n_layers;
  int n_heads;
  int n_kv_heads;
  int max_ctx;
  float scale;
  C2hState* state;
};

constexpr int VOCAB_TILES = 4;  // 32-row tiles per vocab workgroup

struct VocabParams {
  WeightRef w;
  int n_vocab;
  int n_embd;
  int x_sel;  // 1: read x_buf[state->nx_in]
  const float* x;
  const float* x_buf[2];
  const int32_t* token_ids;
  int apply_penalty;
  float* logits_out;  // optional pre-penalty logits
  float* part_v;
  int* part_i;
  C2hState* state;
};

__global__ void k_quantize_q8k(const float* __restrict__ x, int nb, uint8_t* __restrict__ y);
__global__ void k_gemv(GemvParams P);
__global__ void k_rmsnorm(NormParams P);
__global__ void k_attention(AttnParams P);
__global__ void k_vocab(VocabParams P);
__global__ void k_argmax_final(const float* pv, const int* pi, int n, C2hState* state);

}  // namespace c2h
