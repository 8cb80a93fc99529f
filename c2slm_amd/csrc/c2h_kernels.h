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
  int32_t seq;      // step number, handed to the host with the step's token
  // head_dim 64: the RoPE row of pos (cos at [0, 32), sin at [32, 64)), so
  // that decode attention reads it with pos instead of after it
  float rope[64];
  // forward count: the final RMSNorm of every forward advances it, and the
  // tags of a launch's handover (k_attn_oproj) are epoch * 256 + layer.
  // Last field: the host's state copies stop before it (kStatePushBytes),
  // so it only ever moves forward.
  uint32_t epoch;
};
constexpr size_t kStatePushBytes = offsetof(C2hState, epoch);

// Q8_K row as the GEMVs keep it in LDS: quants packed four per dword, the
// f32 scale and the sixteen 16-element sums widened to int32.
// Block rows are padded to 68 dwords so that neighbouring blocks start in
// different LDS banks.
template <int NB>
struct alignas(16) Q8KRow {
  uint32_t q[NB][68];
  int32_t bs[NB][16];  // 16-byte aligned rows (an item reads its sums whole)
  float d[NB];
};
constexpr int LDS_Q8K_BLOCKS = 64;  // 16384 columns (the reference's Q8_K scratch, engine/pool.go:59)
typedef Q8KRow<LDS_Q8K_BLOCKS> Q8KLds;

// A weight tensor in its device layout:
//   Q4_K: the reference's rows back to back, row stride (cols/256)*144;
//   Q6_K: per super-block 208 bytes ql|qh|scales in q, the fp16 d in d;
//   Q8_0: per row the fp16 block scales (padded to a multiple of 32 halves,
//         64 bytes for 28 blocks) followed by ceil(nb/4) groups of 8 lanes x
//         16 bytes (lane j holds bytes j, j+8, j+16, j+24 of four
//         consecutive blocks); d is unused.
struct WeightRef {
  const uint8_t* q;
  const uint16_t* d;
};

__host__ __device__ inline int q8_0_dpad(int nb8) { return ((nb8 + 31) / 32) * 32; }
__host__ __device__ inline int q8_0_nq(int nb8) { return (nb8 + 3) / 4; }
__host__ __device__ inline size_t q8_0_row_stride(int nb8) { return (size_t)q8_0_dpad(nb8) * 2 + (size_t)q8_0_nq(nb8) * 128; }

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

// One matrix of a GEMV launch.  A workgroup owns `rpw` consecutive rows;
// each of its threads owns one quarter of one super-block of one row
// (Q4_K: one 32-element pair; Q6_K: 16 of the 32 lanes of one half).
struct GemvJob {
  WeightRef w;
  WeightRef w2;
  int type;
  int type2;
  int rows;
  int nb;        // super-blocks per row (floor(cols/256))
  int rpw;       // rows per workgroup = floor(256 / (4*nb))
  int n_wg;      // workgroups of this job (grid row blockIdx.y = job)
  int mode;
  int spare;     // k_attn_block: the job's offset in y_tag (else unused; named so the fields load as one batch)
  float* y;
  const float* bias;
  int32_t* isums;  // optional integer sums (Q4_K: 8 per row-block; Q6_K: 1)
};

constexpr int MAX_JOBS = 4;

// Threads of a row-kernel workgroup.  A wide Q8_K input (12 or more
// super-blocks, quantised by every workgroup) runs on 8 waves: its blocks
// quantise at most three per wave with two waves per SIMD, and the
// workgroup takes twice the rows, which halves the redundant quantisations.
// The norm prologues hold one float4 of x per thread, so rows of more than
// 1024 values (up to 2048) run on 8 waves as well.  The SwiGLU pair of
// narrow rows (up to 4 super-blocks) runs on 8 waves with the gate items on
// the first half and the up items on the second, one item per thread.
__host__ __device__ constexpr int row_threads(int nb, int pro, int mode) {
  return ((pro == PRO_QUANT && nb >= 12) || (pro >= PRO_NORM && nb > 4) || (mode == MODE_SWIGLU && nb <= 4)) ? 512
                                                                                                            : 256;
}
// Threads holding the items of one matrix (rows per workgroup = this / (4 nb)).
__host__ __device__ constexpr int row_item_threads(int nb, int pro, int mode) {
  return (mode == MODE_SWIGLU && nb <= 4) ? row_threads(nb, pro, mode) / 2 : row_threads(nb, pro, mode);
}

struct GemvParams {
  int prologue;
  int nb_in;
  int n_x;      // length of x for the norm prologues
  int n_x_lds;  // LDS floats of the x*x buffer (see chain_lds_floats)
  float eps;
  const float* x;
  const float* norm_w;
  const uint8_t* q8k_in;
  // layer-0 prologues: embed state->token or the argmax of the vocab
  // candidates, publish it (x_out, state->token, token_ids[pos])
  WeightRef emb;
  int n_vocab;
  const float* part_v;
  const int* part_i;
  int n_part;
  float* x_out;
  int32_t* token_ids;
  int max_ctx;
  C2hState* state;
  // step graphs: the chosen token and state->seq, written by layer 0's
  // prologue into host-pinned memory (system scope) so that the host has
  // the token while the rest of the step runs (nullptr: none)
  int32_t* tok_out;
  // k_attn_oproj's o-projection half: its input as {value, tag} words, and
  // the flag a wait that runs out sets (host-pinned)
  const uint64_t* x_tag;
  int* wait_err;
  uint64_t* y_tag;  // k_attn_block's q|k|v half: its outputs again as {value, tag} words (job offset in spare)
  // k_attn_block's parts: X's pending terms [FOLD_NB][pend_n] (the previous
  // layer's k_ffn_block down projection), added to X in block order before
  // use (the qkv part's input, the o-projection's residual); nullptr: none
  const float* x_pend;
  int pend_n;
  int n_jobs;
  GemvJob jobs[MAX_JOBS];
};

// LDS floats for a chained-sum buffer of n values (whole 16-value chunks
// of the speculative sum are readable, with slack).
__host__ __device__ inline int chain_lds_floats(int n) { return ((n + 31) & ~31) + 64; }

struct NormParams {
  const float* x;
  const float* w;
  float eps;
  int n;
  int n_lds;    // chain_lds_floats(n)
  int out_sel;  // 1: write out_buf[state->nx_out] (the forward's last launch: advances state->epoch)
  float* out;
  float* out_buf[2];
  C2hState* state;
  int advance;  // step graphs: leave the state of the next step (pos, seq, normX buffers, RoPE row)
  const float* rope_cos;  // head_dim 64: the RoPE table the advance takes the next row from (else nullptr)
  const float* rope_sin;
  int rope_len;
  // the last layer's FFN launch left X's pending terms [FOLD_NB][n]: x is
  // X + their sum in block order, also written back to x_back; nullptr: none
  const float* x_pend;
  float* x_back;
};

// KV cache: [K|V][layer][kv head][kv_slot(max_ctx)][hd] floats.  K rows are
// position-major (row p at p*hd); V is quad-major within a head slot:
// element (p, d) at vq_index(p, d, hd), so positions 4q..4q+3 of dim d are
// 16 contiguous bytes and quad q (all dims) is 16*hd bytes.  The attention
// chains read four positions per 16-byte access and V chunks copy to LDS as
// is.
__host__ __device__ inline int kv_slot(int max_ctx) { return (max_ctx + 3) & ~3; }
__host__ __device__ inline size_t vq_index(int p, int d, int hd = 64) {
  return ((size_t)(p >> 2) * hd + d) * 4 + (p & 3);
}

// Attention of one layer over the q|k|v the QKV GEMV wrote: RoPE, KV store,
// scores, softmax, AV.  Two exact forms with the same arithmetic:
//   short contexts (T <= the context's split length): k_attn_core, one
//     workgroup per query head does everything with the scores in LDS;
//   long contexts: k_attn_scores (workgroups over position blocks, one K
//     row read for all query heads of a group) -> k_attn_softmax (one
//     workgroup per head, exps in LDS) -> k_attn_av (one workgroup per KV
//     head and 16-dim slice: two waves run the FMA chains of all the group's
//     query heads, the others stage the V slice through LDS).
constexpr int ATT_CH = 128;   // V positions staged in LDS per pass (chunk 0 prefetched)
constexpr int ATT_KPF = 256;  // K rows per LDS chunk of the scores (one per thread)
constexpr int ATT_KPAD = 68;  // floats per staged K row (64 + 4: conflict-free row reads)
// k_attn_core instances by the context they prefetch for: a tier of N
// positions serves T <= N positions attended and reads the first N rows of
// K and of V whole (a CU's loads issue at ~32-44 B/clk whether or not a
// row lies past the stored context, so the tiers step by 32 rows); the any
// tier serves any context up to the split length, K in chunks of ATT_KPF.
constexpr int ATT_TIER_ANY = 0;
constexpr int ATT_TIER_32 = 32;
constexpr int ATT_TIER_64 = 64;
constexpr int ATT_TIER_96 = 96;
constexpr int ATT_TIER_128 = 128;
constexpr int ATT_TIER_256 = 256;
__host__ __device__ inline int attn_tier(int T) {
  return T <= 32 ? ATT_TIER_32 : T <= 64 ? ATT_TIER_64 : T <= 96 ? ATT_TIER_96 : T <= 128 ? ATT_TIER_128
         : T <= 256 ? ATT_TIER_256 : ATT_TIER_ANY;
}
constexpr int ATT_SPLIT_T = 1024;  // default split length (positions attended)
constexpr int ATT_SB = 256;        // positions per k_attn_scores workgroup
constexpr int ATT_AV_CH = 256;     // positions per k_attn_av LDS chunk
constexpr int ATT_AV_THREADS = 256;  // k_attn_av: one chain wave, three staging waves
constexpr int ATT_AV_DSL = 8;        // k_attn_av: dims of a head per workgroup
constexpr int ATT_AV_SLICES = 64 / ATT_AV_DSL;
constexpr int ATT_AV_ITEMS = 6;      // 16-byte staging items per staging lane and chunk
constexpr int ATT_MAX_QPKV = 8;    // query heads per KV head the long form handles
constexpr int ATT_LONG_MAX_CTX = 36864;  // exps of one head in LDS (k_attn_softmax)
// grid (n_heads, tokens) for k_attn_core / k_attn_softmax / k_attn_av and
// (blocks, n_kv_heads, tokens) for k_attn_scores: query token i of a launch
// sits at position state->pos + tok0 + i; decode launches one token.
struct AttnCoreParams {
  const float* q;  // [tokens][q_ld]: n_heads*hd, bias added, before QK-norm and RoPE
  const float* k;  // [tokens][kv_ld]: n_kv_heads*hd
  const float* v;
  const float* q_norm;  // per-head QK-norm weights (hd floats each), nullptr: none
  const float* k_norm;
  float eps;
  float* out;      // attention output [tokens][out_ld]
  uint64_t* out_tag;  // k_attn_oproj: the output again as {value, tag} words
  int n_attn_wg;      // k_attn_oproj: workgroups of the attention half
  int* wait_err;      // k_attn_block: the flag a wait for q|k|v that runs out sets
  int q_ld, kv_ld, out_ld;
  int store_kv;    // 1: K/V of pos come from k/v and are stored by this launch
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
  int tok0;  // first query token of this launch within the q/k/v/out rows
  // long form: scores / probabilities sc[(i*n_heads + h)*sc_ld + p] of
  // launch token i, block maxima bmax[(i*n_heads + h)*n_blk + b]
  float* sc;
  float* bmax;
  int sc_ld;    // (k_pf_attn: the row stride of its LDS scores, pfa_sc_ld)
  int n_blk;
  int n_tok;    // k_pf_attn: query tokens of the prefill pass
  // k_attn_core: 1 = the grid is (ATT_XCDS * qpkv, 1, tokens), n_kv_heads
  // <= ATT_XCDS, and workgroup L serves KV head L % ATT_XCDS, query head
  // L / ATT_XCDS, so the workgroups of one KV head share an XCD and its L2
  // (workgroups go to the XCDs round robin); the workgroups left over exit
  // at once.  0 = the grid is (qpkv, n_kv_heads, tokens).
  int xcd_map;
};
constexpr int ATT_XCDS = 8;

// Causal attention of a prefill pass (k_pf_attn): one workgroup per query
// head and block of PFA_TB query tokens, K and V staged through LDS in
// chunks of PFA_CH positions shared by the block's tokens.
constexpr int PFA_TB = 8;
constexpr int PFA_WAVES_PER_EU = 3;  // occupancy the register budget is sized for (three workgroups per CU)
constexpr int PFA_CH = 128;
constexpr int PFA_KPAD = 68;  // floats per staged K row (64 + 4: conflict-free row reads)
// Row stride (floats) of the block's scores for positions up to pmax.
__host__ __device__ inline int pfa_sc_ld(int pmax) { return ((pmax + 1 + 63) & ~63) + 4; }
// Dynamic LDS of k_pf_attn, in floats: K chunk (V chunk aliases it) | q of
// the block's tokens | scores.
__host__ __device__ inline int pfa_lds_floats(int pmax) { return PFA_CH * PFA_KPAD + PFA_TB * 64 + PFA_TB * pfa_sc_ld(pmax); }

// Dynamic LDS of k_attn_h128 (head_dim 128), in floats: the scores of every
// position up to max_ctx, then (k_attn_h128<H128_VCH>) two chunks of
// H128_VCH positions of V.
constexpr int H128_VCH = 32;
constexpr int H128_VSETS = 6;  // V chunks of k_attn_h128 in flight
__host__ __device__ inline int attn_h128_lds_floats(int max_ctx) { return chain_lds_floats(max_ctx); }
__host__ __device__ inline int attn_h128_v_lds_floats() { return 2 * H128_VCH * 128; }

// Dynamic LDS of k_attn_core, in floats: the staged K rows of the scores
// (ATT_KPF padded rows), which the two staged V chunks of the AV chains
// later reuse | the scores.
__host__ __device__ constexpr int attn_kv_lds_floats() {
  return ATT_KPF * ATT_KPAD > 2 * ATT_CH * 64 ? ATT_KPF * ATT_KPAD : 2 * ATT_CH * 64;
}
__host__ __device__ inline int attn_lds_floats(int max_ctx) { return attn_kv_lds_floats() + chain_lds_floats(max_ctx); }
// Dynamic LDS of k_attn_softmax (exps of up to max_ctx positions) and of
// k_attn_av (three chunks of V quads and probabilities), in floats.
__host__ __device__ inline int attn_softmax_lds_floats(int max_ctx) { return (max_ctx + 3) & ~3; }
// probability rows of k_attn_av padded by 4 floats: the query heads' rows
// start in different LDS banks; three buffers of V quads and probabilities
constexpr int ATT_AV_PLD = ATT_AV_CH + 4;
constexpr int ATT_AV_LDS_FLOATS = 3 * (ATT_AV_CH * ATT_AV_DSL + ATT_MAX_QPKV * ATT_AV_PLD);

// ---- batched prefill (a prompt of up to PF_MAX tokens per pass)

constexpr int PF_TILE = 64;   // rows and tokens of one prefill GEMM workgroup
constexpr int PF_MAX = 512;   // tokens per prefill pass (buffers are sized for it)

// Q8_K rows of a token batch in global memory: token t, block b at
// q[(t*nbs + b)*256], d[t*nbs + b], bs[(t*nbs + b)*16] (bsums as int32).
struct PFQ8 {
  int8_t* q;
  float* d;
  int32_t* bs;
  int nbs;    // block stride per token
  float* dT;  // the scales again, block-major: block b, token t at dT[b*PF_MAX + t]
  // the quants again, by 32-element chunk: chunk k = 8b + c (elements
  // 32c .. 32c+32 of block b), token t at qT[(k*PF_MAX + t)*32]: 32 tokens'
  // chunk is 1 KB contiguous (the A operand of one k_pf_gemm_q6 MFMA)
  int8_t* qT;
};

// Per token: [embed tokens[t] into X[t]] RMSNorm(X[t]) * w -> Q8_K.
struct PFNormParams {
  int embed;
  int n_x;
  float eps;
  float* X;  // [m_pad][n_x]
  const float* norm_w;
  const int32_t* tokens;
  WeightRef emb;
  int n_vocab;
  int m;
  int nb;  // floor(n_x/256) blocks quantised
  PFQ8 out;
  float* xn;  // optional: the normalised rows [m_pad][n_x] as f32
};

// Per token: Q8_K of x[t][0 .. nb*256).
struct PFQuantParams {
  const float* x;
  int ld;
  int m;
  PFQ8 out;
};

struct PFJob {
  WeightRef w, w2;
  const uint4* w6;  // Q6_K: the split copy k_q6_pf_pack builds (k_pf_gemm_q6)
  int type, type2;
  int rows;
  int tile_begin;  // first row tile (blockIdx.x) of this job
  int mode;
  float* y;  // [m_pad][ldy]
  int ldy;
  const float* bias;
};

struct PFGemmParams {
  PFQ8 in;
  int nb;  // super-blocks per row
  int m;   // valid tokens
  int m_pad;
  int n_row_tiles;  // row tiles of all jobs (k_pf_gemm_q6)
  int n_jobs;
  PFJob jobs[3];
};

// Q5_0 / Q8_0 jobs of a batch on f32 rows x[t*ldx .. + n_x); grid (row
// tiles of the jobs, ceil(m / PF_FT)); tile_begin counts row tiles of
// max(1, 256/(n_x/32)) rows (Q5_0) or 32 rows (Q8_0).
constexpr int PF_FT = 16;  // tokens per k_pf_gemm_f workgroup
constexpr int PF_Q50_MAXB = 32;  // Q5_0 blocks per row of k_pf_gemm_q50 (wider rows run k_pf_gemm_f)
struct PFGemmFParams {
  const float* x;
  int ldx;
  int n_x;
  int m;
  int ft;  // k_pf_gemm_f: tokens per workgroup (<= PF_FT)
  int n_jobs;
  PFJob jobs[3];
};

// Per token and KV head: RoPE(k), then K/V stored at pos0 + t.
struct PFRopeParams {
  const float* k;
  const float* v;
  int ld;
  float* kv;
  const float* rope_cos;
  const float* rope_sin;
  int rope_len;
  int pos0;
  int m;
  int layer, n_layers, n_kv_heads, max_ctx;
};


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
__global__ void k_gemv_q8k(GemvParams P);
template <int NB, int PRO, int MODE>
__global__ void k_gemv_row(const float* xp, int n_xp, GemvParams P);  // xp, n_xp: P.x, P.n_x
// Q5_0 / Q8_0 projections on f32 x (PRO_QUANT here means "x as is").
template <int PRO, int MODE>
__global__ void k_gemv_f(GemvParams P);
constexpr int GF_XPAD = 36;  // floats per 32-element block of x in LDS (Q5_0 reads, bank spread)
// Dynamic LDS of k_pf_gemm_f, bytes: x of one token in both layouts.
__host__ __device__ inline int pf_gemm_f_lds_bytes(int n_x) {
  const int nb8 = n_x / 32;
  return (nb8 * GF_XPAD + nb8 * 32) * 4;
}
// Dynamic LDS of k_pf_gemm_q50, bytes: x of half the tokens, the terms.
__host__ __device__ inline int pf_gemm_q50_lds_bytes(int n_x) {
  return ((PF_FT / 2) * (n_x / 32) * GF_XPAD + PF_FT * 256) * 4;
}
constexpr int PF_F_LDS_MAX = ((PF_FT / 2) * PF_Q50_MAXB * GF_XPAD + PF_FT * 256) * 4;
// Dynamic LDS of k_gemv_f, in floats: x padded per block | x permuted | norm chain.
__host__ __device__ inline int gemv_f_lds_floats(int n_x) {
  return (n_x / 32) * GF_XPAD + (n_x / 32) * 32 + chain_lds_floats(n_x);
}
__global__ void k_rmsnorm(NormParams P);
template <int TIER>
__global__ void k_attn_core(C2hState* st, float* kv, const float* qg, const float* kg, const float* vg, int dims,
                            int max_ctx, AttnCoreParams P);  // (P.state, P.kv, P.q, P.k, P.v, attn_dims, P.max_ctx)
// k_attn_core's XCD-grouped grid (P.n_attn_wg workgroups) followed by the
// o-projection's k_gemv_row<NB, PRO_QUANT, MODE_RESID> workgroups of G,
// 256 threads each, one launch; G.x_tag = P.out_tag
// gate|up (xw >> 16 workgroups), then the Q6_K down projection by
// super-block (Gd.jobs[0].n_wg = NBF * ceil(rows / 128) workgroups), 512
// threads each, one launch; Gi.y_tag = Gd.x_tag (h); the terms go to
// Gd.jobs[0].y as [NBF][rows], for the next k_attn_block to add to X
// (GemvParams::x_pend)
// the down blocks of the FFN launch, whose terms the next launch adds to X
constexpr int FOLD_NB = 19;
// k_gemv_row that adds X's pending terms (GemvParams::x_pend) to its norm
// input (PRO_NORM) or residual (MODE_RESID); instances <3, PRO_NORM,
// MODE_BIAS> and <3, PRO_QUANT, MODE_RESID>
template <int NB, int PRO, int MODE>
__global__ void k_gemv_row_pend(const float* xp, int n_xp, GemvParams P);
template <int NBE, int NBF>
__global__ void k_ffn_block(const float* xp, int xw, C2hState* st, int layer, GemvParams Gi, GemvParams Gd);
// The same with Q5_0 / Q8_0 gate|up (k_gemv_f's workgroups, xw >> 16 of
// them), 256 threads per workgroup, the down projection in rows of 64
// (Gd.jobs[0].n_wg = NBF * ceil(rows / 64))
template <int NBF>
__global__ void k_ffn_block_f(C2hState* st, int xw, int layer, GemvParams Gi, GemvParams Gd);
// qkv (3 W workgroups, W = xw >> 16), then k_attn_oproj's two parts, one
// launch; Gq.y_tag = qkv_tag, Go.x_tag = P.out_tag
template <int TIER, int NB>
__global__ void k_attn_block(C2hState* st, float* kv, const float* xp, int xw, const uint64_t* qkv_tag, int dims,
                             int max_ctx, AttnCoreParams P, GemvParams Gq, GemvParams Go);
// k_attn_block with k_gemv_f's float-input q|k|v and o-projection parts
template <int TIER>
__global__ void k_attn_block_f(C2hState* st, float* kv, const float* xp, int xw, const uint64_t* qkv_tag, int dims,
                               int max_ctx, AttnCoreParams P, GemvParams Gq, GemvParams Go);
template <int TIER, int NB>
__global__ void k_attn_oproj(C2hState* st, float* kv, const float* qg, const float* kg, const float* vg, int dims,
                             int max_ctx, AttnCoreParams P, GemvParams G);
// layer | n_layers << 8 | n_kv_heads << 16 | xcd_map << 23 | query heads per KV head << 24
inline int attn_dims(const AttnCoreParams& A, int qpkv) {
  return A.layer | (A.n_layers << 8) | (A.n_kv_heads << 16) | ((A.xcd_map ? 1 : 0) << 23) | (qpkv << 24);
}
__global__ void k_attn_scores(AttnCoreParams P);
__global__ void k_attn_softmax(AttnCoreParams P);
__global__ void k_attn_av(AttnCoreParams P);
template <int VCH>
__global__ void k_attn_h128(AttnCoreParams P);
__global__ void k_pf_attn(AttnCoreParams P);
template <int NB>
__global__ void k_pf_norm_quant(PFNormParams P);
template <int NB>
__global__ void k_pf_quant(PFQuantParams P);
template <int TYPE, int MODE, int TT>  // TT: 16-token sub-tiles per wave (64 or 16 tokens per workgroup)
__global__ void k_pf_gemm(PFGemmParams P);
// Q6_K jobs of a prefill: the reference's integer super-block sum
// isum = sum over sub-blocks of sc * sum(q8 * (q6 - 32)) is, element by
// element, sum(q8 * B) with B = (q6 - 32) * sc in [-4064, 4096], which
// splits exactly into int8 parts hi = B >> 6 (in [-64, 64]) and lo = B & 63:
// isum = 64 * sum(q8 * hi) + sum(q8 * lo), two int8 GEMMs over the 256
// elements.  k_q6_pf_pack writes that split copy of a Q6_K matrix (rows
// padded to 32): per (32-row tile, super-block, 32-element chunk c, part
// hi | lo) 1 KB, lane l's 16 bytes = row l % 32, elements
// 32c + 16 * (l / 32) .. +16 -- one v_mfma_i32_32x32x32_i8 B operand.
// Grid (row tiles, super-blocks), 64 threads.
constexpr size_t PF_Q6_TILE_BYTES = 32 * 512;  // one 32-row tile of one super-block
__global__ void k_q6_pf_pack(WeightRef w, int rows, int nb, uint4* out);
// NS waves per 32 tokens x 32 rows (the super-blocks split between them);
// a 1-D grid of 8 * ceil(n_row_tiles * m_pad / 32 / 8) workgroups of 64 NS
// threads (tile_begin and n_row_tiles in 32-row tiles); dynamic LDS of
// pf_q6_lds_bytes(nb, NS).
template <int MODE, int NS>
__global__ void k_pf_gemm_q6(PFGemmParams P);
__host__ __device__ inline int pf_q6_lds_bytes(int nb, int ns) {
  const int per = (nb + ns - 1) / ns;
  return ns > 1 ? (nb - per) * 16 * 64 * 4 : 0;
}
constexpr int PF_Q6_LDS_MAX = 128 * 1024;

template <int MODE>
__global__ void k_pf_gemm_f(PFGemmFParams P);
template <int MODE>
__global__ void k_pf_gemm_q50(PFGemmFParams P);
__global__ void k_pf_rope_store(PFRopeParams P);
__global__ void k_pf_swiglu(const float* gate, const float* up, float* h, int n, int m);
template <int NB8>
__global__ void k_vocab(const uint8_t* wq, C2hState* st, const float* xb0, const float* xb1, int n_vocab,
                        VocabParams P);  // (P.w.q, P.state, x_buf[0] or x, x_buf[1] or x, P.n_vocab)
constexpr int VOCAB_MIN_NB8 = 24, VOCAB_MAX_NB8 = 32;  // instantiated widths (Q8_0 blocks per row), and 64
// An f32 input vector: x itself, or (sel) the normX buffer the step state
// names, for kernels inside replayed graphs.
struct XSel {
  const float* x;
  const float* buf[2];
  const C2hState* state;
  int sel;
};

struct PickParams {
  const float* logits;
  int n_vocab;
  const int32_t* token_ids;
  int apply_penalty;
  const C2hState* state;
  float* part_v;
  int* part_i;
};
__global__ void k_logits_pick(PickParams P);
__global__ void k_quantize_q8k_sel(XSel X, int nb, uint8_t* __restrict__ y);

// One f32 dot per output (float-x order of each format).  Output i is row
// ids[i] when ids is given (ids outside [0, rows) are skipped), else row i;
// it is stored to y[ids[i]] when scatter is set, else to y[i].  x is 16-byte
// aligned and holds cols floats.
struct DotRowsParams {
  WeightRef w;
  int rows, cols;
  XSel X;
  const int32_t* ids;
  int n;
  int scatter;
  float* y;
};
template <int TYPE>
__global__ void k_dot_rows(DotRowsParams P);
constexpr int DOT_ROWS_PER_WG = 32;
constexpr int DOT_MAX_COLS = 32768;  // x staged in LDS: 128 KB
// Dynamic LDS of k_dot_rows: x of the row's whole groups (32 floats each).
__host__ __device__ inline int dot_rows_lds_bytes(int type, int cols) {
  return (type == 12 || type == 14) ? (cols / 256) * 256 * 4 : (cols / 32) * 32 * 4;  // Q4_K, Q6_K: whole super-blocks
}
__global__ void k_argmax_final(const float* pv, const int* pi, int n, C2hState* state);
__global__ void k_copy16(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n16);
__global__ void k_empty(const int* __restrict__ flag, int* __restrict__ out);
// One wave that returns after `ticks` of the 100 MHz real-time counter
// (bounded: the caller passes at most C2H_DELAY_MAX_TICKS); a timing call
// puts it ahead of eager launches so that they run paced by the GPU, not by
// the host's enqueue rate.
constexpr long long C2H_DELAY_MAX_TICKS = 1000000;  // 10 ms
__global__ void k_delay(long long ticks);
// st->epoch += 1 (one workgroup of 64): the tags launches store after it
// differ from every tag stored before it
__global__ void k_next_epoch(C2hState* st);
// st->epoch += 1: the tags launches store after it differ from every tag
// stored before it
__global__ void k_next_epoch(C2hState* st);
// Producer -> consumer wait in one launch (measurement of the cost of
// replacing a kernel boundary by a counter wait).  Workgroups below n_prod
// (mode 0) are producers: a dependent chain of `work` steps, then their
// share of data_floats outputs, stored with agent-scope stores; once those
// are complete, one agent-scope atomic add per workgroup on counter
// blockIdx % 8.  The others are consumers: they load a 16 KB weight slice,
// then poll the counters (relaxed agent-scope loads, s_sleep between polls)
// until their sum reaches `target`, read every output with agent-scope loads
// and check it.  proto 1 drops the counters: every output is one 8-byte
// agent-scope store of {value, epoch}, and a consumer polls the outputs it
// reads until each carries the launch's epoch.
// mode 1: producers only (no counter); mode 2: consumers only
// (no wait): the same work split over two launches.  Every wait is bounded
// by spin_limit polls; a consumer that runs out sets err[0] = 1 and exits,
// a wrong output value adds to err[1].
struct PcBenchParams {
  unsigned* counters;     // 8 counters, 64 dwords apart
  float* data;            // [data_floats]
  const uint4* weights;   // consumer prefetch: 1,024 uint4 per (launch, consumer)
  float* out;             // one value per consumer workgroup
  int* err;               // [2]
  uint64_t* data_ll;      // proto 1: [data_floats] of {value bits, epoch}
  int n_prod, n_cons, mode, epoch, spin_limit, data_floats, work, w_index;
  int proto;              // 0: counters; 1: each output carries its epoch (no counter)
};
__global__ void k_pc_bench(PcBenchParams P);
__global__ void k_fill_u32(unsigned* p, int n, unsigned v);
__global__ void k_check_rms_scale(uint32_t lo, uint32_t n, unsigned long long* bad, uint32_t* first);

}  // namespace c2h
