/*
 * c2h.h — C ABI of the MI355X (gfx950) decode path for c2slm.
 *
 * Plain C: pointers, sizes and status codes; no exceptions cross it.  Every
 * entry point selects the context's device first (cgo calls may land on any
 * OS thread).  A context owns one HIP stream and all device buffers; it is
 * not safe for concurrent use, like the reference's Engine
 * (engine/pool.go:22-42 keeps unsynchronised task state).
 *
 * Status: 0 = OK, < 0 = error; c2h_last_error() describes the last failure.
 */
#ifndef C2H_H
#define C2H_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define C2H_OK 0
#define C2H_ERR_INVALID (-1)     /* bad argument or shape */
#define C2H_ERR_HIP (-2)         /* a HIP runtime call failed */
#define C2H_ERR_UNSUPPORTED (-3) /* format or shape this build does not run */
#define C2H_ERR_STATE (-4)       /* model incomplete / wrong call order */
#define C2H_ERR_RANGE (-5)       /* position beyond the KV cache */

/* ggml tensor types (gguf/reader.go:21-37) */
#define C2H_F32 0
#define C2H_Q5_0 6
#define C2H_Q8_0 8
#define C2H_Q4_K 12
#define C2H_Q6_K 14

/* Tensor roles: what engine/model.go:114-207 binds.  Per-layer roles take
 * the layer index; global roles ignore it. */
enum c2h_role {
  C2H_ROLE_TOKEN_EMBD = 0,  /* token_embd.weight (also the tied output) */
  C2H_ROLE_OUTPUT = 1,      /* output.weight, when present */
  C2H_ROLE_OUTPUT_NORM = 2, /* output_norm.weight */
  C2H_ROLE_ATTN_NORM = 10,
  C2H_ROLE_ATTN_Q = 11,
  C2H_ROLE_ATTN_Q_BIAS = 12,
  C2H_ROLE_ATTN_K = 13,
  C2H_ROLE_ATTN_K_BIAS = 14,
  C2H_ROLE_ATTN_V = 15,
  C2H_ROLE_ATTN_V_BIAS = 16,
  C2H_ROLE_ATTN_OUT = 17,
  C2H_ROLE_FFN_NORM = 18,
  C2H_ROLE_FFN_GATE = 19,
  C2H_ROLE_FFN_UP = 20,
  C2H_ROLE_FFN_DOWN = 21,
  C2H_ROLE_ATTN_Q_NORM = 22, /* Qwen3 blk.N.attn_q_norm.weight (head_dim floats, engine/model.go:168-170) */
  C2H_ROLE_ATTN_K_NORM = 23  /* Qwen3 blk.N.attn_k_norm.weight (engine/model.go:177-179) */
};

/* Model dimensions, as engine.LoadModel resolves them (engine/model.go:64-145). */
typedef struct c2h_model_desc {
  int32_t n_layers;   /* qwen2.block_count, else qwen3.block_count (24; Qwen3-1.7B 28) */
  int32_t n_embd;     /* *.embedding_length (896; 2048) */
  int32_t n_heads;    /* *.attention.head_count (14; 16) */
  int32_t n_kv_heads; /* *.attention.head_count_kv (2; 8) */
  int32_t head_dim;   /* n_embd / n_heads (64; 128), engine/model.go:137 */
  int32_t n_ff;       /* *.feed_forward_length (4864; 6144) */
  int32_t n_vocab;    /* token_embd dims[1] (151936) */
  int32_t max_ctx;    /* KV positions; engine.MaxContextLen = 16384 (engine/kvcache.go:11);
                         this build runs up to 36864 at head_dim 64, 38848 at 128 */
  float rms_eps;      /* 1e-6 */
  float rope_theta;   /* 1e6 */
  int32_t reserved[6];
} c2h_model_desc;

typedef struct c2h_ctx c2h_ctx;

/* ---- context ------------------------------------------------------------ */

/* Replaces engine.LoadModel's model setup plus engine.NewKVCache and
 * engine.NewArena (engine/model.go:58-210, engine/kvcache.go:49-81,
 * engine/forward.go:28-43): allocates weights, fp32 KV cache
 * [2][L][KVH][max_ctx][HD], activations, and the RoPE table built on the host
 * in float64 exactly as tensor.NewRoPETable (tensor/ops.go:237-257).
 * desc == NULL creates a kernel-only context (stream + scratch) for the
 * c2h_*_dev and c2h_quantize_q8k / c2h_gemv entry points. */
int c2h_create(const c2h_model_desc* desc, int device, c2h_ctx** out);

/* Frees everything (Engine.Close, c2slm.go:44-55).  NULL is a no-op. */
void c2h_destroy(c2h_ctx* ctx);

/* Text of the last error on this context (static text for ctx == NULL). */
const char* c2h_last_error(const c2h_ctx* ctx);

/* Uploads one tensor once, replacing the reference's []byte views into the
 * mmap (gguf/reader.go:497-508) that the hot path reads per token.  `host`
 * is borrowed for the call only.  Quantized rows use the reference's row
 * stride (cols/QK)*blockSize (tensor/ops.go:26,78,121,183), so a 896-wide
 * K-quant row covers 3 super-blocks exactly as the reference reads it;
 * `bytes` must cover rows*stride.  Types: Q4_K/Q6_K/Q5_0/Q8_0 projections
 * (Q4_K/Q6_K multiply a Q8_K row, Q5_0/Q8_0 the f32 input, as
 * engine/model.go:250-270 dispatches; Q8_0 projections up to 1024 columns),
 * Q8_0 embedding, Q8_0/Q4_K/Q6_K/Q5_0 output (the vocab projection:
 * Q8_0 through the fused projection + penalty + argmax kernel, the others
 * as ParallelGEMV computes them, engine/pool.go:122-154), F32 norms and
 * biases. */
int c2h_upload_tensor(c2h_ctx* ctx, int32_t layer, int32_t role, int32_t ggml_type, int64_t rows, int64_t cols,
                      const void* host, size_t bytes);

/* Mirrors KVCache.StoreTokenID (engine/kvcache.go:120-125) for ids the
 * device did not write itself; c2h_forward and c2h_step record their own. */
int c2h_set_token_ids(c2h_ctx* ctx, int32_t pos0, const int32_t* ids, int32_t n);

/* Reads KVCache.TokenIDs[pos0 .. pos0+n) (engine/kvcache.go:25-47), the
 * token fingerprint c2slm_test.go:76-80 checks. */
int c2h_get_token_ids(c2h_ctx* ctx, int32_t pos0, int32_t n, int32_t* out);

/* KVCache.SeqLen (engine/kvcache.go:25-47): the count of materialised
 * positions.  c2h_forward(pos) and c2h_step(pos) set it to pos+1 and
 * c2h_prefill to pos0+n, as Engine.IngestFrom and generate do
 * (c2slm.go:114,187,200,222).  c2h_set_seq is KVCache.Reset (seq_len 0,
 * engine/kvcache.go:101-103) and Rewind (engine/kvcache.go:109-117): no
 * memory moves; entries past the cursor stay until overwritten.
 * seq_len outside [0, max_ctx] returns C2H_ERR_RANGE. */
int c2h_set_seq(c2h_ctx* ctx, int32_t seq_len);
int c2h_get_seq(c2h_ctx* ctx, int32_t* seq_len);

/* ---- decode path -------------------------------------------------------- */

/* engine.Forward(m, cache, a, token, pos) (engine/forward.go:54-138): one
 * decoder step for `token` at `pos`, storing K/V at pos and
 * TokenIDs[pos] = token; writes the final normX to normx_out (n_embd floats,
 * nullable).  pos outside [0, max_ctx) returns C2H_ERR_RANGE (the reference
 * skips RoPE and the KV store silently there, engine/kvcache.go:144-146). */
int c2h_forward(c2h_ctx* ctx, int32_t token, int32_t pos, float* normx_out);

/* Engine.IngestFrom's loop (c2slm.go:107-115: engine.Forward per token at
 * pos0, pos0+1, ...; TokenIDs recorded) for n tokens at once: each layer runs
 * over the whole batch (int8 MFMA GEMMs, causal attention), with every
 * token's arithmetic identical to Forward's, so the KV cache and the final
 * normX (written to normx_out, nullable) equal sequential ingest bit for
 * bit.  Batches of up to 512 tokens per pass.  [pos0, pos0+n) must lie in
 * [0, max_ctx) (C2H_ERR_RANGE otherwise). */
int c2h_prefill(c2h_ctx* ctx, const int32_t* tokens, int32_t n, int32_t pos0, float* normx_out);

/* engine.ComputeLogits(m, a, normX, out, nil) (engine/forward.go:171-191) on
 * the current normX: n_vocab fp32 logits to logits_out. */
int c2h_logits(c2h_ctx* ctx, float* logits_out);

/* One iteration of the generate loop body (c2slm.go:153-222): logits of the
 * current normX, repetition penalty over TokenIDs[max(0,pos-64), pos)
 * skipping im_end/eos, greedy argmax (lowest id on ties), then
 * engine.Forward(best, pos) and TokenIDs[pos] = best.  Only the chosen id
 * crosses to the host.  The new normX becomes current; c2h_restore_normx
 * undoes that for a caller that rejects the token (stop strings,
 * c2slm.go:205-216).  The call returns once the chosen id is known (the
 * step's first layer hands it over through pinned memory); the forward of
 * that token then completes on the context's stream, before any later call
 * on the context reads or writes device state, so results are the same as
 * if the call had waited (c2h_sync waits for it explicitly). */
int c2h_step(c2h_ctx* ctx, int32_t pos, float penalty, int32_t im_end, int32_t eos, int32_t* next_token);

/* Makes the normX that was current before the last c2h_step current again. */
int c2h_restore_normx(c2h_ctx* ctx);

/* Copies the current normX (n_embd floats) to the host. */
int c2h_get_normx(c2h_ctx* ctx, float* normx_out);

/* Copies K or V (which = 0/1) of one layer/KV head for positions [0, n) to
 * the host ([n][head_dim] floats): KVCache.GetKey/GetValue
 * (engine/kvcache.go:159-169). */
int c2h_get_kv(c2h_ctx* ctx, int32_t which, int32_t layer, int32_t kv_head, int32_t n, float* out);

/* The reverse copy, KVCache.StoreKV (engine/kvcache.go:143-157) for a run of
 * positions of one layer/KV head: src holds [n][head_dim] floats written to
 * positions [pos0, pos0+n) of K or V (which = 0/1); for callers that restore
 * or pre-fill a cache.  The range must lie in [0, max_ctx). */
int c2h_set_kv(c2h_ctx* ctx, int32_t which, int32_t layer, int32_t kv_head, int32_t pos0, int32_t n,
               const float* src);

/* ---- kernel entry points (tensor/ops.go operators) ----------------------- */

/* tensor.QuantizeRowQ8_K (tensor/ops.go:170-172): floor(cols/256) blocks of
 * 292 bytes (f32 d | int8 qs[256] | int16 bsums[16]) from host x. */
int c2h_quantize_q8k(c2h_ctx* ctx, const float* x, int32_t cols, void* q8k_out);

/* No counterpart in the reference: c2h_quantize_q8k for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments, results and
 * errors, but it calls no allocator: x and the Q8_K blocks are staged in a
 * fixed device scratch, one per GPU, set up by c2h_create.  cols above
 * C2H_NOALLOC_MAX_COLS returns C2H_ERR_INVALID.  Every context on a GPU
 * shares that GPU's scratch.  Calls from one process take a per-GPU lock
 * from the copy in to the copy out, so they run one after another; calls
 * from different processes on one GPU each have their own scratch. */
#define C2H_NOALLOC_MAX_COLS 16384 /* 64 Q8_K super-blocks: 84 KB of device scratch per GPU */
int c2h_quantize_q8k_noalloc(c2h_ctx* ctx, const float* x, int32_t cols, void* q8k_out);

/* tensor.GEMVQ4_K_Q8_K / GEMVQ6_K_Q8_K / GEMVQ8_0 / GEMVQ5_0
 * (tensor/ops.go:25-203) on host buffers.  w is the reference's native
 * layout (row stride as above); xq is the Q8_K row for Q4_K/Q6_K and the
 * f32 vector for Q8_0 and Q5_0.
 * isums_out (nullable, K-quants only) receives the integer sums: Q4_K 8 per
 * (row, super-block), the 32-element sums in q8 order; Q6_K 1 per
 * (row, super-block), the scaled super-block sum. */
int c2h_gemv(c2h_ctx* ctx, int32_t ggml_type, const void* w, const void* xq, int32_t rows, int32_t cols, float* y,
             int32_t* isums_out);

/* Device-layout size and host-side repack of one weight tensor
 * (native reference layout -> the layout the kernels read).  Byte count
 * per row is unchanged except for alignment padding of Q8_0 rows whose
 * block count is not a multiple of 4. */
size_t c2h_packed_size(int32_t ggml_type, int64_t rows, int64_t cols);
int c2h_pack_weights(int32_t ggml_type, int64_t rows, int64_t cols, const void* native, size_t native_bytes,
                     void* packed, size_t packed_bytes);

/* Device-pointer forms for device-resident pipelines and measurement; they
 * run on the context stream and return without synchronising
 * (c2h_sync waits).  w_packed is in the c2h_pack_weights layout; x of
 * c2h_quantize_q8k_dev is 16-byte aligned (C2H_ERR_INVALID otherwise). */
int c2h_quantize_q8k_dev(c2h_ctx* ctx, const float* x, int32_t cols, void* q8k_out);
int c2h_gemv_dev(c2h_ctx* ctx, int32_t ggml_type, const void* w_packed, const void* xq, int32_t rows, int32_t cols,
                 float* y, int32_t* isums_out);
int c2h_sync(c2h_ctx* ctx);

/* engine.DispatchGEMV with a nil pool (engine/model.go:250-270): y = W·x on
 * the f32 vector x through each format's float row function --
 * tensor.GEMVQ4_K / GEMVQ6_K (DotQ4_K / DotQ6_K, tensor/ops.go:112-168),
 * GEMVQ8_0 and GEMVQ5_0 (tensor/ops.go:25-110) -- over floor(cols/256)
 * super-blocks or floor(cols/32) blocks per row.  Any other ggml type, or a
 * row with no whole block, yields zeros (the reference's fallback).  Host
 * buffers; w in the native layout, x holds cols floats. */
int c2h_gemv_f32(c2h_ctx* ctx, int32_t ggml_type, const void* w, const float* x, int32_t rows, int32_t cols,
                 float* y);
/* Device-pointer form: w_packed in the c2h_pack_weights layout, x 16-byte
 * aligned; runs on the context stream without synchronising. */
int c2h_gemv_f32_dev(c2h_ctx* ctx, int32_t ggml_type, const void* w_packed, const float* x, int32_t rows,
                     int32_t cols, float* y);

/* engine.ComputeLogits(m, a, normX, out, targetTokens) with a target list
 * (engine/forward.go:171-212) on the current normX: for each id of ids in
 * [0, n_vocab), logits_out[id] = DotQ*(row id of the output matrix, normX)
 * (computeSingleTokenLogit: the float-x dot of the output's format, also
 * for K-quants, whose full projection uses the Q8_K row instead);
 * out-of-range ids are skipped and every other entry of logits_out (n_vocab
 * floats) is left as it was.  n_ids == 0 projects the whole vocabulary like
 * c2h_logits (the reference's empty-list branch). */
int c2h_logits_ids(c2h_ctx* ctx, const int32_t* ids, int32_t n_ids, float* logits_out);
/* Device-pointer form (ids and logits in device memory, logits n_vocab
 * floats); runs on the context stream without synchronising. */
int c2h_logits_ids_dev(c2h_ctx* ctx, const int32_t* ids, int32_t n_ids, float* logits);

/* ---- measurement --------------------------------------------------------- */

/* Average device time (ms) of `iters` launches of the fused vocab projection
 * + penalty + argmax kernel, each bracketed by its own pair of HIP events on
 * the context stream; uses the current normX and pos.  With in_step != 0 a
 * forward pass (token 0 at pos, all layers) runs between launches, so the
 * 144 MB matrix is read from HBM as inside a decode step rather than from
 * the 256 MB last-level cache; that forward pass overwrites the KV entry at
 * pos and the non-current normX buffer.  With in_step == 0 the launches run
 * back to back.  With in_step == 2 they run back to back alternating
 * between the matrix and a device copy of it (twice the matrix in flight,
 * more than the last-level cache holds, so every launch reads its rows from
 * HBM), timed by one pair of events around all of them. */
int c2h_time_vocab(c2h_ctx* ctx, int32_t iters, int32_t pos, int32_t in_step, float* ms_per_launch);

/* Measurement aid with no counterpart in the reference: average device time
 * (ms) of `iters` launches of the float-x row dots behind c2h_gemv_f32 and
 * c2h_logits_ids, each bracketed by HIP events on the context stream.  Host
 * inputs (w in the native layout, x of cols floats, ids nullable) are
 * uploaded first; without ids rows 0..n-1 are computed, with ids the n
 * listed rows.  With flush_bytes > 0 a device copy of flush_bytes bytes runs
 * before each launch (not timed), so the matrix comes from HBM rather than
 * the last-level cache.  y_out (nullable) receives the n results. */
int c2h_time_dot_rows(c2h_ctx* ctx, int32_t ggml_type, const void* w, const float* x, int32_t rows, int32_t cols,
                      const int32_t* ids, int32_t n, int32_t iters, int64_t flush_bytes, float* y_out,
                      float* ms_per_launch);

/* Measurement aid with no counterpart in the reference: `reps` plain
 * device-to-device copies of `bytes` (a multiple of 16) between two scratch
 * buffers it allocates and frees; the average ms per copy.  Its known
 * traffic calibrates the memory counters of a profiler run. */
int c2h_copy_bench(c2h_ctx* ctx, int64_t bytes, int32_t reps, float* ms_per_copy);

/* Measurement aid with no counterpart in the reference: the device time
 * (µs) per kernel of a captured graph of `n` dependent launches of an empty
 * kernel (`grid` workgroups of 256 threads), best of `reps` replays -- the
 * floor a chain of decode kernels pays per launch. */
int c2h_launch_floor(c2h_ctx* ctx, int32_t n, int32_t grid, int32_t reps, float* us_per_kernel);

/* Measurement aid with no counterpart in the reference: the cost of a
 * producer -> consumer dependency inside one launch against a kernel
 * boundary.  Fused: `n_launch` dependent launches of n_prod + n_cons
 * workgroups (256 threads); the producers run `work` dependent float steps,
 * store 896 floats between them and signal per-XCD counters; the consumers
 * prefetch 16 KB of weights each, wait on the counters (bounded), then read
 * and check the 896 floats.  Split: the same work as a producer launch then
 * a consumer launch, n_launch times.  Best of `reps` graph replays; µs per
 * fused launch and per split pair.  proto 0 signals through the counters;
 * proto 1 stores each float with its launch number in one 8-byte store and
 * the consumers poll the floats themselves (no counter).  C2H_ERR_HIP if a
 * wait ran out or a consumer read a stale value. */
int c2h_time_producer_consumer(c2h_ctx* ctx, int32_t n_prod, int32_t n_cons, int32_t work, int32_t n_launch,
                               int32_t reps, int32_t proto, float* us_fused, float* us_split);

/* Self-check with no counterpart in the reference: the RMSNorm scale
 * f32(1/sqrt(f64(v))) as the kernels compute it (a reciprocal square root
 * estimate and one Newton step for normal positive v) against the IEEE
 * square root and division, for every float whose bit pattern lies in
 * [lo, hi) (hi <= 2^32); *mismatches receives their number (0 expected, NaN
 * results of either form equal) and *first_bits the lowest mismatching
 * pattern (0xffffffff if none). */
int c2h_check_rms_scale(c2h_ctx* ctx, uint32_t lo, uint64_t hi, uint64_t* mismatches, uint32_t* first_bits);

/* Kernels of one decoder layer, for c2h_time_layer_kernel. */
#define C2H_KERNEL_QKV 0        /* RMSNorm + Q8_K + q|k|v GEMV + bias */
#define C2H_KERNEL_ATTN 1       /* RoPE, KV store, scores, softmax, AV */
#define C2H_KERNEL_ATTN_OUT 2   /* Q8_K(attn) + o GEMV + residual */
#define C2H_KERNEL_FFN_IN 3     /* RMSNorm + Q8_K + gate|up GEMV + SwiGLU */
#define C2H_KERNEL_FFN_OUT 4    /* Q8_K(h) + down GEMV + residual */
#define C2H_KERNEL_FINAL_NORM 5 /* the final RMSNorm */
/* The launches a decode step runs where the model has their instances
 * (head_dim 64, K-quant projections, rows of 3 super-blocks; C2H_ERR_UNSUPPORTED
 * otherwise): */
#define C2H_KERNEL_ATTN_BLOCK 6 /* QKV + ATTN + ATTN_OUT in one launch (layers past 0) */
#define C2H_KERNEL_ATTN_OPROJ 7 /* ATTN + ATTN_OUT in one launch (layer 0) */
#define C2H_KERNEL_FFN_BLOCK 8  /* FFN_IN + FFN_OUT but the residual add in one launch (Q6_K down of 19 blocks) */

/* Measurement aid with no counterpart in the reference: average device time
 * (ms) of one decoder-layer kernel, `iters` launches back to back on the
 * context stream between one pair of HIP events (captured != 0: as one
 * captured graph, replayed once untimed first, unless the context runs
 * without graphs (C2H_NO_GRAPH=1); 0: eager launches, behind a short
 * bounded wait on the GPU so that the host has enqueued them all before the
 * first runs), layer
 * i % n_layers on launch i (so each launch reads another layer's weights,
 * as inside a step), after one untimed round over the layers.  The q|k|v kernel runs the
 * later layers' prologue (RMSNorm of X) on every layer.  Inputs are the
 * context's current buffers, at position SeqLen, which must be below
 * max_ctx (else C2H_ERR_RANGE): the attention kernel writes the KV entries
 * of that position, which no later read depends on until a forward or step
 * at SeqLen rewrites them; X, which the residual kernels update, is restored
 * afterwards, and so is the normX buffer the final-norm kernel writes (the
 * one c2h_restore_normx switches back to).  A fused kernel (6-8) is timed
 * only where every layer's tensors are of the types it reads, at SeqLen + 1
 * attended positions (else C2H_ERR_UNSUPPORTED); the call ends by advancing
 * the state's handover epoch, so the next forward takes none of the words
 * they left. */
int c2h_time_layer_kernel(c2h_ctx* ctx, int32_t kernel, int32_t iters, int32_t captured, float* ms_per_launch);

/* Measurement aid with no counterpart in the reference: average device time
 * (ms) of the operator GEMV behind c2h_gemv_dev (tensor.GEMVQ4_K_Q8_K /
 * GEMVQ6_K_Q8_K / GEMVQ8_0 / GEMVQ5_0), `iters` launches between one pair of
 * HIP events.  Host inputs: w in the native layout, xq the Q8_K row (K-quants)
 * or the f32 vector.  With rotate_bytes > 0 the launches rotate over enough
 * device copies of w to cover rotate_bytes (more than the 256 MB last-level
 * cache: each launch reads w from HBM); with 0 they reuse one copy. */
int c2h_time_gemv(c2h_ctx* ctx, int32_t ggml_type, const void* w, const void* xq, int32_t rows, int32_t cols,
                  int32_t iters, int64_t rotate_bytes, float* ms_per_launch);

/* The same for the quantiser behind c2h_quantize_q8k_dev on cols (256..16384)
 * host floats x. */
int c2h_time_quantize_q8k(c2h_ctx* ctx, const float* x, int32_t cols, int32_t iters, int64_t rotate_bytes,
                          float* ms_per_launch);

/* Average device time (ms) of `iters` decode steps (graph replays) at
 * positions pos, pos+1, ...; tokens are fed back on the device, and the
 * state is copied once: each step's final norm advances it for the next. */
int c2h_time_steps(c2h_ctx* ctx, int32_t pos, int32_t iters, float penalty, int32_t im_end, int32_t eos,
                   float* ms_per_step);

#ifdef __cplusplus
}
#endif
#endif /* C2H_H */
