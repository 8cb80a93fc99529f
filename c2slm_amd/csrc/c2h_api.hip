// Host side of the C ABI in include/c2h.h: context, weight upload and
// repack, HIP-graph capture of the decode step, and the entry points.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <initializer_list>
#include <cstdio>
#include <mutex>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/c2h.h"
#include "c2h_device.h"
#include "c2h_kernels.h"

using namespace c2h;

namespace {

constexpr int kStateRing = 256;
constexpr int PF_ATT_SUB = 16;  // batch tokens per long-context attention launch

struct Tensor {
  uint8_t* q = nullptr;
  uint16_t* d = nullptr;
  uint4* pf6 = nullptr;  // Q6_K: the split copy batched prefill reads (built at its first use)
  int type = -1;
  int64_t rows = 0, cols = 0;
  bool present() const { return q != nullptr; }
  WeightRef ref() const { return WeightRef{q, d}; }
};

struct Layer {
  float *attn_norm = nullptr, *bq = nullptr, *bk = nullptr, *bv = nullptr, *ffn_norm = nullptr;
  float *q_norm = nullptr, *k_norm = nullptr;  // Qwen3 per-head QK-norm weights (head_dim each)
  Tensor wq, wk, wv, wo, wg, wu, wd;
};

}  // namespace

struct c2h_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  bool has_model = false;
  c2h_model_desc desc{};
  std::string err;
  std::vector<void*> allocs;

  std::vector<Layer> layers;
  Tensor embd, output;
  float* output_norm = nullptr;

  float *X = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr, *h = nullptr;
  uint64_t* attn_tag = nullptr;  // the attention output as {value, tag} words (k_attn_oproj)
  uint64_t* qkv_tag = nullptr;   // q|k|v as {value, tag} words (k_attn_block)
  uint64_t* h_tag = nullptr;     // the SwiGLU output as {value, tag} words (k_ffn_block)
  float* dterm = nullptr;        // k_ffn_block's down terms [FOLD_NB][n_embd], added to X by the next k_attn_block
  bool fuse_oproj = true;        // attention and o-projection in one launch where an instance exists
  bool fuse_qkv = true;          // and qkv with them (layers past 0)
  bool fuse_ffn = true;          // ffn_in and ffn_out in one launch where an instance exists
  bool h128_staged = false;      // head_dim 128: k_attn_h128<H128_VCH> (V through LDS) fits beside the scores
  float* normx[2] = {nullptr, nullptr};
  int nx_cur = 0, nx_prev = 0;
  float* kv = nullptr;
  int32_t* token_ids = nullptr;
  float *rope_cos = nullptr, *rope_sin = nullptr;
  std::vector<float> rope_cos_h, rope_sin_h;  // head_dim 64: host copies for the state's RoPE row
  float* part_v = nullptr;
  int* part_i = nullptr;
  int n_part = 0;
  float* logits = nullptr;
  C2hState* state_dev = nullptr;
  C2hState* state_ring = nullptr;  // pinned
  int32_t* tok_host = nullptr;     // pinned: {token, seq} written by a step's layer 0; [2] the wait flag
  unsigned step_seq = 0;           // last step number handed to the device
  // the state a completed step graph leaves on the device (its final norm
  // advances pos, seq and the normX buffers); valid until the next push
  C2hState state_pred{};
  bool state_pred_valid = false;
  unsigned ring_next = 0;

  // graphs by attention form (attn_form): k_attn_core's tiers of 32, 64,
  // 96, 128 and 256 positions, its any tier up to att_split positions, the
  // long-context kernels beyond
  hipGraphExec_t g_step[7] = {}, g_fwd[7] = {};
  bool graphs_ready = false;
  bool use_graphs = true;
  size_t attn_lds = 0;
  int att_split = 0;     // positions attended up to which k_attn_core runs
  int pfa_max_pos = 0;   // prefill passes ending at or below this many positions run k_pf_attn
  bool long_attn = false;
  float* att_sc = nullptr;  // [PF_ATT_SUB][n_heads][sc_ld] scores / probabilities
  float* att_bmax = nullptr;
  int att_sc_ld = 0, att_n_blk = 0;
  int32_t seq_len = 0;   // KVCache.SeqLen (engine/kvcache.go:25-47)

  // batched prefill buffers (allocated by the first c2h_prefill)
  struct {
    bool ready = false;
    float *X = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr;
    float *g = nullptr, *u = nullptr, *h = nullptr;
    float* xn = nullptr;  // normalised rows as f32 (Q5_0 / Q8_0 projections)
    int8_t* q8 = nullptr;
    float* q8d = nullptr;
    float* q8dT = nullptr;  // the Q8_K scales block-major [nbs][PF_MAX]
    int8_t* q8T = nullptr;  // the Q8_K quants chunk-major [nbs * 8][PF_MAX][32]
    int32_t* q8bs = nullptr;
    int32_t* tok = nullptr;
    int nbs = 0;
  } pf;

  // restricted-logits staging (c2h_logits_ids): ids in, compact logits out
  int32_t* ids_dev = nullptr;
  float* ids_y = nullptr;
  int ids_cap = 0;
  bool dot_attr = false;  // k_dot_rows LDS limit raised
  uint8_t* vq8k = nullptr;  // Q8_K row of normX for a K-quant output.weight
  uint8_t* noalloc = nullptr;  // this device's copy of `scratch` (c2h_quantize_q8k_noalloc)
};

// Device scratch of c2h_quantize_q8k_noalloc, which calls no allocator:
// the staged f32 row (C2H_NOALLOC_MAX_COLS floats) followed by the Q8_K
// blocks the kernel writes (C2H_NOALLOC_MAX_COLS/256 blocks of 292 bytes).
// Every GPU holds its own copy until the process ends.  In host code the
// name is a host-side stand-in, never a device address: host code uses
// only the address hipGetSymbolAddress returned for the device (ctx->noalloc).
constexpr size_t kNoAllocX = (size_t)C2H_NOALLOC_MAX_COLS * 4;
constexpr size_t kNoAllocY = (size_t)(C2H_NOALLOC_MAX_COLS / 256) * 292;
static __device__ __align__(256) uint8_t scratch[kNoAllocX + kNoAllocY];

namespace {

int fail(c2h_ctx* c, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  if (c) c->err = buf;
  return code;
}

#define HIPCHK(c, call)                                                                                 \
  do {                                                                                                  \
    hipError_t e_ = (call);                                                                             \
    if (e_ != hipSuccess) return fail((c), C2H_ERR_HIP, "%s failed: %s", #call, hipGetErrorString(e_)); \
  } while (0)

// Host<->device copies go on the context stream and complete before
// returning: a plain hipMemcpy runs on the null stream, which the
// (non-blocking) context stream does not wait for, and from pageable memory
// it may return before its DMA lands -- a kernel launched next on the
// context stream could read the old bytes.
inline hipError_t stream_copy(hipStream_t st, void* dst, const void* src, size_t bytes, hipMemcpyKind kind) {
  hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, st);
  if (e != hipSuccess) return e;
  return hipStreamSynchronize(st);
}

template <class T>
int dalloc(c2h_ctx* c, T** p, size_t bytes) {
  void* ptr = nullptr;
  HIPCHK(c, hipMalloc(&ptr, bytes < 256 ? 256 : bytes));
  c->allocs.push_back(ptr);
  *p = reinterpret_cast<T*>(ptr);
  return C2H_OK;
}

// Frees one allocation dalloc made (and forgets it).
void dfree(c2h_ctx* c, void* p) {
  auto it = std::find(c->allocs.begin(), c->allocs.end(), p);
  if (it != c->allocs.end()) c->allocs.erase(it);
  (void)hipFree(p);
}

int nb_k(int64_t cols) { return (int)(cols / 256); }
int nb8_of(int64_t cols) { return (int)(cols / 32); }
int nq_of(int64_t cols) { return (nb8_of(cols) + 3) / 4; }

size_t native_row_bytes(int type, int64_t cols) {
  switch (type) {
    case C2H_Q4_K: return (size_t)nb_k(cols) * BS_Q4K;
    case C2H_Q6_K: return (size_t)nb_k(cols) * BS_Q6K;
    case C2H_Q8_0: return (size_t)nb8_of(cols) * BS_Q8_0;
    case C2H_Q5_0: return (size_t)nb8_of(cols) * BS_Q5_0;
    case C2H_F32: return (size_t)cols * 4;
  }
  return 0;
}

// Sizes of the q and d parts of the device layout.
void packed_parts(int type, int64_t rows, int64_t cols, size_t* qb, size_t* db) {
  *qb = *db = 0;
  switch (type) {
    case C2H_Q4_K: *qb = (size_t)rows * nb_k(cols) * BS_Q4K; break;
    case C2H_Q6_K:
      *qb = (size_t)rows * nb_k(cols) * BS_Q6K_PACKED;
      *db = (size_t)rows * nb_k(cols) * 2;
      break;
    case C2H_Q8_0: *qb = (size_t)rows * q8_0_row_stride(nb8_of(cols)); break;
    case C2H_Q5_0: *qb = (size_t)rows * nb8_of(cols) * 24; break;
  }
}

void pack_host(int type, int64_t rows, int64_t cols, const uint8_t* src, uint8_t* qdst, uint8_t* ddst) {
  if (type == C2H_Q4_K) {
    memcpy(qdst, src, (size_t)rows * nb_k(cols) * BS_Q4K);
  } else if (type == C2H_Q6_K) {
    size_t n = (size_t)rows * nb_k(cols);
    for (size_t i = 0; i < n; ++i) {
      memcpy(qdst + i * BS_Q6K_PACKED, src + i * BS_Q6K, BS_Q6K_PACKED);
      memcpy(ddst + i * 2, src + i * BS_Q6K + 208, 2);
    }
  } else if (type == C2H_Q8_0) {
    // per row: fp16 scales padded to dpad halves, then the lane-interleaved quants
    (void)ddst;
    const int nb8 = nb8_of(cols);
    const size_t stride = q8_0_row_stride(nb8), dbytes = (size_t)q8_0_dpad(nb8) * 2;
    memset(qdst, 0, (size_t)rows * stride);
    for (int64_t r = 0; r < rows; ++r) {
      const uint8_t* row = src + (size_t)r * nb8 * BS_Q8_0;
      uint8_t* dr = qdst + (size_t)r * stride;
      uint8_t* qr = dr + dbytes;
      for (int b = 0; b < nb8; ++b) {
        const uint8_t* blk = row + (size_t)b * BS_Q8_0;
        memcpy(dr + (size_t)b * 2, blk, 2);
        int bq = b >> 2, bb = b & 3;
        for (int j = 0; j < 8; ++j)
          for (int i = 0; i < 4; ++i) qr[(bq * 8 + j) * 16 + bb * 4 + i] = blk[2 + j + 8 * i];
      }
    }
  } else if (type == C2H_Q5_0) {
    // per row: the 16 quant bytes of every block, then (qh u32, d u16, 0 u16) per block
    (void)ddst;
    const int nb8 = nb8_of(cols);
    for (int64_t r = 0; r < rows; ++r) {
      const uint8_t* row = src + (size_t)r * nb8 * BS_Q5_0;
      uint8_t* qr = qdst + (size_t)r * nb8 * 24;
      uint8_t* hr = qr + (size_t)nb8 * 16;
      for (int b = 0; b < nb8; ++b) {
        const uint8_t* blk = row + (size_t)b * BS_Q5_0;
        memcpy(qr + (size_t)b * 16, blk + 6, 16);
        memcpy(hr + (size_t)b * 8, blk + 2, 4);
        memcpy(hr + (size_t)b * 8 + 4, blk, 2);
        hr[b * 8 + 6] = hr[b * 8 + 7] = 0;
      }
    }
  }
}

int check_type_shape(c2h_ctx* c, int type, int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return fail(c, C2H_ERR_INVALID, "rows/cols must be positive");
  if (type == C2H_Q4_K || type == C2H_Q6_K) {
    if (cols < 256) return fail(c, C2H_ERR_UNSUPPORTED, "K-quant rows need at least 256 columns");
    if (nb_k(cols) > LDS_Q8K_BLOCKS) return fail(c, C2H_ERR_UNSUPPORTED, "more than 16384 columns");
    return C2H_OK;
  }
  if (type == C2H_Q8_0 || type == C2H_Q5_0) {
    if (cols < 32) return fail(c, C2H_ERR_UNSUPPORTED, "Q8_0/Q5_0 rows need at least 32 columns");
    return C2H_OK;
  }
  return fail(c, C2H_ERR_UNSUPPORTED, "ggml type %d is not run by this build", type);
}

int upload_quant(c2h_ctx* c, Tensor* t, int type, int64_t rows, int64_t cols, const void* host, size_t bytes) {
  int rc = check_type_shape(c, type, rows, cols);
  if (rc) return rc;
  size_t need = (size_t)rows * native_row_bytes(type, cols);
  if (bytes < need) return fail(c, C2H_ERR_INVALID, "tensor payload %zu bytes < %zu needed", bytes, need);
  size_t qb, db;
  packed_parts(type, rows, cols, &qb, &db);
  std::vector<uint8_t> qh(qb), dh(db);
  pack_host(type, rows, cols, reinterpret_cast<const uint8_t*>(host), qh.data(), dh.data());
  uint8_t* q;
  if ((rc = dalloc(c, &q, qb))) return rc;
  HIPCHK(c, stream_copy(c->stream, q, qh.data(), qb, hipMemcpyHostToDevice));
  uint16_t* d = nullptr;
  if (db) {
    if ((rc = dalloc(c, &d, db))) return rc;
    HIPCHK(c, stream_copy(c->stream, d, dh.data(), db, hipMemcpyHostToDevice));
  }
  if (t->pf6) {  // the split prefill copy of the previous contents
    HIPCHK(c, hipStreamSynchronize(c->stream));
    dfree(c, t->pf6);
    t->pf6 = nullptr;
  }
  t->q = q;
  t->d = d;
  t->type = type;
  t->rows = rows;
  t->cols = cols;
  c->graphs_ready = false;
  return C2H_OK;
}

int upload_f32(c2h_ctx* c, float** dst, int64_t n_expected, int type, int64_t rows, int64_t cols, const void* host,
               size_t bytes) {
  if (type != C2H_F32) return fail(c, C2H_ERR_UNSUPPORTED, "norm/bias tensors must be F32");
  if (rows * cols != n_expected || bytes < (size_t)n_expected * 4)
    return fail(c, C2H_ERR_INVALID, "F32 tensor has %lld elements, expected %lld", (long long)(rows * cols),
                (long long)n_expected);
  int rc;
  if (!*dst && (rc = dalloc(c, dst, (size_t)n_expected * 4))) return rc;
  HIPCHK(c, stream_copy(c->stream, *dst, host, (size_t)n_expected * 4, hipMemcpyHostToDevice));
  c->graphs_ready = false;
  return C2H_OK;
}

// ------------------------------------------------------------- launches

// k_gemv_q8k: the external Q8_K row plus 256 term and 256 scale slots.
size_t gemv_q8k_lds_bytes() { return sizeof(Q8KLds) + (size_t)512 * sizeof(float); }

void add_job(GemvParams& P, const Tensor& w, const Tensor* w2, int mode, float* y, const float* bias,
             int32_t* isums) {
  GemvJob& J = P.jobs[P.n_jobs++];
  J.w = w.ref();
  J.type = w.type;
  if (w2) {
    J.w2 = w2->ref();
    J.type2 = w2->type;
  } else {
    J.w2 = WeightRef{nullptr, nullptr};
    J.type2 = w.type;
  }
  J.rows = (int)w.rows;
  if (w.type == C2H_Q5_0 || w.type == C2H_Q8_0) {  // k_gemv_f: 32-element blocks
    J.nb = nb8_of(w.cols);
    J.rpw = (w.type == C2H_Q5_0) ? std::max(1, 256 / J.nb) : 32;
  } else {
    J.nb = nb_k(w.cols);
    J.rpw = 256 / (4 * J.nb);
  }
  J.n_wg = (J.rows + J.rpw - 1) / J.rpw;
  J.mode = mode;
  J.y = y;
  J.bias = bias;
  J.isums = isums;
}

// Grid of a GEMV launch: one row per job, as wide as its widest job.
dim3 job_grid(const GemvParams& P) {
  int w = 1;
  for (int j = 0; j < P.n_jobs; ++j) w = std::max(w, P.jobs[j].n_wg);
  return dim3(w, P.n_jobs);
}

typedef void (*GemvKernel)(const float*, int, GemvParams);  // k_gemv_row
typedef void (*GemvFKernel)(GemvParams);                     // k_gemv_f

// Row-kernel instance for (super-blocks per row, prologue, mode); nullptr
// when this build has none for that width.
GemvKernel gemv_row_kernel(int nb, int pro, int mode) {
  if (pro == PRO_QUANT && mode == MODE_RESID) {
    switch (nb) {
      case 3: return k_gemv_row<3, PRO_QUANT, MODE_RESID>;
      case 4: return k_gemv_row<4, PRO_QUANT, MODE_RESID>;
      case 12: return k_gemv_row<12, PRO_QUANT, MODE_RESID>;
      case 19: return k_gemv_row<19, PRO_QUANT, MODE_RESID>;
      case 8: return k_gemv_row<8, PRO_QUANT, MODE_RESID>;
      case 24: return k_gemv_row<24, PRO_QUANT, MODE_RESID>;
      case 6: return k_gemv_row<6, PRO_QUANT, MODE_RESID>;
      case 35: return k_gemv_row<35, PRO_QUANT, MODE_RESID>;
      case 43: return k_gemv_row<43, PRO_QUANT, MODE_RESID>;
      default: return nullptr;
    }
  }
  if (pro == PRO_NORM && mode == MODE_SWIGLU) {
    switch (nb) {
      case 3: return k_gemv_row<3, PRO_NORM, MODE_SWIGLU>;
      case 4: return k_gemv_row<4, PRO_NORM, MODE_SWIGLU>;
      case 8: return k_gemv_row<8, PRO_NORM, MODE_SWIGLU>;
      case 6: return k_gemv_row<6, PRO_NORM, MODE_SWIGLU>;
      default: return nullptr;
    }
  }
  if (mode == MODE_BIAS && nb == 3) {
    if (pro == PRO_NORM) return k_gemv_row<3, PRO_NORM, MODE_BIAS>;
    if (pro == PRO_EMBED_NORM) return k_gemv_row<3, PRO_EMBED_NORM, MODE_BIAS>;
    if (pro == PRO_ARGMAX_EMBED_NORM) return k_gemv_row<3, PRO_ARGMAX_EMBED_NORM, MODE_BIAS>;
  }
  if (mode == MODE_BIAS && nb == 4) {
    if (pro == PRO_NORM) return k_gemv_row<4, PRO_NORM, MODE_BIAS>;
    if (pro == PRO_EMBED_NORM) return k_gemv_row<4, PRO_EMBED_NORM, MODE_BIAS>;
    if (pro == PRO_ARGMAX_EMBED_NORM) return k_gemv_row<4, PRO_ARGMAX_EMBED_NORM, MODE_BIAS>;
  }
  if (mode == MODE_BIAS && nb == 6) {
    if (pro == PRO_NORM) return k_gemv_row<6, PRO_NORM, MODE_BIAS>;
    if (pro == PRO_EMBED_NORM) return k_gemv_row<6, PRO_EMBED_NORM, MODE_BIAS>;
    if (pro == PRO_ARGMAX_EMBED_NORM) return k_gemv_row<6, PRO_ARGMAX_EMBED_NORM, MODE_BIAS>;
  }
  if (mode == MODE_BIAS && nb == 8) {
    if (pro == PRO_NORM) return k_gemv_row<8, PRO_NORM, MODE_BIAS>;
    if (pro == PRO_EMBED_NORM) return k_gemv_row<8, PRO_EMBED_NORM, MODE_BIAS>;
    if (pro == PRO_ARGMAX_EMBED_NORM) return k_gemv_row<8, PRO_ARGMAX_EMBED_NORM, MODE_BIAS>;
  }
  return nullptr;
}

bool float_input(int type) { return type == C2H_Q5_0 || type == C2H_Q8_0; }

// k_gemv_f instance for (prologue, mode); nullptr when none is built.
GemvFKernel gemv_f_kernel(int pro, int mode) {
  if (mode == MODE_BIAS) {
    if (pro == PRO_NORM) return k_gemv_f<PRO_NORM, MODE_BIAS>;
    if (pro == PRO_EMBED_NORM) return k_gemv_f<PRO_EMBED_NORM, MODE_BIAS>;
    if (pro == PRO_ARGMAX_EMBED_NORM) return k_gemv_f<PRO_ARGMAX_EMBED_NORM, MODE_BIAS>;
  }
  if (pro == PRO_NORM && mode == MODE_SWIGLU) return k_gemv_f<PRO_NORM, MODE_SWIGLU>;
  if (pro == PRO_QUANT && mode == MODE_RESID) return k_gemv_f<PRO_QUANT, MODE_RESID>;
  if (pro == PRO_QUANT && mode == MODE_STORE) return k_gemv_f<PRO_QUANT, MODE_STORE>;
  return nullptr;
}

// A float-input launch over all its jobs (P.n_x = the input length).
void launch_gemv_f(c2h_ctx* c, GemvParams& P) {
  GemvFKernel k = gemv_f_kernel(P.prologue, P.jobs[0].mode);
  const size_t lds = (size_t)gemv_f_lds_floats(P.n_x) * sizeof(float);
  hipLaunchKernelGGL(k, job_grid(P), dim3(256), lds, c->stream, P);
}

// rows per workgroup and workgroups of each job of a k_gemv_row launch
void prep_gemv_row(GemvParams& P) {
  const int ni = row_item_threads(P.jobs[0].nb, P.prologue, P.jobs[0].mode);
  for (int j = 0; j < P.n_jobs; ++j) {
    GemvJob& J = P.jobs[j];
    J.rpw = ni / (4 * J.nb);
    J.n_wg = (J.rows + J.rpw - 1) / J.rpw;
  }
}

// A row-kernel launch over all its jobs (same width and mode); the norm
// prologues need the x*x chain buffer.
void launch_gemv_row(c2h_ctx* c, GemvParams& P) {
  const int nt = row_threads(P.jobs[0].nb, P.prologue, P.jobs[0].mode);
  prep_gemv_row(P);
  const GemvJob& J = P.jobs[0];
  GemvKernel k = gemv_row_kernel(J.nb, P.prologue, J.mode);
  size_t lds = (P.prologue != PRO_QUANT) ? (size_t)P.n_x_lds * sizeof(float) : 0;
  hipLaunchKernelGGL(k, job_grid(P), dim3(nt), lds, c->stream, P.x, P.n_x, P);
}

GemvParams base_params(c2h_ctx* c) {
  GemvParams P;
  memset(&P, 0, sizeof(P));
  P.eps = c->desc.rms_eps;
  P.emb = c->embd.ref();
  P.n_vocab = c->desc.n_vocab;
  P.part_v = c->part_v;
  P.part_i = c->part_i;
  P.n_part = c->n_part;
  P.token_ids = c->token_ids;
  P.max_ctx = c->desc.max_ctx;
  P.state = c->state_dev;
  return P;
}

const Tensor& out_weight(c2h_ctx* c) { return c->output.present() ? c->output : c->embd; }

typedef void (*VocabKernel)(const uint8_t*, C2hState*, const float*, const float*, int, VocabParams);

// The vocab kernel instance for rows of nb8 Q8_0 blocks (nullptr outside
// the instantiated widths) and its dynamic LDS (x permuted).
VocabKernel vocab_kernel(int nb8) {
  switch (nb8) {
    case 24: return k_vocab<24>;
    case 25: return k_vocab<25>;
    case 26: return k_vocab<26>;
    case 27: return k_vocab<27>;
    case 28: return k_vocab<28>;
    case 29: return k_vocab<29>;
    case 30: return k_vocab<30>;
    case 31: return k_vocab<31>;
    case 32: return k_vocab<32>;
    case 48: return k_vocab<48>;
    case 64: return k_vocab<64>;
    default: return nullptr;
  }
}
size_t vocab_lds(int64_t cols) { return (size_t)nq_of((int)cols) * 4 * 32 * sizeof(float); }

// Grid of the vocab kernel for a rows x cols Q8_0 matrix: up to two
// workgroups per CU (fewer if the occupancy is lower), at most one per
// 32-row tile, then trimmed so every workgroup walks the same number of
// tiles (151,936 x 896: 475 workgroups of 10 tiles rather than 512 of 9 or
// 10).  Measured over 1..18 per CU and 6..12 tiles per workgroup: two per
// CU keeps the most of the matrix streaming under the arithmetic, and equal
// walks remove a last round in which most of the GPU waits.
int vocab_grid(c2h_ctx* c, int64_t rows, int64_t cols, int* grid) {
  VocabKernel k = vocab_kernel(nb8_of(cols));
  if (!k)
    return fail(c, C2H_ERR_UNSUPPORTED, "Q8_0 vocab rows of %lld columns (this build: %d..%d, 1536 and 2048)",
                (long long)cols, 32 * VOCAB_MIN_NB8, 32 * VOCAB_MAX_NB8);
  int per_cu = 0, n_cu = 0;
  HIPCHK(c, hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, 256, vocab_lds(cols)));
  HIPCHK(c, hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, c->device));
  const int64_t tiles = (rows + 31) / 32;
  const int64_t g0 = std::max<int64_t>(1, std::min<int64_t>(tiles, (int64_t)std::min(std::max(per_cu, 1), 2) * std::max(n_cu, 1)));
  // as few workgroups as give every one the same number of tiles (up to one
  // less for the last): no final round with most of the GPU idle
  int64_t per_wg = (tiles + g0 - 1) / g0;
  // C2H_VOCAB_TILES_PER_WG overrides the tiles per workgroup (measurement aid)
  if (const char* e = getenv("C2H_VOCAB_TILES_PER_WG")) per_wg = std::max(1, atoi(e));
  *grid = (int)((tiles + per_wg - 1) / per_wg);
  return C2H_OK;
}

XSel plain_x(const float* x) {
  XSel X;
  memset(&X, 0, sizeof(X));
  X.x = x;
  return X;
}

void launch_dot_rows(c2h_ctx* c, int type, WeightRef w, int rows, int cols, XSel X, const int32_t* ids, int n,
                     int scatter, float* y);
int dot_rows_ready(c2h_ctx* c, int64_t cols);

// The vocab projection of the step: the fused Q8_0 kernel (logits, penalty
// and argmax candidates in one pass), or for the other output formats the
// pooled DispatchGEMV (engine/pool.go:122-154: Q4_K / Q6_K on the Q8_K row
// of normX, Q5_0 on f32 normX) into logits_out (else the context's logits
// buffer), then k_logits_pick for the penalty and the candidates.
void enqueue_vocab(c2h_ctx* c, int apply_penalty, float* logits_out, int x_sel, const float* x,
                   const uint8_t* q8_rows = nullptr) {
  const Tensor& ow = out_weight(c);
  if (ow.type != C2H_Q8_0) {
    XSel X;
    memset(&X, 0, sizeof(X));
    X.x = x;
    X.buf[0] = c->normx[0];
    X.buf[1] = c->normx[1];
    X.state = c->state_dev;
    X.sel = x_sel;
    float* y = logits_out ? logits_out : c->logits;
    if (ow.type == C2H_Q5_0) {
      launch_dot_rows(c, ow.type, ow.ref(), (int)ow.rows, (int)ow.cols, X, nullptr, (int)ow.rows, 0, y);
    } else {
      const int nb = nb_k(ow.cols);
      hipLaunchKernelGGL(k_quantize_q8k_sel, dim3((nb + 3) / 4), dim3(256), 0, c->stream, X, nb, c->vq8k);
      GemvParams P;
      memset(&P, 0, sizeof(P));
      P.prologue = PRO_Q8K;
      P.q8k_in = c->vq8k;
      P.nb_in = nb;
      add_job(P, ow, nullptr, MODE_STORE, y, nullptr, nullptr);
      hipLaunchKernelGGL(k_gemv_q8k, job_grid(P), dim3(256), gemv_q8k_lds_bytes(), c->stream, P);
    }
    if (apply_penalty || !logits_out) {
      PickParams K;
      memset(&K, 0, sizeof(K));
      K.logits = y;
      K.n_vocab = c->desc.n_vocab;
      K.token_ids = c->token_ids;
      K.apply_penalty = apply_penalty;
      K.state = c->state_dev;
      K.part_v = c->part_v;
      K.part_i = c->part_i;
      hipLaunchKernelGGL(k_logits_pick, dim3(c->n_part), dim3(256), 0, c->stream, K);
    }
    return;
  }
  VocabParams V;
  memset(&V, 0, sizeof(V));
  V.w = out_weight(c).ref();
  if (q8_rows) V.w.q = q8_rows;  // a copy of the packed Q8_0 matrix (measurement)
  V.n_vocab = c->desc.n_vocab;
  V.n_embd = c->desc.n_embd;
  V.x_sel = x_sel;
  V.x = x;
  V.x_buf[0] = c->normx[0];
  V.x_buf[1] = c->normx[1];
  V.token_ids = c->token_ids;
  V.apply_penalty = apply_penalty;
  V.logits_out = logits_out;
  V.part_v = c->part_v;
  V.part_i = c->part_i;
  V.state = c->state_dev;
  hipLaunchKernelGGL(vocab_kernel(nb8_of(c->desc.n_embd)), dim3(c->n_part), dim3(256), vocab_lds(c->desc.n_embd),
                     c->stream, V.w.q, V.state, x_sel ? V.x_buf[0] : V.x, x_sel ? V.x_buf[1] : V.x, V.n_vocab, V);
}

AttnCoreParams attn_params(c2h_ctx* c, int layer) {
  const c2h_model_desc& D = c->desc;
  AttnCoreParams A;
  memset(&A, 0, sizeof(A));
  A.kv = c->kv;
  A.rope_cos = c->rope_cos;
  A.rope_sin = c->rope_sin;
  A.rope_len = D.max_ctx;
  A.layer = layer;
  A.n_layers = D.n_layers;
  A.n_heads = D.n_heads;
  A.n_kv_heads = D.n_kv_heads;
  A.max_ctx = D.max_ctx;
  A.scale = (float)(1.0 / std::sqrt((double)D.head_dim));
  A.eps = D.rms_eps;
  A.q_norm = c->layers[layer].q_norm;
  A.k_norm = c->layers[layer].k_norm;
  A.state = c->state_dev;
  A.sc = c->att_sc;
  A.bmax = c->att_bmax;
  A.sc_ld = c->att_sc_ld;
  A.n_blk = c->att_n_blk;
  return A;
}

// Long-context attention of `ntok` query tokens (rows tok0..): scores over
// every block of the context, softmax, AV.  Blocks past a token's context
// return at once, so the grid covers max_ctx and graphs replay at any pos.
void enqueue_attn_long(c2h_ctx* c, const AttnCoreParams& A, int ntok) {
  const c2h_model_desc& D = c->desc;
  hipLaunchKernelGGL(k_attn_scores, dim3(c->att_n_blk, D.n_kv_heads, ntok), dim3(256), 0, c->stream, A);
  hipLaunchKernelGGL(k_attn_softmax, dim3(D.n_heads, ntok), dim3(1024),
                     (size_t)attn_softmax_lds_floats(D.max_ctx) * 4, c->stream, A);
  hipLaunchKernelGGL(k_attn_av, dim3(D.n_kv_heads * ATT_AV_SLICES, ntok), dim3(ATT_AV_THREADS),
                     (size_t)ATT_AV_LDS_FLOATS * 4, c->stream,
                     A);
}

// Attention forms of a decode step by the positions T it attends to:
// k_attn_core sized for T <= 32, 64, 96, 128, 256 (the tiers), for
// T <= att_split, and the long-context kernels past the split.
enum : int {
  ATT_FORM_32 = 0, ATT_FORM_64, ATT_FORM_96, ATT_FORM_128, ATT_FORM_256, ATT_FORM_CORE, ATT_FORM_LONG, ATT_FORMS
};
constexpr int kFormTier[ATT_FORM_CORE] = {ATT_TIER_32, ATT_TIER_64, ATT_TIER_96, ATT_TIER_128, ATT_TIER_256};
static_assert(sizeof(c2h_ctx::g_step) / sizeof(hipGraphExec_t) == ATT_FORMS, "one graph per attention form");

int attn_form(const c2h_ctx* c, int T) {
  if (c->desc.head_dim == 128) return ATT_FORM_32;  // k_attn_h128 serves every T
  if (c->long_attn && T > c->att_split) return ATT_FORM_LONG;
  for (int f = 0; f < ATT_FORM_CORE; ++f)
    if (T <= kFormTier[f]) return f;
  return ATT_FORM_CORE;
}

// Whether some decode position of this context runs the form.
bool form_used(const c2h_ctx* c, int form) {
  if (c->desc.head_dim == 128) return form == ATT_FORM_32;
  const int tmax = c->long_attn ? c->att_split : c->desc.max_ctx;  // largest T of the core forms
  if (form == ATT_FORM_LONG) return c->long_attn;
  return form == 0 || tmax > kFormTier[form - 1];
}

// The k_attn_core instance of a core form.
decltype(&k_attn_core<ATT_TIER_ANY>) attn_core_kernel(int form) {
  switch (form) {
    case ATT_FORM_32: return k_attn_core<ATT_TIER_32>;
    case ATT_FORM_64: return k_attn_core<ATT_TIER_64>;
    case ATT_FORM_96: return k_attn_core<ATT_TIER_96>;
    case ATT_FORM_128: return k_attn_core<ATT_TIER_128>;
    case ATT_FORM_256: return k_attn_core<ATT_TIER_256>;
    default: return k_attn_core<ATT_TIER_ANY>;
  }
}

// One projection of a layer (w2: the paired up matrix of SwiGLU).
struct ProjJob {
  const Tensor* w;
  const Tensor* w2;
  float* y;
  const float* bias;
};

// The matrices of one projection group launched by input kind: Q4_K/Q6_K
// read the Q8_K row of x (k_gemv_row), Q5_0/Q8_0 read x as f32 (k_gemv_f),
// as engine/model.go:250-270 dispatches.  The first launch carries the
// group's prologue; for layer 0's embed/argmax prologues a second launch
// normalises the X the first one published.  x: the input (X for the norm
// prologues), n_x its length.
void launch_group(c2h_ctx* c, std::initializer_list<ProjJob> jobs, int pro, int mode, const float* x, int n_x,
                  const float* norm_w) {
  bool first = true;
  for (int kind = 0; kind < 2; ++kind) {
    GemvParams P = base_params(c);
    for (const ProjJob& j : jobs)
      if (float_input(j.w->type) == (kind == 1)) add_job(P, *j.w, j.w2, mode, j.y, j.bias, nullptr);
    if (P.n_jobs == 0) continue;
    P.prologue = (!first && (pro == PRO_EMBED_NORM || pro == PRO_ARGMAX_EMBED_NORM)) ? PRO_NORM : pro;
    if (P.prologue == PRO_ARGMAX_EMBED_NORM) P.tok_out = c->tok_host;
    P.x = x;
    P.x_out = c->X;
    P.n_x = n_x;
    P.n_x_lds = chain_lds_floats(n_x);
    P.norm_w = norm_w;
    P.nb_in = kind == 0 ? nb_k(n_x) : nb8_of(n_x);
    if (kind == 0)
      launch_gemv_row(c, P);
    else
      launch_gemv_f(c, P);
    first = false;
  }
}

// The launches of one decoder layer (engine/forward.go:65-131), each on its
// own so the measurement entry points can time them one by one.
// q|k|v = W * x(RMSNorm(X)) + bias; layer 0 embeds the token first (pro).
// pend (layers past 0 with K-quant q/k/v of 3 super-blocks): the previous
// layer's FFN launch left its terms for X (dterm), added by k_gemv_row_pend.
void enqueue_qkv(c2h_ctx* c, int l, int pro, bool pend = false) {
  Layer& L = c->layers[l];
  if (!pend) {
    launch_group(c, {{&L.wq, nullptr, c->q, L.bq}, {&L.wk, nullptr, c->k, L.bk}, {&L.wv, nullptr, c->v, L.bv}}, pro,
                 MODE_BIAS, c->X, c->desc.n_embd, L.attn_norm);
    return;
  }
  const int E = c->desc.n_embd;
  GemvParams P = base_params(c);
  add_job(P, L.wq, nullptr, MODE_BIAS, c->q, L.bq, nullptr);
  add_job(P, L.wk, nullptr, MODE_BIAS, c->k, L.bk, nullptr);
  add_job(P, L.wv, nullptr, MODE_BIAS, c->v, L.bv, nullptr);
  P.prologue = PRO_NORM;
  P.x = c->X;
  P.x_out = c->X;
  P.n_x = E;
  P.n_x_lds = chain_lds_floats(E);
  P.norm_w = L.attn_norm;
  P.nb_in = nb_k(E);
  P.x_pend = c->dterm;
  P.pend_n = E;
  prep_gemv_row(P);
  hipLaunchKernelGGL((k_gemv_row_pend<3, PRO_NORM, MODE_BIAS>), job_grid(P), dim3(row_threads(3, PRO_NORM, MODE_BIAS)),
                     (size_t)P.n_x_lds * sizeof(float), c->stream, P.x, P.n_x, P);
}

// attention: RoPE, KV store, scores, softmax, AV
void enqueue_attn(c2h_ctx* c, int l, int form) {
  const c2h_model_desc& D = c->desc;
  AttnCoreParams A = attn_params(c, l);
  A.q = c->q;
  A.k = c->k;
  A.v = c->v;
  A.out = c->attn;
  A.store_kv = 1;
  const dim3 grid(D.n_heads / D.n_kv_heads, D.n_kv_heads);
  if (D.head_dim == 128) {
    A.sc_ld = attn_h128_lds_floats(D.max_ctx);  // the V chunks follow the scores
    hipLaunchKernelGGL(c->h128_staged ? k_attn_h128<H128_VCH> : k_attn_h128<0>, grid, dim3(256), c->attn_lds,
                       c->stream, A);
  }
  else if (form == ATT_FORM_LONG)
    enqueue_attn_long(c, A, 1);
  else {
    A.xcd_map = D.n_kv_heads <= ATT_XCDS ? 1 : 0;
    const dim3 xgrid(ATT_XCDS * (D.n_heads / D.n_kv_heads));
    hipLaunchKernelGGL(attn_core_kernel(form), A.xcd_map ? xgrid : grid, dim3(256), c->attn_lds, c->stream, A.state,
                       A.kv, A.q, A.k, A.v, attn_dims(A, D.n_heads / D.n_kv_heads), A.max_ctx, A);
  }
}

// The k_attn_block instance of a core form.
decltype(&k_attn_block<ATT_TIER_32, 3>) attn_block_kernel(int form) {
  switch (form) {
    case ATT_FORM_32: return k_attn_block<ATT_TIER_32, 3>;
    case ATT_FORM_64: return k_attn_block<ATT_TIER_64, 3>;
    case ATT_FORM_96: return k_attn_block<ATT_TIER_96, 3>;
    case ATT_FORM_128: return k_attn_block<ATT_TIER_128, 3>;
    case ATT_FORM_256: return k_attn_block<ATT_TIER_256, 3>;
    default: return k_attn_block<ATT_TIER_ANY, 3>;
  }
}

// The k_attn_block_f instance of a core form.
decltype(&k_attn_block_f<ATT_TIER_32>) attn_block_f_kernel(int form) {
  switch (form) {
    case ATT_FORM_32: return k_attn_block_f<ATT_TIER_32>;
    case ATT_FORM_64: return k_attn_block_f<ATT_TIER_64>;
    case ATT_FORM_96: return k_attn_block_f<ATT_TIER_96>;
    case ATT_FORM_128: return k_attn_block_f<ATT_TIER_128>;
    case ATT_FORM_256: return k_attn_block_f<ATT_TIER_256>;
    default: return k_attn_block_f<ATT_TIER_ANY>;
  }
}

// The k_attn_oproj instance of a core form.
decltype(&k_attn_oproj<ATT_TIER_ANY, 3>) attn_oproj_kernel(int form) {
  switch (form) {
    case ATT_FORM_32: return k_attn_oproj<ATT_TIER_32, 3>;
    case ATT_FORM_64: return k_attn_oproj<ATT_TIER_64, 3>;
    case ATT_FORM_96: return k_attn_oproj<ATT_TIER_96, 3>;
    case ATT_FORM_128: return k_attn_oproj<ATT_TIER_128, 3>;
    case ATT_FORM_256: return k_attn_oproj<ATT_TIER_256, 3>;
    default: return k_attn_oproj<ATT_TIER_ANY, 3>;
  }
}

// Whether layer l's attention and o-projection run as one launch
// (k_attn_oproj): the head_dim 64 decode forms over the XCD-grouped grid,
// and a K-quant o-projection of 3 super-blocks per row (the instances built).
bool fuse_attn_oproj(const c2h_ctx* c, int l, int form) {
  const c2h_model_desc& D = c->desc;
  return c->fuse_oproj && D.head_dim == 64 && form < ATT_FORM_LONG && D.n_kv_heads <= ATT_XCDS &&
         !float_input(c->layers[l].wo.type) && nb_k(D.n_embd) == 3;
}

// Whether layer l runs qkv in that launch too (k_attn_block): past layer 0
// (whose qkv embeds the token), with K-quant q|k|v.
bool fuse_attn_block(const c2h_ctx* c, int l, int form) {
  const Layer& L = c->layers[l];
  return l > 0 && c->fuse_qkv && fuse_attn_oproj(c, l, form) && !float_input(L.wq.type) &&
         !float_input(L.wk.type) && !float_input(L.wv.type);
}

// The attention part of the fused launches: k_attn_core's XCD-grouped grid,
// output also tagged
AttnCoreParams fused_attn_params(c2h_ctx* c, int l) {
  const c2h_model_desc& D = c->desc;
  AttnCoreParams A = attn_params(c, l);
  A.q = c->q;
  A.k = c->k;
  A.v = c->v;
  A.out = c->attn;
  A.store_kv = 1;
  A.xcd_map = 1;
  A.out_tag = c->attn_tag;
  A.n_attn_wg = ATT_XCDS * (D.n_heads / D.n_kv_heads);
  A.wait_err = c->tok_host + 2;
  return A;
}

// The o-projection part: X += Wo * x(attn), x read tagged
GemvParams fused_oproj_params(c2h_ctx* c, int l) {
  const c2h_model_desc& D = c->desc;
  GemvParams P = base_params(c);
  add_job(P, c->layers[l].wo, nullptr, MODE_RESID, c->X, nullptr, nullptr);
  P.prologue = PRO_QUANT;
  P.x = c->attn;
  P.x_out = c->X;
  P.n_x = D.n_embd;
  P.n_x_lds = chain_lds_floats(D.n_embd);
  P.nb_in = nb_k(D.n_embd);
  P.x_tag = c->attn_tag;
  P.wait_err = c->tok_host + 2;
  prep_gemv_row(P);
  return P;
}

// Whether layer l runs qkv, attention and attn_out as one launch of the
// float-input GEMV (k_attn_block_f): past layer 0, the head_dim 64 decode
// forms over the XCD-grouped grid, Q5_0 / Q8_0 q, k, v and o.
bool fuse_attn_block_f(const c2h_ctx* c, int l, int form) {
  const c2h_model_desc& D = c->desc;
  const Layer& L = c->layers[l];
  return l > 0 && c->fuse_qkv && D.head_dim == 64 && form < ATT_FORM_LONG && D.n_kv_heads <= ATT_XCDS &&
         float_input(L.wq.type) && float_input(L.wk.type) && float_input(L.wv.type) && float_input(L.wo.type);
}

// qkv + attention + attn_out in one launch, the GEMV parts k_gemv_f's
// pend: the previous layer's FFN launch left its terms for X (dterm)
void enqueue_attn_block_f(c2h_ctx* c, int l, int form, bool pend) {
  const c2h_model_desc& D = c->desc;
  Layer& L = c->layers[l];
  const int E = D.n_embd, KVd = D.n_kv_heads * D.head_dim;
  GemvParams Q = base_params(c);
  add_job(Q, L.wq, nullptr, MODE_BIAS, c->q, L.bq, nullptr);
  add_job(Q, L.wk, nullptr, MODE_BIAS, c->k, L.bk, nullptr);
  add_job(Q, L.wv, nullptr, MODE_BIAS, c->v, L.bv, nullptr);
  Q.jobs[0].spare = 0;
  Q.jobs[1].spare = E;
  Q.jobs[2].spare = E + KVd;
  Q.prologue = PRO_NORM;
  Q.x = c->X;
  Q.x_out = c->X;
  Q.n_x = E;
  Q.n_x_lds = chain_lds_floats(E);
  Q.norm_w = L.attn_norm;
  Q.nb_in = nb8_of(E);
  Q.y_tag = c->qkv_tag;
  Q.x_pend = pend ? c->dterm : nullptr;
  Q.pend_n = E;
  int w = 1;
  for (int j = 0; j < Q.n_jobs; ++j) w = std::max(w, Q.jobs[j].n_wg);
  const AttnCoreParams A = fused_attn_params(c, l);
  GemvParams P = base_params(c);
  add_job(P, L.wo, nullptr, MODE_RESID, c->X, nullptr, nullptr);
  P.prologue = PRO_QUANT;
  P.x = c->attn;
  P.x_out = c->X;
  P.n_x = E;
  P.n_x_lds = chain_lds_floats(E);
  P.nb_in = nb8_of(E);
  P.x_tag = c->attn_tag;
  P.wait_err = c->tok_host + 2;
  P.x_pend = Q.x_pend;
  P.pend_n = E;
  const size_t lds = std::max(c->attn_lds, (size_t)gemv_f_lds_floats(E) * sizeof(float));
  hipLaunchKernelGGL(attn_block_f_kernel(form), dim3(3 * w + A.n_attn_wg + P.jobs[0].n_wg), dim3(256), lds,
                     c->stream, A.state, A.kv, (const float*)c->X, w << 16, (const uint64_t*)c->qkv_tag,
                     attn_dims(A, D.n_heads / D.n_kv_heads), A.max_ctx, A, Q, P);
}

// attention + attn_out in one launch: the attention workgroups first, then
// the o-projection's, which wait for the tagged output
void enqueue_attn_oproj(c2h_ctx* c, int l, int form) {
  const c2h_model_desc& D = c->desc;
  const AttnCoreParams A = fused_attn_params(c, l);
  const GemvParams P = fused_oproj_params(c, l);
  hipLaunchKernelGGL(attn_oproj_kernel(form), dim3(A.n_attn_wg + P.jobs[0].n_wg), dim3(256), c->attn_lds, c->stream,
                     A.state, A.kv, A.q, A.k, A.v, attn_dims(A, D.n_heads / D.n_kv_heads), A.max_ctx, A, P);
}

// qkv + attention + attn_out in one launch (layers past 0): q|k|v = W *
// x(RMSNorm(X)) + bias on 3 W workgroups (job-major, W the widest job's
// count), stored tagged as well, then the two parts of k_attn_oproj, the
// attention's reading q|k|v tagged
// pend: the previous layer's k_ffn_block left its terms for X (dterm)
void enqueue_attn_block(c2h_ctx* c, int l, int form, bool pend) {
  const c2h_model_desc& D = c->desc;
  Layer& L = c->layers[l];
  const int E = D.n_embd, KVd = D.n_kv_heads * D.head_dim;
  GemvParams Q = base_params(c);
  add_job(Q, L.wq, nullptr, MODE_BIAS, c->q, L.bq, nullptr);
  add_job(Q, L.wk, nullptr, MODE_BIAS, c->k, L.bk, nullptr);
  add_job(Q, L.wv, nullptr, MODE_BIAS, c->v, L.bv, nullptr);
  Q.jobs[0].spare = 0;
  Q.jobs[1].spare = E;
  Q.jobs[2].spare = E + KVd;
  Q.prologue = PRO_NORM;
  Q.x = c->X;
  Q.x_out = c->X;
  Q.n_x = E;
  Q.n_x_lds = chain_lds_floats(E);
  Q.norm_w = L.attn_norm;
  Q.nb_in = nb_k(E);
  Q.y_tag = c->qkv_tag;
  Q.x_pend = pend ? c->dterm : nullptr;
  Q.pend_n = E;
  prep_gemv_row(Q);
  int w = 1;
  for (int j = 0; j < Q.n_jobs; ++j) w = std::max(w, Q.jobs[j].n_wg);
  // the k and v jobs' workgroups (the same rows); the rest of their W exit
  // at entry.  Rows of 3 super-blocks (E < 1024) keep W < 50.
  const int nkv = std::max(Q.jobs[1].n_wg, Q.jobs[2].n_wg);
  const AttnCoreParams A = fused_attn_params(c, l);
  GemvParams P = fused_oproj_params(c, l);
  P.x_pend = Q.x_pend;
  P.pend_n = E;
  const size_t lds = std::max(c->attn_lds, (size_t)Q.n_x_lds * sizeof(float));
  hipLaunchKernelGGL(attn_block_kernel(form), dim3(3 * w + A.n_attn_wg + P.jobs[0].n_wg), dim3(256), lds, c->stream,
                     A.state, A.kv, (const float*)c->X, E | (w << 16) | (nkv << 24), (const uint64_t*)c->qkv_tag,
                     attn_dims(A, D.n_heads / D.n_kv_heads), A.max_ctx, A, Q, P);
}

// attn_out: X += Wo * x(attn)
// pend: as in enqueue_qkv, the residual X + the previous FFN's terms
void enqueue_attn_out(c2h_ctx* c, int l, bool pend = false) {
  if (!pend) {
    launch_group(c, {{&c->layers[l].wo, nullptr, c->X, nullptr}}, PRO_QUANT, MODE_RESID, c->attn, c->desc.n_embd,
                 nullptr);
    return;
  }
  const int E = c->desc.n_embd;
  GemvParams P = base_params(c);
  add_job(P, c->layers[l].wo, nullptr, MODE_RESID, c->X, nullptr, nullptr);
  P.prologue = PRO_QUANT;
  P.x = c->attn;
  P.x_out = c->X;
  P.n_x = E;
  P.n_x_lds = chain_lds_floats(E);
  P.nb_in = nb_k(E);
  P.x_pend = c->dterm;
  P.pend_n = E;
  prep_gemv_row(P);
  hipLaunchKernelGGL((k_gemv_row_pend<3, PRO_QUANT, MODE_RESID>), job_grid(P),
                     dim3(row_threads(3, PRO_QUANT, MODE_RESID)), 0, c->stream, P.x, P.n_x, P);
}

// ffn_in: h = SwiGLU(Wg * n, Wu * n), n = x(RMSNorm(X))
void enqueue_ffn_in(c2h_ctx* c, int l) {
  Layer& L = c->layers[l];
  launch_group(c, {{&L.wg, &L.wu, c->h, nullptr}}, PRO_NORM, MODE_SWIGLU, c->X, c->desc.n_embd, L.ffn_norm);
}

// ffn_out: X += Wd * x(h)
void enqueue_ffn_out(c2h_ctx* c, int l) {
  launch_group(c, {{&c->layers[l].wd, nullptr, c->X, nullptr}}, PRO_QUANT, MODE_RESID, c->h, c->desc.n_ff, nullptr);
}

// Whether layer l runs q|k|v, attention and attn_out as launches of their
// own that can add X's pending terms (k_gemv_row_pend): past layer 0, no
// fused attention launch at this form, K-quant q/k/v/o rows of 3
// super-blocks.
bool pend_separate(const c2h_ctx* c, int l, int form) {
  const Layer& L = c->layers[l];
  return l > 0 && nb_k(c->desc.n_embd) == 3 && !fuse_attn_block(c, l, form) && !fuse_attn_block_f(c, l, form) &&
         !fuse_attn_oproj(c, l, form) && !float_input(L.wq.type) && !float_input(L.wk.type) &&
         !float_input(L.wv.type) && !float_input(L.wo.type);
}

// The tensor types the FFN launch reads on layer l: a Q6_K down projection
// of FOLD_NB super-blocks (the instances built), and gate/up either K-quants
// of 3 super-blocks per row (k_ffn_block) or both the same Q5_0 / Q8_0 type
// over rows of a multiple of 128 values (k_ffn_block_f); rows of at most
// 1,024 values (the final norm adds the last layer's terms with 256
// threads, a float4 each).
bool ffn_block_types(const c2h_ctx* c, int l) {
  const c2h_model_desc& D = c->desc;
  const Layer& L = c->layers[l];
  if (nb_k(D.n_ff) != FOLD_NB || L.wd.type != C2H_Q6_K || D.n_embd > 1024) return false;
  const bool fg = float_input(L.wg.type), fu = float_input(L.wu.type);
  if (!fg && !fu) return nb_k(D.n_embd) == 3;
  return fg && fu && L.wg.type == L.wu.type && D.n_embd % 128 == 0;
}

// Whether layer l's FFN runs as one launch that leaves its residual add to
// the next launch: the next layer's fused attention launch (k_attn_block or
// k_attn_block_f) or its q|k|v and attn_out launches (pend_separate), or
// after the last layer the final norm, which add the terms.
bool defer_ffn(const c2h_ctx* c, int l, int form) {
  if (!c->fuse_ffn || !ffn_block_types(c, l)) return false;
  return l + 1 >= c->desc.n_layers || fuse_attn_block(c, l + 1, form) || fuse_attn_block_f(c, l + 1, form) ||
         pend_separate(c, l + 1, form);
}

// ffn_in + ffn_out but for the residual add in one launch: gate|up stores h
// tagged, the down projection runs by super-block on the tagged h and
// leaves its terms in dterm for the next fused attention launch to add to X
void enqueue_ffn_block(c2h_ctx* c, int l) {
  const c2h_model_desc& D = c->desc;
  Layer& L = c->layers[l];
  const bool fin = float_input(L.wg.type);
  GemvParams I = base_params(c);
  add_job(I, L.wg, &L.wu, MODE_SWIGLU, c->h, nullptr, nullptr);
  I.jobs[0].spare = 0;
  I.prologue = PRO_NORM;
  I.x = c->X;
  I.x_out = c->X;
  I.n_x = D.n_embd;
  I.n_x_lds = chain_lds_floats(D.n_embd);
  I.norm_w = L.ffn_norm;
  I.nb_in = fin ? nb8_of(D.n_embd) : nb_k(D.n_embd);
  I.y_tag = c->h_tag;
  if (!fin) prep_gemv_row(I);
  GemvParams O = base_params(c);
  add_job(O, L.wd, nullptr, MODE_RESID, c->dterm, nullptr, nullptr);
  const int rw = fin ? 64 : 128;  // down rows per workgroup: 256 or 512 threads
  O.jobs[0].n_wg = FOLD_NB * ((D.n_embd + rw - 1) / rw);  // down_block_body workgroups
  O.x = c->h;
  O.n_x = D.n_ff;
  O.x_tag = c->h_tag;
  O.wait_err = c->tok_host + 2;
  const int n_in = I.jobs[0].n_wg;
  if (fin)
    hipLaunchKernelGGL(k_ffn_block_f<FOLD_NB>, dim3(n_in + O.jobs[0].n_wg), dim3(256),
                       (size_t)gemv_f_lds_floats(D.n_embd) * sizeof(float), c->stream, c->state_dev, n_in << 16, l, I,
                       O);
  else
    hipLaunchKernelGGL((k_ffn_block<3, FOLD_NB>), dim3(n_in + O.jobs[0].n_wg), dim3(512),
                       (size_t)I.n_x_lds * sizeof(float), c->stream, (const float*)c->X, D.n_embd | (n_in << 16),
                       c->state_dev, l, I, O);
}

// k_rmsnorm holds one float4 per thread
int norm_threads(int n) { return n <= 1024 ? 256 : 512; }

// the final RMSNorm into the normX buffer the step state names; a step
// graph's also leaves the next step's state (advance)
// pend: the last layer's FFN launch left its terms for X (dterm)
void enqueue_final_norm(c2h_ctx* c, int advance = 0, bool pend = false) {
  const c2h_model_desc& D = c->desc;
  NormParams N;
  memset(&N, 0, sizeof(N));
  N.x = c->X;
  N.w = c->output_norm;
  N.eps = D.rms_eps;
  N.n = D.n_embd;
  N.out_sel = 1;
  N.out_buf[0] = c->normx[0];
  N.out_buf[1] = c->normx[1];
  N.state = c->state_dev;
  N.n_lds = chain_lds_floats(D.n_embd);
  N.advance = advance;
  N.x_pend = pend ? c->dterm : nullptr;
  N.x_back = c->X;
  if (D.head_dim == 64) {  // the advance leaves the next position's RoPE row in the state
    N.rope_cos = c->rope_cos;
    N.rope_sin = c->rope_sin;
    N.rope_len = D.max_ctx;
  }
  hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(norm_threads(D.n_embd)), (size_t)N.n_lds * sizeof(float), c->stream, N);
}

// The 24-layer body of engine.Forward plus the final RMSNorm; layer 0 embeds
// either state->token (forward) or the argmax of the vocab partials (step).
// form selects the attention kernels.
void enqueue_layers(c2h_ctx* c, bool from_argmax, int form) {
  bool pend = false;  // the previous layer's FFN left its residual add to this layer's k_attn_block
  for (int l = 0; l < c->desc.n_layers; ++l) {
    if (fuse_attn_block(c, l, form)) {
      enqueue_attn_block(c, l, form, pend);
    } else if (fuse_attn_block_f(c, l, form)) {
      enqueue_attn_block_f(c, l, form, pend);
    } else {
      // (pend here means pend_separate: layer l > 0, no fused launch)
      enqueue_qkv(c, l, (l == 0) ? (from_argmax ? PRO_ARGMAX_EMBED_NORM : PRO_EMBED_NORM) : PRO_NORM, pend);
      if (fuse_attn_oproj(c, l, form)) {
        enqueue_attn_oproj(c, l, form);
      } else {
        enqueue_attn(c, l, form);
        enqueue_attn_out(c, l, pend);
      }
    }
    pend = defer_ffn(c, l, form);
    if (pend) {
      enqueue_ffn_block(c, l);
    } else {
      enqueue_ffn_in(c, l);
      enqueue_ffn_out(c, l);
    }
  }
  enqueue_final_norm(c, from_argmax ? 1 : 0, pend);
}

void enqueue_step(c2h_ctx* c, int form) {
  enqueue_vocab(c, 1, nullptr, 1, nullptr);
  enqueue_layers(c, true, form);
}

int validate_model(c2h_ctx* c) {
  if (!c->has_model) return fail(c, C2H_ERR_STATE, "context has no model");
  if (!c->embd.present() || c->embd.type != C2H_Q8_0)
    return fail(c, C2H_ERR_STATE, "token_embd (Q8_0) not uploaded");
  if (c->output.present() && c->output.type == C2H_Q5_0) {
    int rc = dot_rows_ready(c, c->output.cols);
    if (rc) return rc;
  }
  if (!c->output_norm) return fail(c, C2H_ERR_STATE, "output_norm not uploaded");
  for (int l = 0; l < c->desc.n_layers; ++l) {
    Layer& L = c->layers[l];
    if (!L.attn_norm || !L.ffn_norm) return fail(c, C2H_ERR_STATE, "layer %d norms missing", l);
    if ((L.q_norm || L.k_norm) && c->desc.head_dim != 128)
      return fail(c, C2H_ERR_UNSUPPORTED, "layer %d: QK-norm runs with head_dim 128", l);
    const Tensor* ts[] = {&L.wq, &L.wk, &L.wv, &L.wo, &L.wg, &L.wu, &L.wd};
    for (const Tensor* t : ts) {
      if (!t->present()) return fail(c, C2H_ERR_STATE, "layer %d projection missing", l);
      if (t->type != C2H_Q4_K && t->type != C2H_Q6_K && t->type != C2H_Q5_0 && t->type != C2H_Q8_0)
        return fail(c, C2H_ERR_UNSUPPORTED, "layer %d: projections must be Q4_K, Q6_K, Q5_0 or Q8_0", l);
      const int64_t want_cols = (t == &L.wd) ? c->desc.n_ff : c->desc.n_embd;
      if (t->cols != want_cols) return fail(c, C2H_ERR_INVALID, "layer %d: projection has %lld columns, expected %lld", l,
                                            (long long)t->cols, (long long)want_cols);
      if (t->type == C2H_Q8_0 && nb8_of(t->cols) > 32)
        return fail(c, C2H_ERR_UNSUPPORTED, "layer %d: Q8_0 projections run up to 1024 columns", l);
      if (float_input(t->type) && t != &L.wd && c->desc.n_embd > 1024)
        return fail(c, C2H_ERR_UNSUPPORTED, "layer %d: Q5_0/Q8_0 projections need n_embd <= 1024", l);
    }
    if (L.wg.cols != L.wu.cols || L.wg.rows != L.wu.rows)
      return fail(c, C2H_ERR_INVALID, "layer %d gate/up shapes differ", l);
    if (float_input(L.wg.type) != float_input(L.wu.type) || (float_input(L.wg.type) && L.wg.type != L.wu.type))
      return fail(c, C2H_ERR_UNSUPPORTED, "layer %d: gate and up must both be Q5_0, both Q8_0, or both K-quants", l);
  }
  return C2H_OK;
}

void destroy_graphs(c2h_ctx* c) {
  for (int t = 0; t < ATT_FORMS; ++t) {
    if (c->g_step[t]) (void)hipGraphExecDestroy(c->g_step[t]);
    if (c->g_fwd[t]) (void)hipGraphExecDestroy(c->g_fwd[t]);
    c->g_step[t] = c->g_fwd[t] = nullptr;
  }
}

int build_graphs(c2h_ctx* c) {
  if (c->graphs_ready) return C2H_OK;
  int rc = validate_model(c);
  if (rc) return rc;
  destroy_graphs(c);
  if (c->use_graphs) {
    for (int form = 0; form < ATT_FORMS; ++form) {
      if (!form_used(c, form)) continue;
      for (int which = 0; which < 2; ++which) {
        hipGraph_t g;
        HIPCHK(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
        if (which == 0)
          enqueue_step(c, form);
        else
          enqueue_layers(c, false, form);
        HIPCHK(c, hipStreamEndCapture(c->stream, &g));
        hipGraphExec_t ge;
        HIPCHK(c, hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        (void)hipGraphDestroy(g);
        (which == 0 ? c->g_step : c->g_fwd)[form] = ge;
      }
    }
  }
  c->graphs_ready = true;
  return C2H_OK;
}

// Writes the per-launch state through a ring of pinned slots; the stream
// orders the copy before the graph.  Slots are reused only after a sync.
int push_state(c2h_ctx* c, const C2hState& s) {
  c->state_pred_valid = false;
  unsigned slot = c->ring_next++ % kStateRing;
  if (slot == 0 && c->ring_next > 1) HIPCHK(c, hipStreamSynchronize(c->stream));
  C2hState& t = c->state_ring[slot];
  t = s;
  if (!c->rope_cos_h.empty()) {  // the RoPE row of pos, as the decode attention tiers read it
    const int rp = std::min(std::max(s.pos, 0), c->desc.max_ctx - 1);
    memcpy(t.rope, &c->rope_cos_h[(size_t)rp * 32], 32 * 4);
    memcpy(t.rope + 32, &c->rope_sin_h[(size_t)rp * 32], 32 * 4);
  }
  // (the epoch, the last field, stays the device's)
  HIPCHK(c, hipMemcpyAsync(c->state_dev, &c->state_ring[slot], kStatePushBytes, hipMemcpyHostToDevice, c->stream));
  return C2H_OK;
}

// A handover wait inside a launch (k_attn_oproj) that ran out sets the
// pinned flag; the next entry point that checks reports it, once.
int check_wait_flag(c2h_ctx* c) {
  if (!c->tok_host || __atomic_load_n(&c->tok_host[2], __ATOMIC_ACQUIRE) == 0) return C2H_OK;
  __atomic_store_n(&c->tok_host[2], 0, __ATOMIC_RELEASE);
  return fail(c, C2H_ERR_HIP, "a wait for the attention output inside a launch ran out");
}

// Decode at `pos` attends to pos+1 positions.
int run_graph(c2h_ctx* c, bool step, int pos) {
  const int form = attn_form(c, pos + 1);
  if (c->use_graphs) {
    HIPCHK(c, hipGraphLaunch(step ? c->g_step[form] : c->g_fwd[form], c->stream));
  } else {
    if (step)
      enqueue_step(c, form);
    else
      enqueue_layers(c, false, form);
    HIPCHK(c, hipGetLastError());
  }
  return C2H_OK;
}

thread_local std::string g_create_err;

// `scratch`'s address on each device, looked up once per device (with that
// device current) by the first c2h_create on it.
constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
uint8_t* g_noalloc[kMaxDevices] = {};
std::mutex g_noalloc_call_mu[kMaxDevices];  // held by c2h_quantize_q8k_noalloc per device

int noalloc_setup(c2h_ctx* c) {
  if (c->device < 0 || c->device >= kMaxDevices)
    return fail(c, C2H_ERR_UNSUPPORTED, "device %d beyond the %d this build tracks", c->device, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (!g_noalloc[c->device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(c, C2H_ERR_HIP, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
    g_noalloc[c->device] = reinterpret_cast<uint8_t*>(p);
  }
  c->noalloc = g_noalloc[c->device];
  return C2H_OK;
}

}  // namespace

namespace {

// Device offset of one layer/KV head slot of K (which 0) or V (which 1).
size_t kv_slot_offset(const c2h_model_desc& D, int which, int layer, int kv_head) {
  return (((size_t)which * D.n_layers + layer) * D.n_kv_heads + kv_head) * (size_t)kv_slot(D.max_ctx) * D.head_dim;
}

int check_kv_args(c2h_ctx* c, int which, int layer, int kv_head, int pos0, int n) {
  if (!c->has_model) return fail(c, C2H_ERR_STATE, "kernel-only context");
  const c2h_model_desc& D = c->desc;
  if (which < 0 || which > 1 || layer < 0 || layer >= D.n_layers || kv_head < 0 || kv_head >= D.n_kv_heads)
    return fail(c, C2H_ERR_INVALID, "kv index out of range");
  if (pos0 < 0 || n < 0 || (int64_t)pos0 + n > D.max_ctx)
    return fail(c, C2H_ERR_RANGE, "positions [%d, %d) outside [0, %d)", pos0, pos0 + n, D.max_ctx);
  return C2H_OK;
}

// V rows [pos0, pos0+n) <-> the quad-major slot: the covering quads travel
// whole and are (re)ordered on the host.
int v_rows_copy(c2h_ctx* c, int layer, int kv_head, int pos0, int n, float* rows, bool to_device) {
  const c2h_model_desc& D = c->desc;
  const int hd = D.head_dim, qf = 4 * hd;  // floats per quad
  const int q0 = pos0 >> 2, q1 = (pos0 + n + 3) >> 2;
  std::vector<float> quads((size_t)(q1 - q0) * qf);
  float* dev = c->kv + kv_slot_offset(D, 1, layer, kv_head) + (size_t)q0 * qf;
  HIPCHK(c, stream_copy(c->stream, quads.data(), dev, quads.size() * 4, hipMemcpyDeviceToHost));
  for (int p = pos0; p < pos0 + n; ++p)
    for (int d = 0; d < hd; ++d) {
      float& q = quads[vq_index(p, d, hd) - (size_t)q0 * qf];
      float& r = rows[(size_t)(p - pos0) * hd + d];
      if (to_device)
        q = r;
      else
        r = q;
    }
  if (to_device) HIPCHK(c, stream_copy(c->stream, dev, quads.data(), quads.size() * 4, hipMemcpyHostToDevice));
  return C2H_OK;
}

}  // namespace

// ====================================================================== ABI

extern "C" {

int c2h_create(const c2h_model_desc* desc, int device, c2h_ctx** out) {
  if (!out) return C2H_ERR_INVALID;
  *out = nullptr;
  c2h_ctx* c = new c2h_ctx();
  c->device = device;
  g_create_err.clear();
  auto bail = [&](int rc) {
    g_create_err = c->err.empty() ? "HIP runtime call failed during create" : c->err;
    c2h_destroy(c);
    return rc;
  };
  if (hipSetDevice(device) != hipSuccess) {
    g_create_err = "hipSetDevice failed";
    delete c;
    return C2H_ERR_HIP;
  }
  if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
    g_create_err = "hipStreamCreate failed";
    delete c;
    return C2H_ERR_HIP;
  }
  const char* ng = getenv("C2H_NO_GRAPH");
  c->use_graphs = !(ng && ng[0] == '1');
  // measurement aid: C2H_NO_FUSE=1 separate launches, =qkv qkv on its own,
  // =ffn the FFN's two launches apart
  const char* nf = getenv("C2H_NO_FUSE");
  c->fuse_oproj = !(nf && nf[0] == '1');
  c->fuse_qkv = c->fuse_oproj && !(nf && strcmp(nf, "qkv") == 0);
  c->fuse_ffn = c->fuse_oproj && !(nf && strcmp(nf, "ffn") == 0);
  void* pinned = nullptr;
  if (hipHostMalloc(&pinned, sizeof(C2hState) * kStateRing + 64, hipHostMallocDefault) != hipSuccess) return bail(C2H_ERR_HIP);
  c->state_ring = reinterpret_cast<C2hState*>(pinned);
  c->tok_host = reinterpret_cast<int32_t*>(reinterpret_cast<uint8_t*>(pinned) + sizeof(C2hState) * kStateRing);
  c->tok_host[0] = 0;
  c->tok_host[1] = -1;
  c->tok_host[2] = 0;
  int rc;
  if ((rc = noalloc_setup(c))) return bail(rc);
  if ((rc = dalloc(c, &c->state_dev, sizeof(C2hState)))) return bail(rc);
  // the epoch (which no state push writes) starts at 0
  if (hipMemsetAsync(c->state_dev, 0, sizeof(C2hState), c->stream) != hipSuccess) return bail(C2H_ERR_HIP);
  if (!desc) {
    C2hState s0;
    memset(&s0, 0, sizeof(s0));
    s0.penalty = 1.15f;
    s0.im_end = -1;
    s0.eos = -1;
    if (push_state(c, s0) || hipStreamSynchronize(c->stream) != hipSuccess) return bail(C2H_ERR_HIP);
    *out = c;
    return C2H_OK;
  }
  const c2h_model_desc& D = *desc;
  if (D.n_layers <= 0 || D.n_embd <= 0 || D.n_heads <= 0 || D.n_kv_heads <= 0 || D.n_ff <= 0 || D.n_vocab <= 0 ||
      D.max_ctx <= 0)
    return bail(fail(c, C2H_ERR_INVALID, "model dimensions must be positive"));
  if (D.n_layers > 255) return bail(fail(c, C2H_ERR_UNSUPPORTED, "this build runs up to 255 layers"));
  // engine/model.go:137: head_dim = n_embd / n_heads (64 for Qwen2.5-0.5B,
  // 128 for Qwen3-1.7B)
  if ((D.head_dim != 64 && D.head_dim != 128) || D.n_embd != D.n_heads * D.head_dim || D.n_heads % D.n_kv_heads)
    return bail(fail(c, C2H_ERR_UNSUPPORTED, "this build runs head_dim 64 or 128 with n_embd = n_heads*head_dim"));
  if (D.n_embd < 256 || D.n_ff < 256)
    return bail(fail(c, C2H_ERR_UNSUPPORTED, "K-quant projections need n_embd and n_ff of at least 256"));
  if (D.n_embd % 32 || D.n_embd > 2048 || D.n_ff % 4 || D.n_ff > 16384)
    return bail(fail(c, C2H_ERR_UNSUPPORTED, "n_embd must be a multiple of 32 up to 2048, n_ff up to 16384"));
  if (!gemv_row_kernel(nb_k(D.n_embd), PRO_NORM, MODE_BIAS) || !gemv_row_kernel(nb_k(D.n_embd), PRO_QUANT, MODE_RESID) ||
      !gemv_row_kernel(nb_k(D.n_embd), PRO_NORM, MODE_SWIGLU) ||
      !gemv_row_kernel(nb_k(D.n_ff), PRO_QUANT, MODE_RESID))
    return bail(fail(c, C2H_ERR_UNSUPPORTED,
                     "no kernel instance for n_embd %d / n_ff %d (built: n_embd/256 in {3,4,6,8}, n_ff/256 in "
                     "{3,4,6,8,12,19,24,35,43})",
                     D.n_embd, D.n_ff));
  c->desc = D;
  c->has_model = true;
  c->layers.resize(D.n_layers);
  const int E = D.n_embd, KV = D.n_kv_heads * D.head_dim, F = D.n_ff;
  if ((rc = dalloc(c, &c->X, E * 4)) || (rc = dalloc(c, &c->q, E * 4)) || (rc = dalloc(c, &c->k, KV * 4)) ||
      (rc = dalloc(c, &c->v, KV * 4)) || (rc = dalloc(c, &c->attn, E * 4)) || (rc = dalloc(c, &c->h, F * 4)) ||
      (rc = dalloc(c, &c->normx[0], E * 4)) || (rc = dalloc(c, &c->normx[1], E * 4)) ||
      (rc = dalloc(c, &c->attn_tag, (size_t)E * 8)) || (rc = dalloc(c, &c->qkv_tag, (size_t)(E + 2 * KV) * 8)) ||
      (rc = dalloc(c, &c->h_tag, (size_t)F * 8)) || (rc = dalloc(c, &c->dterm, (size_t)FOLD_NB * E * 4)))
    return bail(rc);
  // tag 0xffffffff: no launch's (its layer field would be 255)
  if (hipMemsetAsync(c->attn_tag, 0xff, (size_t)E * 8, c->stream) != hipSuccess ||
      hipMemsetAsync(c->qkv_tag, 0xff, (size_t)(E + 2 * KV) * 8, c->stream) != hipSuccess ||
      hipMemsetAsync(c->h_tag, 0xff, (size_t)F * 8, c->stream) != hipSuccess ||
      hipMemsetAsync(c->dterm, 0, (size_t)FOLD_NB * E * 4, c->stream) != hipSuccess)
    return bail(C2H_ERR_HIP);
  size_t kv_bytes = (size_t)2 * D.n_layers * D.n_kv_heads * kv_slot(D.max_ctx) * D.head_dim * 4;
  if ((rc = dalloc(c, &c->kv, kv_bytes))) return bail(rc);
  if ((rc = dalloc(c, &c->token_ids, (size_t)D.max_ctx * 4))) return bail(rc);
  // cleared on the context stream (before any of its work), finished here
  if (hipMemsetAsync(c->kv, 0, kv_bytes, c->stream) != hipSuccess ||
      hipMemsetAsync(c->token_ids, 0, (size_t)D.max_ctx * 4, c->stream) != hipSuccess ||
      hipMemsetAsync(c->normx[0], 0, E * 4, c->stream) != hipSuccess ||
      hipMemsetAsync(c->normx[1], 0, E * 4, c->stream) != hipSuccess || hipStreamSynchronize(c->stream) != hipSuccess)
    return bail(fail(c, C2H_ERR_HIP, "clearing the KV cache and state"));
  // RoPE table, tensor.NewRoPETable (tensor/ops.go:237-257) in float64
  {
    int half = D.head_dim / 2;
    std::vector<float> cs((size_t)D.max_ctx * half), sn((size_t)D.max_ctx * half);
    for (int p = 0; p < D.max_ctx; ++p)
      for (int i = 0; i < half; ++i) {
        double freq = 1.0 / std::pow((double)D.rope_theta, (double)(2 * i) / (double)D.head_dim);
        double val = (double)p * freq;
        cs[(size_t)p * half + i] = (float)std::cos(val);
        sn[(size_t)p * half + i] = (float)std::sin(val);
      }
    if ((rc = dalloc(c, &c->rope_cos, cs.size() * 4)) || (rc = dalloc(c, &c->rope_sin, sn.size() * 4))) return bail(rc);
    if (stream_copy(c->stream, c->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        stream_copy(c->stream, c->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
      return bail(fail(c, C2H_ERR_HIP, "rope upload"));
    if (half == 32) {
      c->rope_cos_h = std::move(cs);
      c->rope_sin_h = std::move(sn);
    }
  }
  if ((rc = vocab_grid(c, D.n_vocab, D.n_embd, &c->n_part))) return bail(rc);
  if ((rc = dalloc(c, &c->part_v, (size_t)c->n_part * 4)) || (rc = dalloc(c, &c->part_i, (size_t)c->n_part * 4)) ||
      (rc = dalloc(c, &c->logits, (size_t)D.n_vocab * 4)) ||
      (rc = dalloc(c, &c->vq8k, (size_t)nb_k(D.n_embd) * BS_Q8K)))
    return bail(rc);
  // Attention: k_attn_core while a token attends to at most att_split
  // positions (staged V | all scores in LDS, within the 160 KB of a gfx950
  // workgroup, 8 KB kept for static shared data), the long-context kernels
  // beyond.  C2H_ATT_SPLIT overrides the split length (measurement aid).
  for (const void* k : {(const void*)k_pf_gemm_q6<MODE_BIAS, 2>, (const void*)k_pf_gemm_q6<MODE_RESID, 2>})
    if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, PF_Q6_LDS_MAX) != hipSuccess)
      return bail(fail(c, C2H_ERR_HIP, "prefill Q6_K GEMM LDS attribute"));
  if (D.head_dim == 128) {  // k_attn_h128 at every T: the scores of max_ctx positions in LDS
    c->attn_lds = (size_t)attn_h128_lds_floats(D.max_ctx) * 4;
    if (c->attn_lds > 152u * 1024)
      return bail(fail(c, C2H_ERR_UNSUPPORTED, "head_dim 128 runs up to %d positions", 152 * 256 - 64));
    // V staged through LDS where its two chunks fit beside the scores
    c->h128_staged = c->attn_lds + (size_t)attn_h128_v_lds_floats() * 4 <= 152u * 1024;
    if (c->h128_staged) c->attn_lds += (size_t)attn_h128_v_lds_floats() * 4;
    if (hipFuncSetAttribute(c->h128_staged ? (const void*)k_attn_h128<H128_VCH> : (const void*)k_attn_h128<0>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)c->attn_lds) != hipSuccess)
      return bail(fail(c, C2H_ERR_HIP, "attention LDS attribute"));
    c->att_split = D.max_ctx;
  } else {
    c->att_split = ATT_SPLIT_T;
    if (const char* sp = getenv("C2H_ATT_SPLIT")) c->att_split = std::max(1, atoi(sp));
    while (c->att_split > 1 && (size_t)attn_lds_floats(c->att_split) * 4 > 152u * 1024) --c->att_split;
    c->att_split = std::min(c->att_split, D.max_ctx);
    c->long_attn = D.max_ctx > c->att_split;
    c->attn_lds = (size_t)attn_lds_floats(c->att_split) * 4;
    {
      for (int form = 0; form <= ATT_FORM_CORE; ++form)
        if (hipFuncSetAttribute((const void*)attn_core_kernel(form), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)c->attn_lds) != hipSuccess ||
            hipFuncSetAttribute((const void*)attn_oproj_kernel(form), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)c->attn_lds) != hipSuccess ||
            hipFuncSetAttribute((const void*)attn_block_kernel(form), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)std::max(c->attn_lds, (size_t)chain_lds_floats(D.n_embd) * 4)) != hipSuccess ||
            hipFuncSetAttribute((const void*)attn_block_f_kernel(form), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)std::max(c->attn_lds, (size_t)gemv_f_lds_floats(D.n_embd) * 4)) != hipSuccess)
          return bail(fail(c, C2H_ERR_HIP, "attention LDS attribute"));
      const void* pff[] = {(const void*)k_pf_gemm_f<MODE_BIAS>, (const void*)k_pf_gemm_f<MODE_RESID>,
                           (const void*)k_pf_gemm_q50<MODE_BIAS>, (const void*)k_pf_gemm_q50<MODE_RESID>};
      for (const void* k : pff)
        if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, PF_F_LDS_MAX) != hipSuccess)
          return bail(fail(c, C2H_ERR_HIP, "prefill GEMM LDS attribute"));
      // k_pf_attn keeps the scores of up to att_split positions per token in LDS
      c->pfa_max_pos = c->att_split;
      while (c->pfa_max_pos > 1 && (size_t)pfa_lds_floats(c->pfa_max_pos - 1) * 4 > 152u * 1024) --c->pfa_max_pos;
      if (hipFuncSetAttribute((const void*)k_pf_attn, hipFuncAttributeMaxDynamicSharedMemorySize,
                              pfa_lds_floats(c->pfa_max_pos - 1) * 4) != hipSuccess)
        return bail(fail(c, C2H_ERR_HIP, "prefill attention LDS attribute"));
    }
    if (c->long_attn) {
      if (D.max_ctx > ATT_LONG_MAX_CTX)
        return bail(fail(c, C2H_ERR_UNSUPPORTED, "max_ctx %d above the %d positions of the exact attention kernels",
                         D.max_ctx, ATT_LONG_MAX_CTX));
      if (D.n_heads / D.n_kv_heads > ATT_MAX_QPKV)
        return bail(fail(c, C2H_ERR_UNSUPPORTED, "more than %d query heads per KV head", ATT_MAX_QPKV));
      c->att_sc_ld = (D.max_ctx + 3) & ~3;
      c->att_n_blk = (D.max_ctx + ATT_SB - 1) / ATT_SB;
      if ((rc = dalloc(c, &c->att_sc, (size_t)PF_ATT_SUB * D.n_heads * c->att_sc_ld * 4)) ||
          (rc = dalloc(c, &c->att_bmax, (size_t)PF_ATT_SUB * D.n_heads * c->att_n_blk * 4)))
        return bail(rc);
      if (hipFuncSetAttribute((const void*)k_attn_softmax, hipFuncAttributeMaxDynamicSharedMemorySize,
                              attn_softmax_lds_floats(D.max_ctx) * 4) != hipSuccess ||
          hipFuncSetAttribute((const void*)k_attn_av, hipFuncAttributeMaxDynamicSharedMemorySize,
                              ATT_AV_LDS_FLOATS * 4) != hipSuccess)
        return bail(fail(c, C2H_ERR_HIP, "long attention LDS attribute"));
    }
  }
  C2hState s0;
  memset(&s0, 0, sizeof(s0));
  s0.penalty = 1.15f;
  s0.nx_out = 1;
  if (push_state(c, s0) || hipStreamSynchronize(c->stream) != hipSuccess) return bail(C2H_ERR_HIP);
  *out = c;
  return C2H_OK;
}

void c2h_destroy(c2h_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  destroy_graphs(c);
  for (void* p : c->allocs) (void)hipFree(p);
  if (c->ids_dev) (void)hipFree(c->ids_dev);
  if (c->ids_y) (void)hipFree(c->ids_y);
  if (c->state_ring) (void)hipHostFree(c->state_ring);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  delete c;
}

const char* c2h_last_error(const c2h_ctx* c) {
  if (!c) return g_create_err.c_str();
  return c->err.c_str();
}

int c2h_upload_tensor(c2h_ctx* c, int32_t layer, int32_t role, int32_t type, int64_t rows, int64_t cols,
                      const void* host, size_t bytes) {
  if (!c || !host) return C2H_ERR_INVALID;
  if (!c->has_model) return fail(c, C2H_ERR_STATE, "kernel-only context");
  HIPCHK(c, hipSetDevice(c->device));
  const c2h_model_desc& D = c->desc;
  const int64_t E = D.n_embd, KV = (int64_t)D.n_kv_heads * D.head_dim, F = D.n_ff, V = D.n_vocab;
  auto want = [&](int64_t r, int64_t cl) -> int {
    if (rows != r || cols != cl)
      return fail(c, C2H_ERR_INVALID, "role %d: shape %lldx%lld, expected %lldx%lld", role, (long long)rows,
                  (long long)cols, (long long)r, (long long)cl);
    return C2H_OK;
  };
  int rc;
  if (role == C2H_ROLE_TOKEN_EMBD) {
    if ((rc = want(V, E))) return rc;
    if (type != C2H_Q8_0) return fail(c, C2H_ERR_UNSUPPORTED, "token_embd must be Q8_0");
    return upload_quant(c, &c->embd, type, rows, cols, host, bytes);
  }
  if (role == C2H_ROLE_OUTPUT) {
    if ((rc = want(V, E))) return rc;
    // Q8_0 runs the fused vocab kernel; Q4_K / Q6_K / Q5_0 the pooled GEMV and k_logits_pick
    return upload_quant(c, &c->output, type, rows, cols, host, bytes);
  }
  if (role == C2H_ROLE_OUTPUT_NORM) return upload_f32(c, &c->output_norm, E, type, rows, cols, host, bytes);
  if (layer < 0 || layer >= D.n_layers) return fail(c, C2H_ERR_INVALID, "layer %d out of range", layer);
  Layer& L = c->layers[layer];
  switch (role) {
    case C2H_ROLE_ATTN_NORM: return upload_f32(c, &L.attn_norm, E, type, rows, cols, host, bytes);
    case C2H_ROLE_FFN_NORM: return upload_f32(c, &L.ffn_norm, E, type, rows, cols, host, bytes);
    case C2H_ROLE_ATTN_Q_BIAS: return upload_f32(c, &L.bq, E, type, rows, cols, host, bytes);
    case C2H_ROLE_ATTN_K_BIAS: return upload_f32(c, &L.bk, KV, type, rows, cols, host, bytes);
    case C2H_ROLE_ATTN_V_BIAS: return upload_f32(c, &L.bv, KV, type, rows, cols, host, bytes);
    case C2H_ROLE_ATTN_Q_NORM: return upload_f32(c, &L.q_norm, D.head_dim, type, rows, cols, host, bytes);
    case C2H_ROLE_ATTN_K_NORM: return upload_f32(c, &L.k_norm, D.head_dim, type, rows, cols, host, bytes);
    case C2H_ROLE_ATTN_Q: if ((rc = want(E, E))) return rc; return upload_quant(c, &L.wq, type, rows, cols, host, bytes);
    case C2H_ROLE_ATTN_K: if ((rc = want(KV, E))) return rc; return upload_quant(c, &L.wk, type, rows, cols, host, bytes);
    case C2H_ROLE_ATTN_V: if ((rc = want(KV, E))) return rc; return upload_quant(c, &L.wv, type, rows, cols, host, bytes);
    case C2H_ROLE_ATTN_OUT: if ((rc = want(E, E))) return rc; return upload_quant(c, &L.wo, type, rows, cols, host, bytes);
    case C2H_ROLE_FFN_GATE: if ((rc = want(F, E))) return rc; return upload_quant(c, &L.wg, type, rows, cols, host, bytes);
    case C2H_ROLE_FFN_UP: if ((rc = want(F, E))) return rc; return upload_quant(c, &L.wu, type, rows, cols, host, bytes);
    case C2H_ROLE_FFN_DOWN: if ((rc = want(E, F))) return rc; return upload_quant(c, &L.wd, type, rows, cols, host, bytes);
  }
  return fail(c, C2H_ERR_INVALID, "unknown role %d", role);
}

int c2h_set_token_ids(c2h_ctx* c, int32_t pos0, const int32_t* ids, int32_t n) {
  if (!c || (!ids && n > 0)) return C2H_ERR_INVALID;
  if (!c->has_model) return fail(c, C2H_ERR_STATE, "kernel-only context");
  if (pos0 < 0 || n < 0 || pos0 + n > c->desc.max_ctx) return fail(c, C2H_ERR_RANGE, "token ids out of range");
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if (n) HIPCHK(c, stream_copy(c->stream, c->token_ids + pos0, ids, (size_t)n * 4, hipMemcpyHostToDevice));
  return C2H_OK;
}

int c2h_forward(c2h_ctx* c, int32_t token, int32_t pos, float* normx_out) {
  if (!c) return C2H_ERR_INVALID;
  HIPCHK(c, hipSetDevice(c->device));
  int rc = build_graphs(c);
  if (rc) return rc;
  if (pos < 0 || pos >= c->desc.max_ctx) return fail(c, C2H_ERR_RANGE, "pos %d outside [0, %d)", pos, c->desc.max_ctx);
  C2hState s;
  memset(&s, 0, sizeof(s));
  s.pos = pos;
  s.token = token;
  s.penalty = 1.15f;
  s.nx_in = c->nx_cur;
  s.nx_out = c->nx_cur ^ 1;
  if ((rc = push_state(c, s))) return rc;
  if ((rc = run_graph(c, false, pos))) return rc;
  c->nx_prev = c->nx_cur;
  c->nx_cur ^= 1;
  c->seq_len = pos + 1;
  if (normx_out) {
    HIPCHK(c, hipMemcpyAsync(normx_out, c->normx[c->nx_cur], (size_t)c->desc.n_embd * 4, hipMemcpyDeviceToHost,
                             c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return check_wait_flag(c);
  }
  return C2H_OK;
}

namespace {

// The split copy (k_q6_pf_pack) of every Q6_K layer projection, built on
// the stream at the first batched prefill after its upload.
int pf_q6_ready(c2h_ctx* c) {
  for (Layer& L : c->layers)
    for (Tensor* t : {&L.wq, &L.wk, &L.wv, &L.wo, &L.wg, &L.wu, &L.wd}) {
      if (t->type != C2H_Q6_K || t->pf6) continue;
      const int tiles = (int)((t->rows + 31) / 32), nb = nb_k(t->cols);
      int rc = dalloc(c, &t->pf6, (size_t)tiles * nb * PF_Q6_TILE_BYTES);
      if (rc) return rc;
      hipLaunchKernelGGL(k_q6_pf_pack, dim3(tiles, nb), dim3(64), 0, c->stream, t->ref(), (int)t->rows, nb, t->pf6);
      HIPCHK(c, hipGetLastError());
    }
  return C2H_OK;
}

int pf_alloc(c2h_ctx* c) {
  if (c->pf.ready) return C2H_OK;
  const c2h_model_desc& D = c->desc;
  const size_t E = D.n_embd, KV = (size_t)D.n_kv_heads * D.head_dim, F = D.n_ff, M = PF_MAX;
  auto& p = c->pf;
  p.nbs = std::max(nb_k(D.n_embd), nb_k(D.n_ff));
  int rc;
  if ((rc = dalloc(c, &p.X, M * E * 4)) || (rc = dalloc(c, &p.q, M * E * 4)) || (rc = dalloc(c, &p.k, M * KV * 4)) ||
      (rc = dalloc(c, &p.v, M * KV * 4)) || (rc = dalloc(c, &p.attn, M * E * 4)) ||
      (rc = dalloc(c, &p.g, M * F * 4)) || (rc = dalloc(c, &p.u, M * F * 4)) || (rc = dalloc(c, &p.h, M * F * 4)) ||
      (rc = dalloc(c, &p.xn, M * E * 4)) ||
      (rc = dalloc(c, &p.q8, M * p.nbs * QK_K)) || (rc = dalloc(c, &p.q8d, M * p.nbs * 4)) ||
      (rc = dalloc(c, &p.q8dT, M * p.nbs * 4)) || (rc = dalloc(c, &p.q8T, M * p.nbs * QK_K)) ||
      (rc = dalloc(c, &p.q8bs, M * p.nbs * 16 * 4)) || (rc = dalloc(c, &p.tok, M * 4)))
    return rc;
  p.ready = true;
  return C2H_OK;
}

// Waves per Q6_K tile: two, each half of the super-blocks, while the
// second wave's terms fit PF_Q6_LDS_MAX (rows of up to 65 super-blocks,
// which covers n_ff up to the 16384 c2h_create accepts); one beyond.
int pf_q6_split(int nb) { return pf_q6_lds_bytes(nb, 2) <= PF_Q6_LDS_MAX ? 2 : 1; }
typedef void (*PFGemmKernel)(PFGemmParams);
PFGemmKernel pf_gemm_kernel(int type, int mode, bool small_tile = false, int q6_split = 1) {
  if (type == C2H_Q4_K) {
    if (small_tile)
      return mode == MODE_RESID ? k_pf_gemm<T_Q4_K, MODE_RESID, 1> : k_pf_gemm<T_Q4_K, MODE_BIAS, 1>;
    return mode == MODE_RESID ? k_pf_gemm<T_Q4_K, MODE_RESID, 4> : k_pf_gemm<T_Q4_K, MODE_BIAS, 4>;
  }
  if (q6_split == 2) return mode == MODE_RESID ? k_pf_gemm_q6<MODE_RESID, 2> : k_pf_gemm_q6<MODE_BIAS, 2>;
  return mode == MODE_RESID ? k_pf_gemm_q6<MODE_RESID, 1> : k_pf_gemm_q6<MODE_BIAS, 1>;
}
// A Q4_K launch whose 64 x 64 tiles would leave CUs idle runs 64-row x
// 16-token workgroups instead (four times as many).
constexpr int PF_SMALL_TILE_WG = 512;

// y[t][r] (=|+=) W * x[t] for the given matrices: Q4_K / Q6_K on the
// Q8_K rows (one MFMA launch per type), Q5_0 / Q8_0 on the f32 rows xf
// (one k_pf_gemm_f launch), as engine/model.go:250-270 dispatches.
void pf_gemm(c2h_ctx* c, int m, int m_pad, int nb, int mode, std::initializer_list<const Tensor*> ws,
             std::initializer_list<float*> ys, std::initializer_list<const float*> biases,
             std::initializer_list<int> ldys, const float* xf, int ldxf, int n_x) {
  std::vector<const Tensor*> W(ws);
  std::vector<float*> Y(ys);
  std::vector<const float*> B(biases);
  std::vector<int> L(ldys);
  for (int type : {(int)C2H_Q4_K, (int)C2H_Q6_K}) {
    PFGemmParams P;
    memset(&P, 0, sizeof(P));
    P.in = PFQ8{c->pf.q8, c->pf.q8d, c->pf.q8bs, c->pf.nbs, c->pf.q8dT, c->pf.q8T};
    P.nb = nb;
    P.m = m;
    int tiles = 0;
    // Q6_K: 32-row tiles of one wave (k_pf_gemm_q6); Q4_K: PF_TILE rows
    const int rows_per_tile = (type == C2H_Q6_K) ? 32 : PF_TILE;
    for (size_t i = 0; i < W.size(); ++i) {
      if (W[i]->type != type) continue;
      PFJob& J = P.jobs[P.n_jobs++];
      J.w = W[i]->ref();
      J.type = type;
      J.rows = (int)W[i]->rows;
      J.tile_begin = tiles;
      tiles += (J.rows + rows_per_tile - 1) / rows_per_tile;
      if (type == C2H_Q6_K) J.w6 = W[i]->pf6;  // built by pf_q6_ready before the first pass
      J.mode = mode;
      J.y = Y[i];
      J.ldy = L[i];
      J.bias = B[i];
    }
    if (P.n_jobs == 0) continue;
    P.m_pad = m_pad;
    P.n_row_tiles = tiles;
    if (type == C2H_Q6_K) {
      const int per_xcd = (tiles * (m_pad / 32) + 7) / 8;
      const int ns = pf_q6_split(nb);
      hipLaunchKernelGGL(pf_gemm_kernel(type, mode, false, ns), dim3(8 * per_xcd), dim3(64 * ns),
                         (size_t)pf_q6_lds_bytes(nb, ns), c->stream, P);
    } else {
      const bool small = tiles * (m_pad / PF_TILE) < PF_SMALL_TILE_WG;
      hipLaunchKernelGGL(pf_gemm_kernel(type, mode, small), dim3(tiles, m_pad / (small ? 16 : PF_TILE)), dim3(256), 0,
                         c->stream, P);
    }
  }
  // float-input jobs: Q5_0 rows of up to PF_Q50_MAXB blocks in one
  // k_pf_gemm_q50 launch, the others (Q8_0, wider Q5_0) in one k_pf_gemm_f
  const int nb8 = n_x / 32;
  for (int batched = 1; batched >= 0; --batched) {
    PFGemmFParams F;
    memset(&F, 0, sizeof(F));
    F.x = xf;
    F.ldx = ldxf;
    F.n_x = n_x;
    F.m = m;
    int tiles = 0;
    for (size_t i = 0; i < W.size(); ++i) {
      if (!float_input(W[i]->type)) continue;
      const bool q50b = W[i]->type == C2H_Q5_0 && nb8 <= PF_Q50_MAXB;
      if (q50b != (batched == 1)) continue;
      PFJob& J = F.jobs[F.n_jobs++];
      J.w = W[i]->ref();
      J.type = W[i]->type;
      J.rows = (int)W[i]->rows;
      J.tile_begin = tiles;
      const int R = (J.type == C2H_Q5_0) ? std::max(1, 256 / nb8) : 32;
      tiles += (J.rows + R - 1) / R;
      J.mode = mode;
      J.y = Y[i];
      J.ldy = L[i];
      J.bias = B[i];
    }
    if (F.n_jobs == 0) continue;
    if (batched) {
      auto k = (mode == MODE_RESID) ? k_pf_gemm_q50<MODE_RESID> : k_pf_gemm_q50<MODE_BIAS>;
      hipLaunchKernelGGL(k, dim3(tiles, (m + PF_FT - 1) / PF_FT), dim3(256), (size_t)pf_gemm_q50_lds_bytes(n_x),
                         c->stream, F);
    } else {
      // tokens one after another per workgroup: fewer of them when the rows
      // alone would leave CUs idle (the 128 rows of attn_v)
      F.ft = PF_FT;
      while (F.ft > 1 && tiles * ((m + F.ft - 1) / F.ft) < 512) F.ft /= 2;
      auto k = (mode == MODE_RESID) ? k_pf_gemm_f<MODE_RESID> : k_pf_gemm_f<MODE_BIAS>;
      hipLaunchKernelGGL(k, dim3(tiles, (m + F.ft - 1) / F.ft), dim3(256), (size_t)pf_gemm_f_lds_bytes(n_x),
                         c->stream, F);
    }
  }
}

typedef void (*PFNormKernel)(PFNormParams);
typedef void (*PFQuantKernel)(PFQuantParams);
PFNormKernel pf_norm_kernel(int nb) { return nb == 3 ? k_pf_norm_quant<3> : k_pf_norm_quant<4>; }
PFQuantKernel pf_quant_kernel(int nb) {
  switch (nb) {
    case 3: return k_pf_quant<3>;
    case 4: return k_pf_quant<4>;
    case 12: return k_pf_quant<12>;
    default: return k_pf_quant<19>;
  }
}

// One pass of up to PF_MAX tokens at positions pos0.. (engine.Forward per
// token, batched layer by layer).
int pf_pass(c2h_ctx* c, const int32_t* tokens, int m, int pos0) {
  const c2h_model_desc& D = c->desc;
  const int E = D.n_embd, KV = D.n_kv_heads * D.head_dim, F = D.n_ff;
  const int m_pad = (m + PF_TILE - 1) / PF_TILE * PF_TILE;
  auto& p = c->pf;
  int rc;
  HIPCHK(c, hipMemcpyAsync(p.tok, tokens, (size_t)m * 4, hipMemcpyHostToDevice, c->stream));
  HIPCHK(c, hipMemcpyAsync(c->token_ids + pos0, p.tok, (size_t)m * 4, hipMemcpyDeviceToDevice, c->stream));
  C2hState s;
  memset(&s, 0, sizeof(s));
  s.pos = pos0;
  s.penalty = 1.15f;
  s.nx_in = c->nx_cur;
  s.nx_out = c->nx_cur ^ 1;
  if ((rc = push_state(c, s))) return rc;
  const PFQ8 q8{p.q8, p.q8d, p.q8bs, p.nbs, p.q8dT, p.q8T};
  const size_t norm_lds = (size_t)chain_lds_floats(E) * 4;
  for (int l = 0; l < D.n_layers; ++l) {
    Layer& L = c->layers[l];
    {  // [embed] RMSNorm -> Q8_K
      PFNormParams N;
      memset(&N, 0, sizeof(N));
      N.embed = (l == 0);
      N.n_x = E;
      N.eps = D.rms_eps;
      N.X = p.X;
      N.norm_w = L.attn_norm;
      N.tokens = p.tok;
      N.emb = c->embd.ref();
      N.n_vocab = D.n_vocab;
      N.m = m;
      N.nb = nb_k(E);
      N.out = q8;
      N.xn = p.xn;
      hipLaunchKernelGGL(pf_norm_kernel(nb_k(E)), dim3(m_pad), dim3(256), norm_lds, c->stream, N);
    }
    pf_gemm(c, m, m_pad, nb_k(E), MODE_BIAS, {&L.wq, &L.wk, &L.wv}, {p.q, p.k, p.v}, {L.bq, L.bk, L.bv},
            {E, KV, KV}, p.xn, E, E);
    {
      PFRopeParams R;
      memset(&R, 0, sizeof(R));
      R.k = p.k;
      R.v = p.v;
      R.ld = KV;
      R.kv = c->kv;
      R.rope_cos = c->rope_cos;
      R.rope_sin = c->rope_sin;
      R.rope_len = D.max_ctx;
      R.pos0 = pos0;
      R.m = m;
      R.layer = l;
      R.n_layers = D.n_layers;
      R.n_kv_heads = D.n_kv_heads;
      R.max_ctx = D.max_ctx;
      hipLaunchKernelGGL(k_pf_rope_store, dim3(m, D.n_kv_heads), dim3(64), 0, c->stream, R);
    }
    {  // causal attention of every token (its K/V and the earlier ones are stored)
      AttnCoreParams A = attn_params(c, l);
      A.q = p.q;
      A.k = p.k;
      A.v = p.v;
      A.out = p.attn;
      A.q_ld = E;
      A.kv_ld = KV;
      A.out_ld = E;
      A.store_kv = 0;
      if (pos0 + m <= c->att_split && pos0 + m <= c->pfa_max_pos) {
        // blocks of PFA_TB query tokens per head, longest first, K/V chunks shared by the block
        A.n_tok = m;
        A.sc_ld = pfa_sc_ld(pos0 + m - 1);
        hipLaunchKernelGGL(k_pf_attn, dim3(D.n_heads * ((m + PFA_TB - 1) / PFA_TB)), dim3(256),
                           (size_t)pfa_lds_floats(pos0 + m - 1) * 4, c->stream, A);
      } else if (pos0 + m <= c->att_split) {
        const size_t lds = (size_t)attn_lds_floats(pos0 + m) * 4;
        hipLaunchKernelGGL(k_attn_core<ATT_TIER_ANY>, dim3(D.n_heads / D.n_kv_heads, D.n_kv_heads, m), dim3(256), lds,
                           c->stream, A.state, A.kv, A.q, A.k, A.v, attn_dims(A, D.n_heads / D.n_kv_heads), A.max_ctx, A);
      } else {
        for (int t0 = 0; t0 < m; t0 += PF_ATT_SUB) {
          A.tok0 = t0;
          enqueue_attn_long(c, A, std::min(PF_ATT_SUB, m - t0));
        }
      }
    }
    {
      PFQuantParams Q{p.attn, E, m, q8};
      hipLaunchKernelGGL(pf_quant_kernel(nb_k(E)), dim3(m_pad), dim3(256), 0, c->stream, Q);
    }
    pf_gemm(c, m, m_pad, nb_k(E), MODE_RESID, {&L.wo}, {p.X}, {nullptr}, {E}, p.attn, E, E);
    {
      PFNormParams N;
      memset(&N, 0, sizeof(N));
      N.n_x = E;
      N.eps = D.rms_eps;
      N.X = p.X;
      N.norm_w = L.ffn_norm;
      N.m = m;
      N.nb = nb_k(E);
      N.out = q8;
      N.xn = p.xn;
      hipLaunchKernelGGL(pf_norm_kernel(nb_k(E)), dim3(m_pad), dim3(256), norm_lds, c->stream, N);
    }
    pf_gemm(c, m, m_pad, nb_k(E), MODE_BIAS, {&L.wg, &L.wu}, {p.g, p.u}, {nullptr, nullptr}, {F, F}, p.xn, E, E);
    hipLaunchKernelGGL(k_pf_swiglu, dim3((F + 255) / 256, m), dim3(256), 0, c->stream, p.g, p.u, p.h, F, m);
    {
      PFQuantParams Q{p.h, F, m, q8};
      hipLaunchKernelGGL(pf_quant_kernel(nb_k(F)), dim3(m_pad), dim3(256), 0, c->stream, Q);
    }
    pf_gemm(c, m, m_pad, nb_k(F), MODE_RESID, {&L.wd}, {p.X}, {nullptr}, {E}, p.h, F, F);
  }
  // normX of the last token (engine/forward.go:135)
  NormParams N;
  memset(&N, 0, sizeof(N));
  N.x = p.X + (size_t)(m - 1) * E;
  N.w = c->output_norm;
  N.eps = D.rms_eps;
  N.n = E;
  N.out = c->normx[c->nx_cur ^ 1];
  N.n_lds = chain_lds_floats(E);
  hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(norm_threads(E)), (size_t)N.n_lds * sizeof(float), c->stream, N);
  HIPCHK(c, hipGetLastError());
  c->nx_prev = c->nx_cur;
  c->nx_cur ^= 1;
  return C2H_OK;
}

}  // namespace

int c2h_prefill(c2h_ctx* c, const int32_t* tokens, int32_t n, int32_t pos0, float* normx_out) {
  if (!c || (!tokens && n > 0) || n < 0) return C2H_ERR_INVALID;
  HIPCHK(c, hipSetDevice(c->device));
  int rc = validate_model(c);
  if (rc) return rc;
  if (pos0 < 0 || (int64_t)pos0 + n > c->desc.max_ctx)
    return fail(c, C2H_ERR_RANGE, "positions [%d, %d) outside [0, %d)", pos0, pos0 + n, c->desc.max_ctx);
  if (n == 0) return C2H_OK;
  if (c->desc.head_dim != 64) {
    // no batched prefill kernels at this head_dim: one forward graph per
    // token, as engine.IngestFrom runs Forward per token (c2slm.go:103-114)
    if ((rc = build_graphs(c))) return rc;
    for (int i = 0; i < n; ++i) {
      C2hState s;
      memset(&s, 0, sizeof(s));
      s.pos = pos0 + i;
      s.token = tokens[i];
      s.penalty = 1.15f;
      s.nx_in = c->nx_cur;
      s.nx_out = c->nx_cur ^ 1;
      if ((rc = push_state(c, s)) || (rc = run_graph(c, false, pos0 + i))) return rc;
      c->nx_prev = c->nx_cur;
      c->nx_cur ^= 1;
      c->seq_len = pos0 + i + 1;
    }
    HIPCHK(c, hipStreamSynchronize(c->stream));
  } else {
    if ((rc = pf_alloc(c)) || (rc = pf_q6_ready(c))) return rc;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    c->ring_next = 0;
    for (int done = 0; done < n;) {
      const int m = std::min(n - done, PF_MAX);
      if ((rc = pf_pass(c, tokens + done, m, pos0 + done))) return rc;
      HIPCHK(c, hipStreamSynchronize(c->stream));  // tokens are copied from the caller's buffer
      done += m;
      c->seq_len = pos0 + done;
    }
  }
  if (normx_out)
    HIPCHK(c, stream_copy(c->stream, normx_out, c->normx[c->nx_cur], (size_t)c->desc.n_embd * 4,
                          hipMemcpyDeviceToHost));
  return C2H_OK;
}

int c2h_logits(c2h_ctx* c, float* logits_out) {
  if (!c || !logits_out) return C2H_ERR_INVALID;
  if (!c->has_model) return fail(c, C2H_ERR_STATE, "kernel-only context");
  HIPCHK(c, hipSetDevice(c->device));
  int rc = validate_model(c);
  if (rc) return rc;
  C2hState s;
  memset(&s, 0, sizeof(s));
  s.penalty = 1.15f;
  s.nx_in = c->nx_cur;
  s.nx_out = c->nx_cur ^ 1;
  if ((rc = push_state(c, s))) return rc;
  enqueue_vocab(c, 0, c->logits, 1, nullptr);
  HIPCHK(c, hipGetLastError());
  HIPCHK(c, hipMemcpyAsync(logits_out, c->logits, (size_t)c->desc.n_vocab * 4, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return C2H_OK;
}

int c2h_step(c2h_ctx* c, int32_t pos, float penalty, int32_t im_end, int32_t eos, int32_t* next_token) {
  if (!c) return C2H_ERR_INVALID;
  HIPCHK(c, hipSetDevice(c->device));
  int rc = build_graphs(c);
  if (rc) return rc;
  if (pos < 0 || pos >= c->desc.max_ctx) return fail(c, C2H_ERR_RANGE, "pos %d outside [0, %d)", pos, c->desc.max_ctx);
  if ((rc = check_wait_flag(c))) return rc;  // a previous forward's
  C2hState s;
  memset(&s, 0, sizeof(s));
  s.pos = pos;
  s.token = 0;
  s.im_end = im_end;
  s.eos = eos;
  s.penalty = penalty;
  s.nx_in = c->nx_cur;
  s.nx_out = c->nx_cur ^ 1;
  s.seq = (int32_t)(++c->step_seq % 0x7ffffffeu) + 1;  // never 0 (other launches) or -1 (initial)
  // the state the previous step left on the device, when it is this one,
  // needs no copy (the token field is not read by a step graph)
  const C2hState& pr = c->state_pred;
  const bool same = c->state_pred_valid && pr.pos == s.pos && pr.im_end == s.im_end && pr.eos == s.eos &&
                    pr.penalty == s.penalty && pr.nx_in == s.nx_in && pr.nx_out == s.nx_out && pr.seq == s.seq;
  if (!same && (rc = push_state(c, s))) return rc;
  c->state_pred_valid = false;  // until the step's token has arrived
  if ((rc = run_graph(c, true, pos))) return rc;
  c->nx_prev = c->nx_cur;
  c->nx_cur ^= 1;
  c->seq_len = pos + 1;
  // The token is the argmax layer 0 takes at the start of the step: it
  // arrives in pinned memory (with s.seq) while the forward of that token
  // still runs, and everything that later reads the step's results is
  // ordered after it on the stream.  If the stream stops without it (an
  // error), the stream's status is reported and the device state is not
  // trusted by the next step (it copies the state again).
  const volatile int32_t* tk = c->tok_host;
  for (unsigned spin = 1;; ++spin) {
    if (__atomic_load_n(&tk[1], __ATOMIC_ACQUIRE) == s.seq) {
      if (next_token) *next_token = tk[0];
      // the state this step's final norm leaves on the device (eager
      // launches run the same final norm)
      c->state_pred = s;
      c->state_pred.pos = s.pos + 1;
      c->state_pred.seq = s.seq % 0x7ffffffe + 1;
      c->state_pred.nx_in = s.nx_out;
      c->state_pred.nx_out = s.nx_out ^ 1;
      c->state_pred_valid = true;
      return C2H_OK;
    }
    if ((spin & 1023u) == 0u) {
      const hipError_t q = hipStreamQuery(c->stream);
      if (q != hipErrorNotReady && __atomic_load_n(&tk[1], __ATOMIC_ACQUIRE) != s.seq) {
        HIPCHK(c, hipStreamSynchronize(c->stream));
        if (q != hipSuccess) return fail(c, C2H_ERR_HIP, "step: %s", hipGetErrorString(q));
        return fail(c, C2H_ERR_HIP, "step %d ended without handing over its token", s.seq);
      }
    }
  }
}

int c2h_restore_normx(c2h_ctx* c) {
  if (!c) return C2H_ERR_INVALID;
  c->nx_cur = c->nx_prev;
  return C2H_OK;
}

int c2h_get_normx(c2h_ctx* c, float* out) {
  if (!c || !out) return C2H_ERR_INVALID;
  if (!c->has_model) return fail(c, C2H_ERR_STATE, "kernel-only context");
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipMemcpyAsync(out, c->normx[c->nx_cur], (size_t)c->desc.n_embd * 4, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return C2H_OK;
}

int c2h_get_kv(c2h_ctx* c, int32_t which, int32_t layer, int32_t kv_head, int32_t n, float* out) {
  if (!c || (!out && n > 0)) return C2H_ERR_INVALID;
  int rc = check_kv_args(c, which, layer, kv_head, 0, n);
  if (rc) return rc;
  const c2h_model_desc& D = c->desc;
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if (n == 0) return C2H_OK;
  if (which == 1) return v_rows_copy(c, layer, kv_head, 0, n, out, false);
  HIPCHK(c, stream_copy(c->stream, out, c->kv + kv_slot_offset(D, 0, layer, kv_head), (size_t)n * D.head_dim * 4,
                      hipMemcpyDeviceToHost));
  return C2H_OK;
}

int c2h_set_kv(c2h_ctx* c, int32_t which, int32_t layer, int32_t kv_head, int32_t pos0, int32_t n, const float* src) {
  if (!c || (!src && n > 0)) return C2H_ERR_INVALID;
  int rc = check_kv_args(c, which, layer, kv_head, pos0, n);
  if (rc) return rc;
  const c2h_model_desc& D = c->desc;
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if (n == 0) return C2H_OK;
  if (which == 1) return v_rows_copy(c, layer, kv_head, pos0, n, const_cast<float*>(src), true);
  HIPCHK(c, stream_copy(c->stream, c->kv + kv_slot_offset(D, 0, layer, kv_head) + (size_t)pos0 * D.head_dim, src,
                      (size_t)n * D.head_dim * 4, hipMemcpyHostToDevice));
  return C2H_OK;
}

int c2h_get_token_ids(c2h_ctx* c, int32_t pos0, int32_t n, int32_t* out) {
  if (!c || (!out && n > 0)) return C2H_ERR_INVALID;
  if (!c->has_model) return fail(c, C2H_ERR_STATE, "kernel-only context");
  if (pos0 < 0 || n < 0 || (int64_t)pos0 + n > c->desc.max_ctx) return fail(c, C2H_ERR_RANGE, "token ids out of range");
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if (n) HIPCHK(c, stream_copy(c->stream, out, c->token_ids + pos0, (size_t)n * 4, hipMemcpyDeviceToHost));
  return C2H_OK;
}

int c2h_set_seq(c2h_ctx* c, int32_t seq_len) {
  if (!c) return C2H_ERR_INVALID;
  if (!c->has_model) return fail(c, C2H_ERR_STATE, "kernel-only context");
  if (seq_len < 0 || seq_len > c->desc.max_ctx)
    return fail(c, C2H_ERR_RANGE, "seq_len %d outside [0, %d]", seq_len, c->desc.max_ctx);
  c->seq_len = seq_len;
  return C2H_OK;
}

int c2h_get_seq(c2h_ctx* c, int32_t* seq_len) {
  if (!c || !seq_len) return C2H_ERR_INVALID;
  *seq_len = c->seq_len;
  return C2H_OK;
}

size_t c2h_packed_size(int32_t type, int64_t rows, int64_t cols) {
  size_t qb, db;
  packed_parts(type, rows, cols, &qb, &db);
  return qb + db;
}

int c2h_pack_weights(int32_t type, int64_t rows, int64_t cols, const void* native, size_t native_bytes, void* packed,
                     size_t packed_bytes) {
  if (!native || !packed) return C2H_ERR_INVALID;
  if (check_type_shape(nullptr, type, rows, cols)) return C2H_ERR_UNSUPPORTED;
  if (native_bytes < (size_t)rows * native_row_bytes(type, cols)) return C2H_ERR_INVALID;
  size_t qb, db;
  packed_parts(type, rows, cols, &qb, &db);
  if (packed_bytes < qb + db) return C2H_ERR_INVALID;
  uint8_t* p = reinterpret_cast<uint8_t*>(packed);
  pack_host(type, rows, cols, reinterpret_cast<const uint8_t*>(native), p, p + qb);
  return C2H_OK;
}

int c2h_quantize_q8k_dev(c2h_ctx* c, const float* x, int32_t cols, void* q8k_out) {
  if (!c || !x || !q8k_out || cols < 0) return C2H_ERR_INVALID;
  HIPCHK(c, hipSetDevice(c->device));
  int nb = cols / 256;
  if (nb == 0) return C2H_OK;
  if (reinterpret_cast<uintptr_t>(x) & 15) return fail(c, C2H_ERR_INVALID, "x must be 16-byte aligned");
  hipLaunchKernelGGL(k_quantize_q8k, dim3((nb + 3) / 4), dim3(256), 0, c->stream, x, nb,
                     reinterpret_cast<uint8_t*>(q8k_out));
  HIPCHK(c, hipGetLastError());
  return C2H_OK;
}

int c2h_gemv_dev(c2h_ctx* c, int32_t type, const void* w_packed, const void* xq, int32_t rows, int32_t cols, float* y,
                 int32_t* isums_out) {
  if (!c || !w_packed || !xq || !y) return C2H_ERR_INVALID;
  int rc = check_type_shape(c, type, rows, cols);
  if (rc) return rc;
  HIPCHK(c, hipSetDevice(c->device));
  size_t qb, db;
  packed_parts(type, rows, cols, &qb, &db);
  Tensor t;
  t.q = reinterpret_cast<uint8_t*>(const_cast<void*>(w_packed));
  t.d = db ? reinterpret_cast<uint16_t*>(t.q + qb) : nullptr;
  t.type = type;
  t.rows = rows;
  t.cols = cols;
  if (type == C2H_Q8_0 && nb8_of(cols) > 32) return fail(c, C2H_ERR_UNSUPPORTED, "Q8_0 rows run up to 1024 columns");
  if (type == C2H_Q5_0 || type == C2H_Q8_0) {  // f32 x: k_gemv_f without a prologue
    GemvParams P;
    memset(&P, 0, sizeof(P));
    P.prologue = PRO_QUANT;
    P.x = reinterpret_cast<const float*>(xq);
    P.n_x = nb8_of(cols) * 32;
    add_job(P, t, nullptr, MODE_STORE, y, nullptr, nullptr);
    launch_gemv_f(c, P);
    HIPCHK(c, hipGetLastError());
    return C2H_OK;
  }
  GemvParams P;
  memset(&P, 0, sizeof(P));
  P.prologue = PRO_Q8K;
  P.q8k_in = reinterpret_cast<const uint8_t*>(xq);
  P.nb_in = nb_k(cols);
  add_job(P, t, nullptr, MODE_STORE, y, nullptr, isums_out);
  hipLaunchKernelGGL(k_gemv_q8k, job_grid(P), dim3(256), gemv_q8k_lds_bytes(), c->stream, P);
  HIPCHK(c, hipGetLastError());
  return C2H_OK;
}

namespace {

bool float_x_type(int type) {
  return type == C2H_Q4_K || type == C2H_Q6_K || type == C2H_Q8_0 || type == C2H_Q5_0;
}

// Super-blocks (K-quants) or blocks (Q8_0 / Q5_0) per row: the reference's
// row functions floor cols to them, and zero of them gives zero dots.
int64_t float_x_blocks(int type, int64_t cols) {
  return (type == C2H_Q4_K || type == C2H_Q6_K) ? cols / 256 : cols / 32;
}

void launch_dot_rows(c2h_ctx* c, int type, WeightRef w, int rows, int cols, XSel X, const int32_t* ids, int n,
                     int scatter, float* y) {
  DotRowsParams P;
  memset(&P, 0, sizeof(P));
  P.w = w;
  P.rows = rows;
  P.cols = cols;
  P.X = X;
  P.ids = ids;
  P.n = n;
  P.scatter = scatter;
  P.y = y;
  const dim3 grid((n + DOT_ROWS_PER_WG - 1) / DOT_ROWS_PER_WG), block(256);
  const size_t lds = dot_rows_lds_bytes(type, cols);
  switch (type) {
    case C2H_Q4_K: hipLaunchKernelGGL(k_dot_rows<T_Q4_K>, grid, block, lds, c->stream, P); break;
    case C2H_Q6_K: hipLaunchKernelGGL(k_dot_rows<T_Q6_K>, grid, block, lds, c->stream, P); break;
    case C2H_Q8_0: hipLaunchKernelGGL(k_dot_rows<T_Q8_0>, grid, block, lds, c->stream, P); break;
    default: hipLaunchKernelGGL(k_dot_rows<T_Q5_0>, grid, block, lds, c->stream, P); break;
  }
}

// Shape checks of the float-x row dots, and (once per context) their LDS
// limit: x is staged whole, up to DOT_MAX_COLS floats.
int dot_rows_ready(c2h_ctx* c, int64_t cols) {
  if (cols > DOT_MAX_COLS) return fail(c, C2H_ERR_UNSUPPORTED, "float-x rows run up to %d columns", DOT_MAX_COLS);
  if (!c->dot_attr) {
    const void* ks[] = {(const void*)k_dot_rows<T_Q4_K>, (const void*)k_dot_rows<T_Q6_K>,
                        (const void*)k_dot_rows<T_Q8_0>, (const void*)k_dot_rows<T_Q5_0>};
    for (const void* k : ks)
      if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, DOT_MAX_COLS * 4) != hipSuccess)
        return fail(c, C2H_ERR_HIP, "row-dot LDS attribute");
    c->dot_attr = true;
  }
  return C2H_OK;
}

// Weight view of a c2h_pack_weights buffer.
WeightRef packed_ref(int type, int64_t rows, int64_t cols, const void* w_packed) {
  size_t qb, db;
  packed_parts(type, rows, cols, &qb, &db);
  WeightRef w;
  w.q = reinterpret_cast<const uint8_t*>(w_packed);
  w.d = db ? reinterpret_cast<const uint16_t*>(w.q + qb) : nullptr;
  return w;
}

}  // namespace

int c2h_gemv_f32_dev(c2h_ctx* c, int32_t type, const void* w_packed, const float* x, int32_t rows, int32_t cols,
                     float* y) {
  if (!c || !x || !y || rows <= 0 || cols <= 0) return C2H_ERR_INVALID;
  HIPCHK(c, hipSetDevice(c->device));
  if (!float_x_type(type) || float_x_blocks(type, cols) == 0) {  // DispatchGEMV's zero fallback / empty rows
    HIPCHK(c, hipMemsetAsync(y, 0, (size_t)rows * 4, c->stream));
    return C2H_OK;
  }
  if (!w_packed) return C2H_ERR_INVALID;
  if (reinterpret_cast<uintptr_t>(x) & 15) return fail(c, C2H_ERR_INVALID, "x must be 16-byte aligned");
  int rc = dot_rows_ready(c, cols);
  if (rc) return rc;
  launch_dot_rows(c, type, packed_ref(type, rows, cols, w_packed), rows, cols, plain_x(x), nullptr, rows, 0, y);
  HIPCHK(c, hipGetLastError());
  return C2H_OK;
}

int c2h_gemv_f32(c2h_ctx* c, int32_t type, const void* w, const float* x, int32_t rows, int32_t cols, float* y) {
  if (!c || !x || !y || rows <= 0 || cols <= 0) return C2H_ERR_INVALID;
  HIPCHK(c, hipSetDevice(c->device));
  if (!float_x_type(type) || float_x_blocks(type, cols) == 0) {
    memset(y, 0, (size_t)rows * 4);
    return C2H_OK;
  }
  if (!w) return C2H_ERR_INVALID;
  if (int rc0 = dot_rows_ready(c, cols)) return rc0;
  const size_t pbytes = c2h_packed_size(type, rows, cols);
  std::vector<uint8_t> packed(pbytes);
  size_t qb, db;
  packed_parts(type, rows, cols, &qb, &db);
  pack_host(type, rows, cols, reinterpret_cast<const uint8_t*>(w), packed.data(), packed.data() + qb);
  uint8_t* dw = nullptr;
  float *dx = nullptr, *dy = nullptr;
  auto cleanup = [&]() {
    if (dw) (void)hipFree(dw);
    if (dx) (void)hipFree(dx);
    if (dy) (void)hipFree(dy);
  };
  if (hipMalloc(&dw, pbytes) != hipSuccess || hipMalloc(&dx, (size_t)cols * 4) != hipSuccess ||
      hipMalloc(&dy, (size_t)rows * 4) != hipSuccess) {
    cleanup();
    return fail(c, C2H_ERR_HIP, "hipMalloc failed");
  }
  int rc = C2H_OK;
  if (stream_copy(c->stream, dw, packed.data(), pbytes, hipMemcpyHostToDevice) != hipSuccess ||
      stream_copy(c->stream, dx, x, (size_t)cols * 4, hipMemcpyHostToDevice) != hipSuccess)
    rc = fail(c, C2H_ERR_HIP, "copy in failed");
  if (!rc) rc = c2h_gemv_f32_dev(c, type, dw, dx, rows, cols, dy);
  if (!rc && hipStreamSynchronize(c->stream) != hipSuccess) rc = fail(c, C2H_ERR_HIP, "kernel failed");
  if (!rc && stream_copy(c->stream, y, dy, (size_t)rows * 4, hipMemcpyDeviceToHost) != hipSuccess)
    rc = fail(c, C2H_ERR_HIP, "copy out failed");
  cleanup();
  return rc;
}

int c2h_logits_ids_dev(c2h_ctx* c, const int32_t* ids, int32_t n_ids, float* logits) {
  if (!c || !logits || n_ids < 0 || (n_ids > 0 && !ids)) return C2H_ERR_INVALID;
  if (!c->has_model) return fail(c, C2H_ERR_STATE, "kernel-only context");
  HIPCHK(c, hipSetDevice(c->device));
  int rc = validate_model(c);
  if (rc) return rc;
  if (n_ids == 0) {  // an empty target list projects the whole vocabulary (engine/forward.go:174,185-190)
    enqueue_vocab(c, 0, logits, 0, c->normx[c->nx_cur]);
    HIPCHK(c, hipGetLastError());
    return C2H_OK;
  }
  const Tensor& t = out_weight(c);
  if ((rc = dot_rows_ready(c, t.cols))) return rc;
  launch_dot_rows(c, t.type, t.ref(), (int)t.rows, (int)t.cols, plain_x(c->normx[c->nx_cur]), ids, n_ids, 1, logits);
  HIPCHK(c, hipGetLastError());
  return C2H_OK;
}

int c2h_logits_ids(c2h_ctx* c, const int32_t* ids, int32_t n_ids, float* logits_out) {
  if (!c || !logits_out || n_ids < 0 || (n_ids > 0 && !ids)) return C2H_ERR_INVALID;
  if (n_ids == 0) return c2h_logits(c, logits_out);
  if (!c->has_model) return fail(c, C2H_ERR_STATE, "kernel-only context");
  HIPCHK(c, hipSetDevice(c->device));
  int rc = validate_model(c);
  if (rc) return rc;
  if (n_ids > c->ids_cap) {
    if (c->ids_dev) (void)hipFree(c->ids_dev);
    if (c->ids_y) (void)hipFree(c->ids_y);
    c->ids_dev = nullptr;
    c->ids_y = nullptr;
    c->ids_cap = 0;
    const int cap = n_ids < 1024 ? 1024 : n_ids;
    HIPCHK(c, hipMalloc(&c->ids_dev, (size_t)cap * 4));
    HIPCHK(c, hipMalloc(&c->ids_y, (size_t)cap * 4));
    c->ids_cap = cap;
  }
  HIPCHK(c, stream_copy(c->stream, c->ids_dev, ids, (size_t)n_ids * 4, hipMemcpyHostToDevice));
  const Tensor& t = out_weight(c);
  if ((rc = dot_rows_ready(c, t.cols))) return rc;
  launch_dot_rows(c, t.type, t.ref(), (int)t.rows, (int)t.cols, plain_x(c->normx[c->nx_cur]), c->ids_dev, n_ids, 0,
                  c->ids_y);
  HIPCHK(c, hipGetLastError());
  std::vector<float> y((size_t)n_ids);
  HIPCHK(c, stream_copy(c->stream, y.data(), c->ids_y, (size_t)n_ids * 4, hipMemcpyDeviceToHost));
  const int vocab = c->desc.n_vocab;
  for (int i = 0; i < n_ids; ++i)  // out-of-range ids are skipped (engine/forward.go:177-179)
    if (ids[i] >= 0 && ids[i] < vocab) logits_out[ids[i]] = y[(size_t)i];
  return C2H_OK;
}

int c2h_sync(c2h_ctx* c) {
  if (!c) return C2H_ERR_INVALID;
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return check_wait_flag(c);
}

int c2h_quantize_q8k(c2h_ctx* c, const float* x, int32_t cols, void* q8k_out) {
  if (!c || !x || !q8k_out || cols < 0) return C2H_ERR_INVALID;
  HIPCHK(c, hipSetDevice(c->device));
  int nb = cols / 256;
  if (nb == 0) return C2H_OK;
  float* dx = nullptr;
  uint8_t* dy = nullptr;
  HIPCHK(c, hipMalloc(&dx, (size_t)nb * 256 * 4));
  if (hipMalloc(&dy, (size_t)nb * BS_Q8K) != hipSuccess) {
    (void)hipFree(dx);
    return fail(c, C2H_ERR_HIP, "hipMalloc");
  }
  int rc = C2H_OK;
  if (stream_copy(c->stream, dx, x, (size_t)nb * 256 * 4, hipMemcpyHostToDevice) != hipSuccess) rc = C2H_ERR_HIP;
  if (!rc) rc = c2h_quantize_q8k_dev(c, dx, cols, dy);
  if (!rc && hipStreamSynchronize(c->stream) != hipSuccess) rc = C2H_ERR_HIP;
  if (!rc && stream_copy(c->stream, q8k_out, dy, (size_t)nb * BS_Q8K, hipMemcpyDeviceToHost) != hipSuccess)
    rc = C2H_ERR_HIP;
  (void)hipFree(dx);
  (void)hipFree(dy);
  if (rc == C2H_ERR_HIP) return fail(c, rc, "quantize copy failed");
  return rc;
}

int c2h_quantize_q8k_noalloc(c2h_ctx* c, const float* x, int32_t cols, void* q8k_out) {
  if (!c || !x || !q8k_out || cols < 0) return C2H_ERR_INVALID;
  if (cols > C2H_NOALLOC_MAX_COLS)
    return fail(c, C2H_ERR_INVALID, "%d columns exceed the no-alloc scratch (%d)", cols, C2H_NOALLOC_MAX_COLS);
  HIPCHK(c, hipSetDevice(c->device));
  const int nb = cols / 256;
  if (nb == 0) return C2H_OK;
  if (!c->noalloc) return fail(c, C2H_ERR_STATE, "no-alloc scratch not set up");
  float* dx = reinterpret_cast<float*>(c->noalloc);
  uint8_t* dy = c->noalloc + kNoAllocX;
  // One call at a time per GPU in this process, from the copy in to the
  // copy out: every context on the GPU shares its scratch.  Every byte the
  // kernel writes is rewritten, nothing needs clearing.
  std::lock_guard<std::mutex> lock(g_noalloc_call_mu[c->device]);
  HIPCHK(c, hipMemcpyAsync(dx, x, (size_t)nb * 256 * 4, hipMemcpyHostToDevice, c->stream));
  hipLaunchKernelGGL(k_quantize_q8k, dim3((nb + 3) / 4), dim3(256), 0, c->stream, dx, nb, dy);
  HIPCHK(c, hipGetLastError());
  HIPCHK(c, hipMemcpyAsync(q8k_out, dy, (size_t)nb * BS_Q8K, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return C2H_OK;
}

int c2h_gemv(c2h_ctx* c, int32_t type, const void* w, const void* xq, int32_t rows, int32_t cols, float* y,
             int32_t* isums_out) {
  if (!c || !w || !xq || !y) return C2H_ERR_INVALID;
  int rc = check_type_shape(c, type, rows, cols);
  if (rc) return rc;
  HIPCHK(c, hipSetDevice(c->device));
  size_t nbytes = (size_t)rows * native_row_bytes(type, cols);
  size_t pbytes = c2h_packed_size(type, rows, cols);
  std::vector<uint8_t> packed(pbytes);
  size_t qb, db;
  packed_parts(type, rows, cols, &qb, &db);
  pack_host(type, rows, cols, reinterpret_cast<const uint8_t*>(w), packed.data(), packed.data() + qb);
  (void)nbytes;
  size_t xbytes = (type == C2H_Q8_0 || type == C2H_Q5_0) ? (size_t)cols * 4 : (size_t)nb_k(cols) * BS_Q8K;
  size_t isz = 0;
  if (isums_out && type == C2H_Q4_K) isz = (size_t)rows * nb_k(cols) * 8 * 4;
  if (isums_out && type == C2H_Q6_K) isz = (size_t)rows * nb_k(cols) * 4;
  uint8_t *dw = nullptr, *dx = nullptr;
  float* dy = nullptr;
  int32_t* di = nullptr;
  auto cleanup = [&]() {
    if (dw) (void)hipFree(dw);
    if (dx) (void)hipFree(dx);
    if (dy) (void)hipFree(dy);
    if (di) (void)hipFree(di);
  };
  if (hipMalloc(&dw, pbytes) != hipSuccess || hipMalloc(&dx, xbytes) != hipSuccess ||
      hipMalloc(&dy, (size_t)rows * 4) != hipSuccess || (isz && hipMalloc(&di, isz) != hipSuccess)) {
    cleanup();
    return fail(c, C2H_ERR_HIP, "hipMalloc failed");
  }
  rc = C2H_OK;
  if (stream_copy(c->stream, dw, packed.data(), pbytes, hipMemcpyHostToDevice) != hipSuccess ||
      stream_copy(c->stream, dx, xq, xbytes, hipMemcpyHostToDevice) != hipSuccess)
    rc = fail(c, C2H_ERR_HIP, "copy in failed");
  if (!rc) rc = c2h_gemv_dev(c, type, dw, dx, rows, cols, dy, di);
  if (!rc && c2h_sync(c)) rc = C2H_ERR_HIP;
  if (!rc && stream_copy(c->stream, y, dy, (size_t)rows * 4, hipMemcpyDeviceToHost) != hipSuccess)
    rc = fail(c, C2H_ERR_HIP, "copy out failed");
  if (!rc && isz && stream_copy(c->stream, isums_out, di, isz, hipMemcpyDeviceToHost) != hipSuccess)
    rc = fail(c, C2H_ERR_HIP, "copy out failed");
  cleanup();
  return rc;
}

int c2h_copy_bench(c2h_ctx* c, int64_t bytes, int32_t reps, float* ms) {
  if (!c || !ms || bytes <= 0 || (bytes & 15) || reps <= 0) return C2H_ERR_INVALID;
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  void *src = nullptr, *dst = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = C2H_OK;
  float t = 0;
  if (hipMalloc(&src, (size_t)bytes) != hipSuccess || hipMalloc(&dst, (size_t)bytes) != hipSuccess ||
      hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    rc = fail(c, C2H_ERR_HIP, "copy bench: allocation failed");
  } else {
    const size_t n16 = (size_t)bytes / 16;
    (void)hipMemsetAsync(src, 1, (size_t)bytes, c->stream);
    (void)hipEventRecord(e0, c->stream);
    for (int i = 0; i < reps; ++i)
      hipLaunchKernelGGL(k_copy16, dim3(8192), dim3(256), 0, c->stream, (const uint4*)src, (uint4*)dst, n16);
    (void)hipEventRecord(e1, c->stream);
    hipError_t e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(&t, e0, e1);
    if (e != hipSuccess) rc = fail(c, C2H_ERR_HIP, "copy bench: %s", hipGetErrorString(e));
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (src) (void)hipFree(src);
  if (dst) (void)hipFree(dst);
  if (rc) return rc;
  *ms = t / reps;
  return C2H_OK;
}

int c2h_check_rms_scale(c2h_ctx* c, uint32_t lo, uint64_t hi, uint64_t* mismatches, uint32_t* first_bits) {
  if (!c || !mismatches || !first_bits || hi > (1ull << 32) || hi < lo) return C2H_ERR_INVALID;
  HIPCHK(c, hipSetDevice(c->device));
  unsigned long long* bad = nullptr;
  hipError_t e = hipMalloc(&bad, 16);
  uint32_t* first = reinterpret_cast<uint32_t*>(bad + 1);
  if (e == hipSuccess) e = hipMemsetAsync(bad, 0, 8, c->stream);
  if (e == hipSuccess) e = hipMemsetAsync(first, 0xff, 4, c->stream);
  constexpr uint64_t kChunk = 1ull << 28;  // patterns per launch (2^20 workgroups)
  for (uint64_t b = lo; e == hipSuccess && b < hi; b += kChunk) {
    const uint32_t n = (uint32_t)std::min<uint64_t>(kChunk, hi - b);
    hipLaunchKernelGGL(k_check_rms_scale, dim3((n + 255) / 256), dim3(256), 0, c->stream, (uint32_t)b, n, bad, first);
    e = hipGetLastError();
  }
  unsigned long long nb = 0;
  uint32_t fb = 0;
  if (e == hipSuccess) e = hipMemcpyAsync(&nb, bad, 8, hipMemcpyDeviceToHost, c->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(&fb, first, 4, hipMemcpyDeviceToHost, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (bad) (void)hipFree(bad);
  if (e != hipSuccess) return fail(c, C2H_ERR_HIP, "rms scale check: %s", hipGetErrorString(e));
  *mismatches = nb;
  *first_bits = fb;
  return C2H_OK;
}

int c2h_launch_floor(c2h_ctx* c, int32_t n, int32_t grid, int32_t reps, float* us) {
  if (!c || !us || n <= 0 || n > 4096 || grid <= 0 || grid > 65536 || reps <= 0) return C2H_ERR_INVALID;
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  int* flag = nullptr;
  hipGraph_t g = nullptr;
  hipGraphExec_t ge = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  float best = 0.0f;
  hipError_t e = hipMalloc(&flag, 16);
  if (e == hipSuccess) e = hipMemsetAsync(flag, 0, 16, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e == hipSuccess) e = hipEventCreate(&e0);
  if (e == hipSuccess) e = hipEventCreate(&e1);
  if (e == hipSuccess) e = hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal);
  if (e == hipSuccess) {
    for (int i = 0; i < n; ++i) hipLaunchKernelGGL(k_empty, dim3(grid), dim3(256), 0, c->stream, flag, flag + 1);
    e = hipStreamEndCapture(c->stream, &g);
  }
  if (e == hipSuccess) e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
  for (int r = 0; e == hipSuccess && r < reps + 2; ++r) {  // two untimed replays first
    float ms = 0.0f;
    e = hipEventRecord(e0, c->stream);
    if (e == hipSuccess) e = hipGraphLaunch(ge, c->stream);
    if (e == hipSuccess) e = hipEventRecord(e1, c->stream);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    if (e == hipSuccess && r >= 2 && (r == 2 || ms < best)) best = ms;
  }
  if (ge) (void)hipGraphExecDestroy(ge);
  if (g) (void)hipGraphDestroy(g);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (flag) (void)hipFree(flag);
  if (e != hipSuccess) return fail(c, C2H_ERR_HIP, "launch floor: %s", hipGetErrorString(e));
  *us = best * 1000.0f / n;
  return C2H_OK;
}

int c2h_time_producer_consumer(c2h_ctx* c, int32_t n_prod, int32_t n_cons, int32_t work, int32_t n_launch,
                               int32_t reps, int32_t proto, float* us_fused, float* us_split) {
  if (!c || !us_fused || !us_split || n_prod <= 0 || n_prod > 4096 || n_cons <= 0 || n_cons > 4096 || work < 0 ||
      work > 100000 || n_launch <= 0 || n_launch > 256 || reps <= 0 || proto < 0 || proto > 1)
    return C2H_ERR_INVALID;
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  constexpr int kData = 896;  // k_pc_bench polls up to 8 x 256 outputs per thread set
  unsigned* counters = nullptr;
  uint64_t* data_ll = nullptr;
  float *data = nullptr, *out = nullptr;
  uint4* weights = nullptr;
  int* err = nullptr;
  hipGraph_t g[2] = {nullptr, nullptr};
  hipGraphExec_t ge[2] = {nullptr, nullptr};
  hipEvent_t e0 = nullptr, e1 = nullptr;
  float best[2] = {0.0f, 0.0f};
  int herr[2] = {0, 0};
  const size_t wbytes = (size_t)n_launch * n_cons * 4 * 256 * sizeof(uint4);
  hipError_t e = hipMalloc(&counters, 8 * 64 * sizeof(unsigned));
  if (e == hipSuccess) e = hipMalloc(&data, kData * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&out, (size_t)n_cons * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&weights, wbytes);
  if (e == hipSuccess) e = hipMalloc(&err, 2 * sizeof(int));
  if (e == hipSuccess) e = hipMalloc(&data_ll, kData * sizeof(uint64_t));
  if (e == hipSuccess) e = hipMemsetAsync(weights, 0x5a, wbytes, c->stream);
  if (e == hipSuccess) e = hipMemsetAsync(err, 0, 2 * sizeof(int), c->stream);
  if (e == hipSuccess) e = hipEventCreate(&e0);
  if (e == hipSuccess) e = hipEventCreate(&e1);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  PcBenchParams P;
  memset(&P, 0, sizeof(P));
  P.counters = counters;
  P.data = data;
  P.weights = weights;
  P.out = out;
  P.err = err;
  P.n_prod = n_prod;
  P.n_cons = n_cons;
  P.spin_limit = 1 << 20;  // polls of >= ~0.5 us each: every wait ends within about a second
  P.data_floats = kData;
  P.work = work;
  P.proto = proto;
  P.data_ll = data_ll;
  // graph 0: the counters (and the tagged outputs' epochs) cleared by a
  // kernel, then n_launch fused launches
  // (epoch i+1: the counters' sum a launch's consumers wait for); graph 1:
  // the same work as a producer launch and a consumer launch per step
  for (int which = 0; which < 2 && e == hipSuccess; ++which) {
    e = hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) break;
    if (which == 0) {
      hipLaunchKernelGGL(k_fill_u32, dim3(2), dim3(256), 0, c->stream, counters, 8 * 64, 0u);
      hipLaunchKernelGGL(k_fill_u32, dim3(8), dim3(256), 0, c->stream, reinterpret_cast<unsigned*>(data_ll),
                         2 * kData, 0u);
    }
    for (int i = 0; i < n_launch; ++i) {
      P.epoch = i + 1;
      P.w_index = i;
      if (which == 0) {
        P.mode = 0;
        hipLaunchKernelGGL(k_pc_bench, dim3(n_prod + n_cons), dim3(256), 0, c->stream, P);
      } else {
        P.mode = 1;
        hipLaunchKernelGGL(k_pc_bench, dim3(n_prod), dim3(256), 0, c->stream, P);
        P.mode = 2;
        hipLaunchKernelGGL(k_pc_bench, dim3(n_cons), dim3(256), 0, c->stream, P);
      }
    }
    e = hipStreamEndCapture(c->stream, &g[which]);
    if (e == hipSuccess) e = hipGraphInstantiate(&ge[which], g[which], nullptr, nullptr, 0);
  }
  for (int r = 0; e == hipSuccess && r < reps + 1; ++r) {  // one untimed replay of each first
    for (int which = 0; which < 2 && e == hipSuccess; ++which) {
      float ms = 0.0f;
      e = hipEventRecord(e0, c->stream);
      if (e == hipSuccess) e = hipGraphLaunch(ge[which], c->stream);
      if (e == hipSuccess) e = hipEventRecord(e1, c->stream);
      if (e == hipSuccess) e = hipEventSynchronize(e1);
      if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
      if (e == hipSuccess && r >= 1 && (r == 1 || ms < best[which])) best[which] = ms;
    }
  }
  if (e == hipSuccess) e = hipMemcpy(herr, err, sizeof(herr), hipMemcpyDeviceToHost);
  for (int i = 0; i < 2; ++i) {
    if (ge[i]) (void)hipGraphExecDestroy(ge[i]);
    if (g[i]) (void)hipGraphDestroy(g[i]);
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  for (void* p : {(void*)counters, (void*)data, (void*)out, (void*)weights, (void*)err, (void*)data_ll})
    if (p) (void)hipFree(p);
  if (e != hipSuccess) return fail(c, C2H_ERR_HIP, "producer/consumer timing: %s", hipGetErrorString(e));
  if (herr[0]) return fail(c, C2H_ERR_HIP, "producer/consumer timing: a consumer's wait ran out");
  if (herr[1]) return fail(c, C2H_ERR_HIP, "producer/consumer timing: %d outputs read stale", herr[1]);
  *us_fused = best[0] * 1000.0f / n_launch;
  *us_split = best[1] * 1000.0f / n_launch;
  return C2H_OK;
}

int c2h_time_vocab(c2h_ctx* c, int32_t iters, int32_t pos, int32_t in_step, float* ms) {
  if (!c || !ms || iters <= 0 || iters > 4096) return C2H_ERR_INVALID;
  HIPCHK(c, hipSetDevice(c->device));
  int rc = build_graphs(c);
  if (rc) return rc;
  if (pos < 0 || pos >= c->desc.max_ctx) return fail(c, C2H_ERR_RANGE, "pos out of range");
  HIPCHK(c, hipStreamSynchronize(c->stream));
  c->ring_next = 0;
  C2hState s;
  memset(&s, 0, sizeof(s));
  s.pos = pos;
  s.penalty = 1.15f;
  s.im_end = -1;
  s.eos = -1;
  s.nx_in = c->nx_cur;
  s.nx_out = c->nx_cur ^ 1;
  if ((rc = push_state(c, s))) return rc;
  enqueue_vocab(c, 1, nullptr, 1, nullptr);  // warm-up
  if (in_step == 2) {
    // launches back to back, alternating between the matrix and a copy of
    // it: a working set of twice the matrix, above the last-level cache, so
    // each launch streams its rows from HBM; one pair of events around all
    const Tensor& ow = out_weight(c);
    if (ow.type != C2H_Q8_0) return fail(c, C2H_ERR_UNSUPPORTED, "alternating timing needs the Q8_0 vocab kernel");
    const size_t bytes = (size_t)ow.rows * q8_0_row_stride(nb8_of(ow.cols));
    uint8_t* cp = nullptr;
    HIPCHK(c, hipMalloc(&cp, bytes));
    hipEvent_t e0 = nullptr, e1 = nullptr;
    rc = C2H_OK;
    if (hipMemcpyAsync(cp, ow.q, bytes, hipMemcpyDeviceToDevice, c->stream) != hipSuccess ||
        hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
      rc = fail(c, C2H_ERR_HIP, "vocab copy");
    if (rc == C2H_OK) {
      enqueue_vocab(c, 1, nullptr, 1, nullptr, cp);  // warm-up of the copy's launch
      (void)hipEventRecord(e0, c->stream);
      for (int i = 0; i < iters; ++i) enqueue_vocab(c, 1, nullptr, 1, nullptr, (i & 1) ? cp : nullptr);
      (void)hipEventRecord(e1, c->stream);
      float t = 0;
      if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&t, e0, e1) != hipSuccess)
        rc = fail(c, C2H_ERR_HIP, "vocab timing");
      else
        *ms = t / iters;
    }
    (void)hipStreamSynchronize(c->stream);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipFree(cp);
    return rc;
  }
  std::vector<hipEvent_t> ev(2 * (size_t)iters, nullptr);
  for (auto& e : ev) HIPCHK(c, hipEventCreate(&e));
  rc = C2H_OK;
  for (int i = 0; i < iters && rc == C2H_OK; ++i) {
    if (in_step) rc = run_graph(c, false, pos);
    if (rc == C2H_OK) {
      (void)hipEventRecord(ev[2 * i], c->stream);
      enqueue_vocab(c, 1, nullptr, 1, nullptr);
      (void)hipEventRecord(ev[2 * i + 1], c->stream);
    }
  }
  double total = 0;
  if (rc == C2H_OK) {
    hipError_t e = hipEventSynchronize(ev.back());
    for (int i = 0; i < iters && e == hipSuccess; ++i) {
      float t = 0;
      e = hipEventElapsedTime(&t, ev[2 * i], ev[2 * i + 1]);
      total += t;
    }
    if (e != hipSuccess) rc = fail(c, C2H_ERR_HIP, "vocab timing: %s", hipGetErrorString(e));
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  if (rc) return rc;
  *ms = (float)(total / iters);
  return C2H_OK;
}

int c2h_time_dot_rows(c2h_ctx* c, int32_t type, const void* w, const float* x, int32_t rows, int32_t cols,
                      const int32_t* ids, int32_t n, int32_t iters, int64_t flush_bytes, float* y_out, float* ms) {
  if (!c || !w || !x || !ms || rows <= 0 || cols <= 0 || n <= 0 || iters <= 0 || iters > 4096 || flush_bytes < 0)
    return C2H_ERR_INVALID;
  if (!float_x_type(type) || float_x_blocks(type, cols) == 0) return fail(c, C2H_ERR_UNSUPPORTED, "no float row dot");
  if (!ids && n > rows) return fail(c, C2H_ERR_INVALID, "n > rows without ids");
  HIPCHK(c, hipSetDevice(c->device));
  if (int rc0 = dot_rows_ready(c, cols)) return rc0;
  const size_t pbytes = c2h_packed_size(type, rows, cols), n16 = (size_t)flush_bytes / 16;
  std::vector<uint8_t> packed(pbytes);
  size_t qb, db;
  packed_parts(type, rows, cols, &qb, &db);
  pack_host(type, rows, cols, reinterpret_cast<const uint8_t*>(w), packed.data(), packed.data() + qb);
  uint8_t* dw = nullptr;
  float *dx = nullptr, *dy = nullptr;
  int32_t* di = nullptr;
  uint4* fl = nullptr;
  std::vector<hipEvent_t> ev(2 * (size_t)iters, nullptr);
  auto cleanup = [&]() {
    (void)hipStreamSynchronize(c->stream);
    for (auto& e : ev)
      if (e) (void)hipEventDestroy(e);
    for (void* p : {(void*)dw, (void*)dx, (void*)dy, (void*)di, (void*)fl})
      if (p) (void)hipFree(p);
  };
  int rc = C2H_OK;
  if (hipMalloc(&dw, pbytes) != hipSuccess || hipMalloc(&dx, (size_t)cols * 4) != hipSuccess ||
      hipMalloc(&dy, (size_t)n * 4) != hipSuccess || (ids && hipMalloc(&di, (size_t)n * 4) != hipSuccess) ||
      (n16 && hipMalloc(&fl, 2 * n16 * 16) != hipSuccess))
    rc = fail(c, C2H_ERR_HIP, "hipMalloc failed");
  if (!rc && (stream_copy(c->stream, dw, packed.data(), pbytes, hipMemcpyHostToDevice) != hipSuccess ||
              stream_copy(c->stream, dx, x, (size_t)cols * 4, hipMemcpyHostToDevice) != hipSuccess ||
              (ids && stream_copy(c->stream, di, ids, (size_t)n * 4, hipMemcpyHostToDevice) != hipSuccess)))
    rc = fail(c, C2H_ERR_HIP, "copy in failed");
  for (auto& e : ev)
    if (!rc && hipEventCreate(&e) != hipSuccess) rc = fail(c, C2H_ERR_HIP, "hipEventCreate");
  const WeightRef wr = packed_ref(type, rows, cols, dw);
  if (!rc) launch_dot_rows(c, type, wr, rows, cols, plain_x(dx), di, n, 0, dy);  // warm-up
  for (int i = 0; i < iters && rc == C2H_OK; ++i) {
    // copying flush_bytes (2x that touched) between launches evicts the matrix from the last-level cache
    if (n16) hipLaunchKernelGGL(k_copy16, dim3(1024), dim3(256), 0, c->stream, fl, fl + n16, n16);
    (void)hipEventRecord(ev[2 * i], c->stream);
    launch_dot_rows(c, type, wr, rows, cols, plain_x(dx), di, n, 0, dy);
    (void)hipEventRecord(ev[2 * i + 1], c->stream);
  }
  if (!rc && hipGetLastError() != hipSuccess) rc = fail(c, C2H_ERR_HIP, "launch failed");
  double total = 0;
  if (!rc) {
    hipError_t e = hipEventSynchronize(ev.back());
    for (int i = 0; i < iters && e == hipSuccess; ++i) {
      float t = 0;
      e = hipEventElapsedTime(&t, ev[2 * i], ev[2 * i + 1]);
      total += t;
    }
    if (e != hipSuccess) rc = fail(c, C2H_ERR_HIP, "dot timing: %s", hipGetErrorString(e));
  }
  if (!rc && y_out && stream_copy(c->stream, y_out, dy, (size_t)n * 4, hipMemcpyDeviceToHost) != hipSuccess)
    rc = fail(c, C2H_ERR_HIP, "copy out failed");
  cleanup();
  if (rc) return rc;
  *ms = (float)(total / iters);
  return C2H_OK;
}

int c2h_time_steps(c2h_ctx* c, int32_t pos, int32_t iters, float penalty, int32_t im_end, int32_t eos, float* ms) {
  if (!c || !ms || iters <= 0) return C2H_ERR_INVALID;
  HIPCHK(c, hipSetDevice(c->device));
  int rc = build_graphs(c);
  if (rc) return rc;
  if (pos < 0 || pos + iters > c->desc.max_ctx) return fail(c, C2H_ERR_RANGE, "positions out of range");
  HIPCHK(c, hipStreamSynchronize(c->stream));
  c->ring_next = 0;  // all earlier state copies have completed
  hipEvent_t e0, e1;
  HIPCHK(c, hipEventCreate(&e0));
  HIPCHK(c, hipEventCreate(&e1));
  HIPCHK(c, hipEventRecord(e0, c->stream));
  for (int i = 0; i < iters; ++i) {
    if (i == 0) {  // later steps run on the state the previous step's final norm advanced
      C2hState s;
      memset(&s, 0, sizeof(s));
      s.pos = pos;
      s.im_end = im_end;
      s.eos = eos;
      s.penalty = penalty;
      s.nx_in = c->nx_cur;
      s.nx_out = c->nx_cur ^ 1;
      // step numbers come from the context's counter, as c2h_step's do: the
      // graphs publish seq .. seq+iters-1 to the token slot c2h_step polls,
      // and the counter moves past them so the next c2h_step's number is new
      s.seq = (int32_t)(++c->step_seq % 0x7ffffffeu) + 1;
      c->step_seq += (unsigned)(iters - 1);
      if ((rc = push_state(c, s))) return rc;
    }
    if ((rc = run_graph(c, true, pos + i))) return rc;
    c->nx_prev = c->nx_cur;
    c->nx_cur ^= 1;
  }
  c->seq_len = pos + iters;
  HIPCHK(c, hipEventRecord(e1, c->stream));
  HIPCHK(c, hipEventSynchronize(e1));
  float t = 0;
  HIPCHK(c, hipEventElapsedTime(&t, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *ms = t / iters;
  return C2H_OK;
}


int c2h_time_layer_kernel(c2h_ctx* c, int32_t kernel, int32_t iters, int32_t captured, float* ms) {
  if (!c || !ms || iters <= 0 || iters > 100000 || kernel < 0 || kernel > C2H_KERNEL_FFN_BLOCK) return C2H_ERR_INVALID;
  HIPCHK(c, hipSetDevice(c->device));
  int rc = build_graphs(c);
  if (rc) return rc;
  const c2h_model_desc& D = c->desc;
  // the attention kernel stores K/V at pos: only a position past the cached
  // rows may be written (a timing call must not change what a caller reads)
  if (c->seq_len >= D.max_ctx)
    return fail(c, C2H_ERR_RANGE, "SeqLen %d leaves no free position below max_ctx %d", c->seq_len, D.max_ctx);
  const int pos = c->seq_len;
  HIPCHK(c, hipStreamSynchronize(c->stream));
  c->ring_next = 0;
  C2hState s;
  memset(&s, 0, sizeof(s));
  s.pos = pos;
  s.penalty = 1.15f;
  s.im_end = -1;
  s.eos = -1;
  s.nx_in = c->nx_cur;
  s.nx_out = c->nx_cur ^ 1;
  if ((rc = push_state(c, s))) return rc;
  const int form = attn_form(c, pos + 1);
  // the timing runs a fused launch on every layer: every layer's tensors
  // must be of the types that launch reads (a file may mix them by layer)
  if (kernel == C2H_KERNEL_ATTN_BLOCK || kernel == C2H_KERNEL_ATTN_OPROJ || kernel == C2H_KERNEL_FFN_BLOCK) {
    bool ok = D.n_layers > 1;
    for (int l = 0; ok && l < D.n_layers; ++l) {
      const Layer& L = c->layers[l];
      if (kernel == C2H_KERNEL_FFN_BLOCK)
        ok = c->fuse_ffn && ffn_block_types(c, l);
      else
        ok = fuse_attn_oproj(c, l, form) &&
             (kernel == C2H_KERNEL_ATTN_OPROJ || (c->fuse_qkv && !float_input(L.wq.type) &&
                                                  !float_input(L.wk.type) && !float_input(L.wv.type)));
    }
    if (!ok) return fail(c, C2H_ERR_UNSUPPORTED, "no fused launch of this kind for every layer at this position");
  }
  // the residual kernels update X and the final norm writes normX[nx_out]:
  // both are restored afterwards
  float* saved = nullptr;
  HIPCHK(c, hipMalloc(&saved, (size_t)D.n_embd * 8));
  float* const nx_out = c->normx[s.nx_out];
  hipEvent_t e0 = nullptr, e1 = nullptr;
  auto one = [&](int i) {
    const int l = i % D.n_layers;
    switch (kernel) {
      case C2H_KERNEL_QKV: enqueue_qkv(c, l, PRO_NORM); break;
      case C2H_KERNEL_ATTN: enqueue_attn(c, l, form); break;
      case C2H_KERNEL_ATTN_OUT: enqueue_attn_out(c, l); break;
      case C2H_KERNEL_FFN_IN: enqueue_ffn_in(c, l); break;
      case C2H_KERNEL_FFN_OUT: enqueue_ffn_out(c, l); break;
      case C2H_KERNEL_ATTN_BLOCK: enqueue_attn_block(c, l, form, l > 0 && defer_ffn(c, l - 1, form)); break;
      case C2H_KERNEL_ATTN_OPROJ: enqueue_attn_oproj(c, l, form); break;
      case C2H_KERNEL_FFN_BLOCK: enqueue_ffn_block(c, l); break;
      default: enqueue_final_norm(c); break;
    }
  };
  if (hipMemcpyAsync(saved, c->X, (size_t)D.n_embd * 4, hipMemcpyDeviceToDevice, c->stream) != hipSuccess ||
      hipMemcpyAsync(saved + D.n_embd, nx_out, (size_t)D.n_embd * 4, hipMemcpyDeviceToDevice, c->stream) !=
          hipSuccess ||
      hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
    rc = fail(c, C2H_ERR_HIP, "kernel timing set-up failed");
  float t = 0.0f;
  hipGraph_t g = nullptr;
  hipGraphExec_t ge = nullptr;
  if (!rc) {
    // eager: the GPU first waits 60 us per launch to come (several times
    // the host's enqueue time of a launch, also under a kernel-trace
    // profiler), so the warm-up and the timed launches run back to back,
    // paced by the GPU rather than by the host's enqueue rate
    const bool eager = !(captured && c->use_graphs);
    if (eager)
      hipLaunchKernelGGL(k_delay, dim3(1), dim3(64), 0, c->stream,
                         std::min<long long>(C2H_DELAY_MAX_TICKS, 6000ll * (iters + D.n_layers)));
    for (int i = 0; i < D.n_layers; ++i) one(i);  // warm-up: every layer once
    // captured: the timed launches replay as one graph (as the decode step
    // does), so the host's launch rate does not pace them; eager when the
    // context runs without graphs (C2H_NO_GRAPH=1)
    hipError_t e = hipSuccess;
    if (!eager) {
      e = hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal);
      if (e == hipSuccess) {
        for (int i = 0; i < iters; ++i) one(i);
        e = hipStreamEndCapture(c->stream, &g);
      }
      if (e == hipSuccess) e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
      if (e == hipSuccess) e = hipGraphLaunch(ge, c->stream);  // warm-up replay
    }
    if (e == hipSuccess) e = hipEventRecord(e0, c->stream);
    if (e == hipSuccess) {
      if (ge)
        e = hipGraphLaunch(ge, c->stream);
      else
        for (int i = 0; i < iters; ++i) one(i);
    }
    if (e == hipSuccess) e = hipEventRecord(e1, c->stream);
    if (e == hipSuccess) e = hipGetLastError();
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(&t, e0, e1);
    if (e != hipSuccess) rc = fail(c, C2H_ERR_HIP, "kernel timing failed: %s", hipGetErrorString(e));
  }
  if (ge) (void)hipGraphExecDestroy(ge);
  if (g) (void)hipGraphDestroy(g);
  // the fused launches above left tags of the current epoch (launch i over
  // layer i mod n_layers, so consecutive launches' tags differ): the next
  // forward's launch of the last timed layer must not take them for its own
  if (!rc) {
    hipLaunchKernelGGL(k_next_epoch, dim3(1), dim3(64), 0, c->stream, c->state_dev);
    if (hipGetLastError() != hipSuccess) rc = fail(c, C2H_ERR_HIP, "advancing the epoch failed");
  }
  if (!rc && (hipMemcpyAsync(c->X, saved, (size_t)D.n_embd * 4, hipMemcpyDeviceToDevice, c->stream) != hipSuccess ||
              hipMemcpyAsync(nx_out, saved + D.n_embd, (size_t)D.n_embd * 4, hipMemcpyDeviceToDevice, c->stream) !=
                  hipSuccess))
    rc = fail(c, C2H_ERR_HIP, "restoring X / normX failed");
  (void)hipStreamSynchronize(c->stream);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  (void)hipFree(saved);
  if (rc) return rc;
  *ms = t / iters;
  return C2H_OK;
}

int c2h_time_gemv(c2h_ctx* c, int32_t type, const void* w, const void* xq, int32_t rows, int32_t cols, int32_t iters,
                  int64_t rotate_bytes, float* ms) {
  if (!c || !w || !xq || !ms || iters <= 0 || iters > 100000 || rotate_bytes < 0) return C2H_ERR_INVALID;
  int rc = check_type_shape(c, type, rows, cols);
  if (rc) return rc;
  if (type == C2H_Q8_0 && nb8_of(cols) > 32) return fail(c, C2H_ERR_UNSUPPORTED, "Q8_0 rows run up to 1024 columns");
  HIPCHK(c, hipSetDevice(c->device));
  const size_t pbytes = c2h_packed_size(type, rows, cols);
  const int64_t ncopy = std::min<int64_t>(65536, std::max<int64_t>(1, (rotate_bytes + (int64_t)pbytes - 1) / (int64_t)pbytes));
  std::vector<uint8_t> packed(pbytes);
  size_t qb, db;
  packed_parts(type, rows, cols, &qb, &db);
  pack_host(type, rows, cols, reinterpret_cast<const uint8_t*>(w), packed.data(), packed.data() + qb);
  const bool fx = (type == C2H_Q8_0 || type == C2H_Q5_0);
  const size_t xbytes = fx ? (size_t)cols * 4 : (size_t)nb_k(cols) * BS_Q8K;
  uint8_t *dw = nullptr, *dx = nullptr;
  float* dy = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (hipMalloc(&dw, pbytes * (size_t)ncopy) != hipSuccess || hipMalloc(&dx, xbytes) != hipSuccess ||
      hipMalloc(&dy, (size_t)rows * 4) != hipSuccess || hipEventCreate(&e0) != hipSuccess ||
      hipEventCreate(&e1) != hipSuccess)
    rc = fail(c, C2H_ERR_HIP, "gemv timing: allocation failed");
  if (!rc && (stream_copy(c->stream, dw, packed.data(), pbytes, hipMemcpyHostToDevice) != hipSuccess ||
              stream_copy(c->stream, dx, xq, xbytes, hipMemcpyHostToDevice) != hipSuccess))
    rc = fail(c, C2H_ERR_HIP, "gemv timing: upload failed");
  for (int64_t i = 1; !rc && i < ncopy; ++i)
    if (hipMemcpyAsync(dw + (size_t)i * pbytes, dw, pbytes, hipMemcpyDeviceToDevice, c->stream) != hipSuccess)
      rc = fail(c, C2H_ERR_HIP, "gemv timing: copies failed");
  float t = 0.0f;
  if (!rc) {
    auto launch = [&](int64_t i) {
      rc = rc ? rc : c2h_gemv_dev(c, type, dw + (size_t)(i % ncopy) * pbytes, dx, rows, cols, dy, nullptr);
    };
    for (int i = 0; i < 20; ++i) launch(ncopy - 1 - i % ncopy);  // warm-up (clocks up, code loaded)
    (void)hipEventRecord(e0, c->stream);
    for (int i = 0; i < iters; ++i) launch(i);
    (void)hipEventRecord(e1, c->stream);
    if (!rc && (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&t, e0, e1) != hipSuccess))
      rc = fail(c, C2H_ERR_HIP, "gemv timing failed");
  }
  (void)hipStreamSynchronize(c->stream);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  for (void* p : {(void*)dw, (void*)dx, (void*)dy})
    if (p) (void)hipFree(p);
  if (rc) return rc;
  *ms = t / iters;
  return C2H_OK;
}

int c2h_time_quantize_q8k(c2h_ctx* c, const float* x, int32_t cols, int32_t iters, int64_t rotate_bytes, float* ms) {
  if (!c || !x || !ms || cols < 256 || cols > 16384 || iters <= 0 || iters > 100000 || rotate_bytes < 0)
    return C2H_ERR_INVALID;
  HIPCHK(c, hipSetDevice(c->device));
  const int nb = cols / 256;
  const size_t xbytes = (size_t)nb * 1024;  // 16-byte aligned rows of the f32 input
  const int64_t ncopy = std::min<int64_t>(65536, std::max<int64_t>(1, (rotate_bytes + (int64_t)xbytes - 1) / (int64_t)xbytes));
  float* dx = nullptr;
  uint8_t* dy = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = C2H_OK;
  if (hipMalloc(&dx, xbytes * (size_t)ncopy) != hipSuccess || hipMalloc(&dy, (size_t)nb * BS_Q8K) != hipSuccess ||
      hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
    rc = fail(c, C2H_ERR_HIP, "quantise timing: allocation failed");
  if (!rc && stream_copy(c->stream, dx, x, xbytes, hipMemcpyHostToDevice) != hipSuccess)
    rc = fail(c, C2H_ERR_HIP, "quantise timing: upload failed");
  for (int64_t i = 1; !rc && i < ncopy; ++i)
    if (hipMemcpyAsync(reinterpret_cast<uint8_t*>(dx) + (size_t)i * xbytes, dx, xbytes, hipMemcpyDeviceToDevice,
                       c->stream) != hipSuccess)
      rc = fail(c, C2H_ERR_HIP, "quantise timing: copies failed");
  float t = 0.0f;
  if (!rc) {
    auto launch = [&](int64_t i) {
      const float* xi = reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(dx) + (size_t)(i % ncopy) * xbytes);
      hipLaunchKernelGGL(k_quantize_q8k, dim3((nb + 3) / 4), dim3(256), 0, c->stream, xi, nb, dy);
    };
    for (int i = 0; i < 20; ++i) launch(ncopy - 1 - i % ncopy);  // warm-up
    (void)hipEventRecord(e0, c->stream);
    for (int i = 0; i < iters; ++i) launch(i);
    (void)hipEventRecord(e1, c->stream);
    if (hipGetLastError() != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
        hipEventElapsedTime(&t, e0, e1) != hipSuccess)
      rc = fail(c, C2H_ERR_HIP, "quantise timing failed");
  }
  (void)hipStreamSynchronize(c->stream);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (dx) (void)hipFree(dx);
  if (dy) (void)hipFree(dy);
  if (rc) return rc;
  *ms = t / iters;
  return C2H_OK;
}

}  // extern "C"
