"""Per-phase cycle stamps of the decode layer kernels (measurement tool).

`build` writes an instrumented copy of the kernel sources into
_build/phase/ at the repository root, with `s_memtime` stamps at the phase
boundaries of k_gemv_row's body (qkv, attn_out, ffn_in, ffn_out) and of
k_attn_core's tiers, in the separate kernels and in the fused launches
(k_attn_block, k_attn_oproj: their parts stamp as the kernels they run; set
C2H_NO_FUSE=1 for the separate launches' figures), and links it as _build/phase/libc2h_phase.so (same C ABI plus
c2h_phase_read).  Nothing is written into the c2slm_amd package.  Lane 0 of every wave writes its stamp per phase into LDS;
at the kernel's end the first and the last workgroup of each launch copy
their stamps into a device array, which every later launch of the same
kernel overwrites, so a read after a run holds the last launch's stamps.
The product library is untouched.

`run [T]` (GPU) loads that library (C2H_LIB), runs the decode workload -- a
synthetic Qwen2.5-0.5B-shaped model, a prefill of T-16 tokens, 16 greedy
steps, the last one attending over T positions (default 48) -- and prints
the table: per phase, the latest wave's stamp minus wave 0's entry stamp, in
shader clocks.  Above 256 positions it prints the any-length attention
tier's stamps wave by wave instead.

    python phase_trace.py build      # CPU: hipcc cross-compiles
    python phase_trace.py run        # GPU
    python phase_trace.py run 512    # GPU, long-context attention
    python phase_trace.py run 48 qwen3   # GPU, the Qwen3-1.7B shape's GEMVs
    python phase_trace.py run 48 real-formats   # GPU, the published format mix (k_gemv_f stamps:
                                                # x = staged in LDS, items = block terms in LDS)
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
BDIR = os.path.join(ROOT, "_build", "phase")
OUT_LIB = os.path.join(BDIR, "libc2h_phase.so")
N_WAVES, N_SLOTS = 8, 16
GEMV_KINDS = ["qkv", "attn_out", "ffn_in", "ffn_out"]
GEMV_PHASES = ["entry", "args", "issued", "x", "norm_end", "quant", "w", "items", "end", "norm_start"]
ATTN_PHASES = ["entry", "args", "issued", "qkv", "rope", "scores", "softmax", "av", "end", "pos", "k_in", "v_in", "max", "exp", "sum"]

_STAMPS = r"""namespace c2h {
__device__ long long g_phase[6][2][8][16];
template <int NB, int PRO, int MODE>
__device__ __forceinline__ int phase_kind() {
  return (PRO == PRO_NORM && MODE == MODE_BIAS)                 ? 0
         : (PRO == PRO_QUANT && MODE == MODE_RESID && NB <= 8)  ? 1
         : (PRO == PRO_NORM && MODE == MODE_SWIGLU)             ? 2
         : (PRO == PRO_QUANT && MODE == MODE_RESID)             ? 3
                                                                : -1;
}
// Stamps go to LDS (lane 0 of each wave, its own row) and are copied to
// g_phase once, at the kernel's end: a global store per stamp would be
// counted by vmcnt, and the kernel's own waits for its loads would then
// wait for the stamps' stores too.
#define PH_DECL \
  __shared__ long long ph_s_[8][16]; \
  if ((threadIdx.x & 63) == 0) \
    for (int k_ = 0; k_ < 16; ++k_) ph_s_[threadIdx.x >> 6][k_] = 0
#define PH_G(k) do { if ((threadIdx.x & 63) == 0) ph_s_[threadIdx.x >> 6][k] = __builtin_amdgcn_s_memtime(); } while (0)
#define PH_G_END do { const int kd_ = phase_kind<NB, PRO, MODE>(); \
  if (kd_ >= 0 && (threadIdx.x & 63) == 0 && by == 0 && (bx == 0 || bx == J.n_wg - 1)) \
    for (int k_ = 0; k_ < 16; ++k_) \
      g_phase[kd_][bx == 0 ? 0 : 1][threadIdx.x >> 6][k_] = ph_s_[threadIdx.x >> 6][k_]; } while (0)
// k_gemv_f's body (float-input projections) stamps into the same slots
template <int PRO, int MODE>
__device__ __forceinline__ int phase_kind_f() {
  return (PRO == PRO_NORM && MODE == MODE_BIAS)       ? 0
         : (PRO == PRO_QUANT && MODE == MODE_RESID)   ? 1
         : (PRO == PRO_NORM && MODE == MODE_SWIGLU)   ? 2
                                                      : -1;
}
#define PH_F_END do { const int kd_ = phase_kind_f<PRO, MODE>(); \
  if (kd_ >= 0 && (threadIdx.x & 63) == 0 && by == 0 && (bx == 0 || bx == J.n_wg - 1)) \
    for (int k_ = 0; k_ < 16; ++k_) \
      g_phase[kd_][bx == 0 ? 0 : 1][threadIdx.x >> 6][k_] = ph_s_[threadIdx.x >> 6][k_]; } while (0)
// the FFN launch's down-projection blocks (slot 3, the ffn_out row)
#define PH_D_END(kd_, first_, last_) do { \
  if ((threadIdx.x & 63) == 0 && ((first_) || (last_))) \
    for (int k_ = 0; k_ < 16; ++k_) \
      g_phase[kd_][(first_) ? 0 : 1][threadIdx.x >> 6][k_] = ph_s_[threadIdx.x >> 6][k_]; } while (0)
#define PH_AT(k, t) do { if ((threadIdx.x & 63) == 0) ph_s_[threadIdx.x >> 6][k] = (t); } while (0)
#define PH_A_END do { const bool f_ = h == 0; \
  const bool l_ = h == P.n_heads - 1; \
  if ((threadIdx.x & 63) == 0 && bz == 0 && (f_ || l_)) \
    for (int k_ = 0; k_ < 16; ++k_) \
      g_phase[TIER == ATT_TIER_ANY ? 5 : 4][f_ ? 0 : 1][threadIdx.x >> 6][k_] = ph_s_[threadIdx.x >> 6][k_]; } while (0)
#define PH_A(k) PH_AT(k, __builtin_amdgcn_s_memtime())
// k_attn_h128 (no k_attn_core runs at head_dim 128): its stamps take the attention slot
#define PH_H_END do { const bool f_ = h == 0; \
  const bool l_ = h == (int)(gridDim.x * gridDim.y) - 1; \
  if ((threadIdx.x & 63) == 0 && blockIdx.z == 0 && (f_ || l_)) \
    for (int k_ = 0; k_ < 16; ++k_) \
      g_phase[4][f_ ? 0 : 1][threadIdx.x >> 6][k_] = ph_s_[threadIdx.x >> 6][k_]; } while (0)
"""


def _patch(text: str, start: str, end: str, edits) -> str:
    i0, i1 = text.index(start), text.index(end)
    body = text[i0:i1]
    for old, new in edits:
        if body.count(old) != 1:
            raise RuntimeError(f"phase site not found once: {old[:70]!r}")
        body = body.replace(old, new)
    body = body.rstrip()
    if not body.endswith("}"):
        raise RuntimeError("kernel body does not end in '}'")
    return text[:i0] + body[:-1] + "  PH_END;\n}\n\n" + text[i1:]


def instrument(kernels: str) -> str:
    s = kernels.replace("namespace c2h {\n", _STAMPS, 1)
    # the bodies shared by the separate kernels and the fused launches
    s = _patch(s, "__device__ __forceinline__ void gemv_row_body(",
               "template <int NB, int PRO, int MODE>\n__global__ void __launch_bounds__(row_threads(NB, PRO, MODE)) k_gemv_row(", [
                   ("  constexpr int NT = row_threads(NB, PRO, MODE);\n",
                    "  PH_DECL;\n  constexpr int NT = row_threads(NB, PRO, MODE);\n"),
                   ("  const int tid = threadIdx.x;\n  const int wave = tid >> 6, lane = tid & 63;\n  // ---- the input",
                    "  PH_G(0);\n  const int tid = threadIdx.x;\n  const int wave = tid >> 6, lane = tid & 63;\n"
                    "  // ---- the input"),
                   ("  if (bx >= J.n_wg) return;  // uniform: the launch's widest job sets the grid\n",
                    "  if (bx >= J.n_wg) return;  // uniform: the launch's widest job sets the grid\n"
                    "  PH_G(1);\n"),
                   ("  if (MODE == MODE_BIAS) yres = (J.bias ? J.bias : xp)[J.bias ? out_row : 0];\n  issue_fence();\n",
                    "  if (MODE == MODE_BIAS) yres = (J.bias ? J.bias : xp)[J.bias ? out_row : 0];\n  issue_fence();\n"
                    "  PH_G(2);\n"),
                   ("\n\n  // ---- prologue: the Q8_K input row in LDS", "\n  asm volatile(\"\" ::\"v\"(xa[0].x));\n  PH_G(3);\n"
                    "\n  // ---- prologue: the Q8_K input row in LDS"),
                   ("    float inv = 0.0f;  //", "    PH_G(9);\n    float inv = 0.0f;  //"),
                   ("    const float4 xn[1] = {norm4(", "    PH_G(4);\n    const float4 xn[1] = {norm4("),
                   ("  // ---- items\n", "  PH_G(5);\n  asm volatile(\"\" ::\"v\"(w1.a.x), \"v\"(w1.c.w));\n"
                    "  PH_G(6);\n  // ---- items\n"),
                   ("  // ---- per-row fold in the reference's order, then the epilogue\n",
                    "  PH_G(7);\n  // ---- per-row fold in the reference's order, then the epilogue\n"),
               ]).replace("PH_END;", "PH_G(8);\n  PH_G_END;", 1)
    s = _patch(s, "__device__ __forceinline__ void attn_core_body(",
               "template <int TIER>\n__global__ void __launch_bounds__(256)\n    k_attn_core(C2hState* __restrict__ st,", [
                   ("  const int tid = threadIdx.x;\n  const int layer = dims & 0xff",
                    "  PH_DECL;\n  const long long ph_entry_ = __builtin_amdgcn_s_memtime();\n"
                    "  const int tid = threadIdx.x;\n  const int layer = dims & 0xff"),
                   ('"s"(P.scale), "s"(P.store_kv));\n', '"s"(P.scale), "s"(P.store_kv));\n'
                    '  PH_A(1);\n'),
                   ("  const int h = g * qpkv + hx;\n", "  const int h = g * qpkv + hx;\n  PH_AT(0, ph_entry_);\n"),
                   ("  const int T = pos + 1;\n", "  asm volatile(\"\" ::\"s\"(pos));\n  PH_A(9);\n  const int T = pos + 1;\n"),
                   ("    __syncthreads();\n    const int p = c0 + tid;\n",
                    "    PH_A(10);\n    __syncthreads();\n    const int p = c0 + tid;\n"),
                   ("    __syncthreads();\n    const float inv = inv_slot;\n",
                    "    PH_A(11);\n    __syncthreads();\n    const float inv = inv_slot;\n"),
                   ("    if (sc[0] != sc[0]) mx = sc[0];\n    for (int p = tid; p < T; p += 256) sc[p] = (float)exp((double)(sc[p] - mx));\n    if constexpr (!ANY && TIER <= SUM_DIRECT_N) pad_chain(sc, T);\n    __syncthreads();\n",
                    "    if (sc[0] != sc[0]) mx = sc[0];\n    PH_A(12);\n    for (int p = tid; p < T; p += 256) sc[p] = (float)exp((double)(sc[p] - mx));\n    if constexpr (!ANY && TIER <= SUM_DIRECT_N) pad_chain(sc, T);\n    __syncthreads();\n    PH_A(13);\n"),
                   ("      while_summing();\n    }\n",
                    "      while_summing();\n    }\n    PH_A(14);\n"),
                   ("  qkv_s[bm][tid & 63] = own;\n  __syncthreads();\n",
                    "  PH_A(2);\n  qkv_s[bm][tid & 63] = own;\n  __syncthreads();\n  PH_A(3);\n"),
                   ("  __syncthreads();\n\n  // (a batch of query tokens",
                    "  __syncthreads();\n  PH_A(4);\n\n  // (a batch of query tokens"),
                   ("  // softmax, then V chunk 0 from registers into LDS buffer 0\n",
                    "  PH_A(5);\n  // softmax, then V chunk 0 from registers into LDS buffer 0\n"),
                   ("    softmax([] {});\n    if (tid < HD && nbat > 0) acc = av_chain_pad(sc, vbuf, nbat, d, acc);\n",
                    "    softmax([] {});\n    PH_A(6);\n    if (tid < HD && nbat > 0) acc = av_chain_pad(sc, vbuf, nbat, d, acc);\n"),
                   ("    });\n    // both roles pass nch barriers, one per chunk\n",
                    "    });\n    PH_A(6);\n    // both roles pass nch barriers, one per chunk\n"),
                   ("  if (tid < HD) {\n    acc = __builtin_fmaf(sc[pos], v_s[d], acc);\n",
                    "  PH_A(7);\n  if (tid < HD) {\n    acc = __builtin_fmaf(sc[pos], v_s[d], acc);\n"),
               ]).replace("PH_END;", "PH_A(8);\n  PH_A_END;", 1)
    # the FFN launch's down blocks (slot 3, the ffn_out row): entry, args, issued (weights), x (h polled,
    # wave 0), quant (wave 0), w (after the barrier), end (terms stored)
    s = _patch(s, "template <int NB, int NT>\n__device__ __forceinline__ void down_block_body(",
               "// The FFN of one layer in one launch", [
                   ("  __shared__ Q8KRow<NB> s;\n", "  __shared__ Q8KRow<NB> s;\n  PH_DECL;\n  PH_G(0);\n"),
                   ("  const int row = g * RW + (tid >> 2), u = tid & 3;\n",
                    "  const int row = g * RW + (tid >> 2), u = tid & 3;\n  PH_G(1);\n"),
                   ("    const float4 v[1] = {poll_tagged4(P.x_tag + b * QK_K + 4 * lane, tag, P.wait_err)};\n    quantize_blocks<1>(v, b, 0, b + 1, s);\n",
                    "    PH_G(2);\n    const float4 v[1] = {poll_tagged4(P.x_tag + b * QK_K + 4 * lane, tag, P.wait_err)};\n    PH_G(3);\n    quantize_blocks<1>(v, b, 0, b + 1, s);\n    PH_G(5);\n"),
                   ("  __syncthreads();\n  if (row < J.rows) {  // whole quads", "  __syncthreads();\n  PH_G(6);\n  if (row < J.rows) {  // whole quads"),
               ]).replace("PH_END;", "PH_G(8);\n  PH_D_END(3, bx == 0, bx == ng * NB - 1);", 1)
    # float-input projections (k_gemv_f): entry, args, issued, norm_start, norm_end, x (staged in LDS),
    # items (the block terms in LDS), end
    s = _patch(s, "__device__ __forceinline__ void gemv_f_body(",
               "template <int PRO, int MODE>\n__global__ void __launch_bounds__(256) k_gemv_f(GemvParams P) {", [
                   ("  constexpr bool PAIRED = (MODE == MODE_SWIGLU);\n",
                    "  constexpr bool PAIRED = (MODE == MODE_SWIGLU);\n  PH_DECL;\n  PH_G(0);\n"),
                   ("  if (bx >= J.n_wg) return;\n", "  if (bx >= J.n_wg) return;\n  PH_G(1);\n"),
                   ("  issue_fence();\n\n  // ---- prologue: x (normalised", "  issue_fence();\n  PH_G(2);\n\n  // ---- prologue: x (normalised"),
                   ("    const float inv = (PRO == PRO_NORM) ? rms_inv_regs(xs, P.n_x, P.eps) : rms_inv4(xa, P.n_x, P.eps, sq, &inv_slot);\n",
                    "    PH_G(9);\n    const float inv = (PRO == PRO_NORM) ? rms_inv_regs(xs, P.n_x, P.eps) : rms_inv4(xa, P.n_x, P.eps, sq, &inv_slot);\n    PH_G(4);\n"),
                   ("  __syncthreads();\n\n  // ---- items and the per-row fold", "  __syncthreads();\n  PH_G(3);\n\n  // ---- items and the per-row fold"),
                   ("    __syncthreads();\n    if (tid < R && nb8 <= 32) {", "    __syncthreads();\n    PH_G(7);\n    if (tid < R && nb8 <= 32) {"),
               ]).replace("PH_END;", "PH_G(8);\n  PH_F_END;", 1)
    # head_dim 128: entry, args, issued, pos, qkv (q|k|v in LDS), rope (QK-norm and RoPE done), scores, max,
    # exp, sum, softmax (normalised), av, end
    s = _patch(s, "template <int VCH>\n__global__ void __launch_bounds__(256) k_attn_h128(AttnCoreParams P) {",
               "template __global__ void k_attn_h128<0>(AttnCoreParams);", [
                   ("  extern __shared__ __align__(16) unsigned char smem[];\n  float* sc = reinterpret_cast<float*>(smem);\n",
                    "  extern __shared__ __align__(16) unsigned char smem[];\n  float* sc = reinterpret_cast<float*>(smem);\n"
                    "  PH_DECL;\n  const long long ph_entry_ = __builtin_amdgcn_s_memtime();\n"),
                   ('"s"(P.scale), "s"(P.state), "s"(P.tok0), "s"(gridDim.x));\n',
                    '"s"(P.scale), "s"(P.state), "s"(P.tok0), "s"(gridDim.x));\n  PH_AT(0, ph_entry_);\n  PH_A(1);\n'),
                   ("  const int T = pos + 1;\n", "  asm volatile(\"\" ::\"s\"(pos));\n  PH_A(9);\n  const int T = pos + 1;\n"),
                   ("  qkv_s[role][e] = own;\n", "  PH_A(2);\n  qkv_s[role][e] = own;\n"),
                   ("  // ---- RoPE: threads 0..63", "  PH_A(3);\n  // ---- RoPE: threads 0..63"),
                   ("  if (P.store_kv && blockIdx.x == 0 && tid < HD", "  PH_A(4);\n  if (P.store_kv && blockIdx.x == 0 && tid < HD"),
                   ("  // ---- softmax: max (x[0] first", "  PH_A(5);\n  // ---- softmax: max (x[0] first"),
                   ("  if (sc[0] != sc[0]) mx = sc[0];\n  for (int p = tid; p < T; p += 256) sc[p] = (float)exp((double)(sc[p] - mx));\n  if (T <= H128_SUM_DIRECT_N) pad_chain(sc, T);\n  __syncthreads();\n",
                    "  if (sc[0] != sc[0]) mx = sc[0];\n  PH_A(12);\n  for (int p = tid; p < T; p += 256) sc[p] = (float)exp((double)(sc[p] - mx));\n  if (T <= H128_SUM_DIRECT_N) pad_chain(sc, T);\n  __syncthreads();\n  PH_A(13);\n"),
                   ("  const float inv = inv_s[2];\n", "  PH_A(14);\n  const float inv = inv_s[2];\n"),
                   ("  // ---- AV: out[d] = fma chain over p of (prob[p], V[p][d])\n",
                    "  PH_A(6);\n  // ---- AV: out[d] = fma chain over p of (prob[p], V[p][d])\n"),
               ]).replace("PH_END;", "PH_A(8);\n  PH_H_END;", 1)
    return s


_READER = r"""
namespace c2h { extern __device__ long long g_phase[6][2][8][16]; }
extern "C" int c2h_phase_read(long long* out) {
  return hipMemcpyFromSymbol(out, HIP_SYMBOL(c2h::g_phase), sizeof(long long) * 6 * 2 * 8 * 16) == hipSuccess ? 0 : -1;
}
"""


def build() -> str:
    from c2slm_amd import build as B
    bdir = BDIR
    shutil.rmtree(bdir, ignore_errors=True)
    src = os.path.join(bdir, "k", "csrc")  # the sources include ../../include/c2h.h
    os.makedirs(src)
    os.symlink(os.path.join(ROOT, "include"), os.path.join(bdir, "include"))
    for f in os.listdir(B.CSRC):
        if os.path.isfile(os.path.join(B.CSRC, f)):
            shutil.copy(os.path.join(B.CSRC, f), src)
    kp = os.path.join(src, "c2h_kernels.hip")
    with open(kp) as f:
        text = instrument(f.read())
    with open(kp, "w") as f:
        f.write(text)
    with open(os.path.join(src, "c2h_api.hip"), "a") as f:
        f.write(_READER)
    flags = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={B.ARCH}", "-ffp-contract=off", "-fgpu-rdc",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", *B.PRELOAD, "-I", os.path.join(ROOT, "include")]
    objs = []
    for name in B.SOURCES:
        obj = os.path.join(bdir, name + ".o")
        res = subprocess.run([B.hipcc(), *flags, "-c", os.path.join(src, name), "-o", obj], capture_output=True,
                             text=True)
        if res.returncode:
            sys.stderr.write(res.stderr[-4000:])
            raise RuntimeError(f"hipcc failed on the instrumented {name}")
        objs.append(obj)
    res = subprocess.run([B.hipcc(), "-shared", "-fPIC", "-fgpu-rdc", "--hip-link", f"--offload-arch={B.ARCH}",
                          *objs, "-o", OUT_LIB], capture_output=True, text=True)
    if res.returncode:
        sys.stderr.write(res.stderr[-4000:])
        raise RuntimeError("link of the instrumented library failed")
    return OUT_LIB


def run(last: int = 48, model: str = "qwen2.5-0.5b") -> None:
    """Prefill last-16 tokens, take 16 greedy steps, print the stamps of the last launches.

    At last <= 256 the table covers every kernel (first and last workgroup, latest wave); above
    256 the attention launch runs the any-length tier, and the table lists its waves one by one.
    """
    if os.environ.get("C2H_LIB") != OUT_LIB:  # the library path is fixed when _lib loads
        env = dict(os.environ, C2H_LIB=OUT_LIB)
        sys.exit(subprocess.run([sys.executable, "-u", os.path.join(ROOT, "phase_trace.py"), "run", str(last), model],
                                env=env, cwd=ROOT).returncode)
    if not 17 <= last <= 1024:
        raise ValueError("last must lie in 17..1024")
    import ctypes as C

    import numpy as np

    from c2slm_amd import _lib as H
    from c2slm_amd import gguf as G
    shape = {"qwen2.5-0.5b": G.QWEN05B, "qwen3": G.QWEN3_1_7B, "real-formats": G.QWEN05B_REAL_FORMATS}[model]
    path = f"/tmp/c2h_phase_{model}.gguf"
    if not os.path.exists(path):
        G.write_synthetic_model(path, shape, seed=20261201)
    gf = G.GGUFFile(path)
    ctx = H.Ctx(H.desc_from_gguf(gf, max_ctx=1024))
    H.load_gguf_into(ctx, gf)
    prompt = np.random.default_rng(20261201).integers(0, gf.tensor_map["token_embd.weight"].dims[1], last - 16)
    ctx.prefill(prompt.astype(np.int32), 0)
    _, im_end, eos = G.special_token_ids(gf)
    for p in range(last - 16, last):
        ctx.step(p, 1.15, im_end, eos)
    ctx.sync()
    buf = (C.c_longlong * (6 * 2 * N_WAVES * N_SLOTS))()
    fn = H.lib().c2h_phase_read
    fn.argtypes = [C.c_void_p]
    if fn(buf) != 0:
        raise RuntimeError("c2h_phase_read failed")
    a = np.array(buf, dtype=np.int64).reshape(6, 2, N_WAVES, N_SLOTS)
    if last > 256 and model != "qwen3":
        print(f"attention, any-length tier, layer 23 of the 16th step, T = {last}; shader clocks from wave 0's"
              " entry, per wave")
        print(f"{'wg':5s} {'wave':4s} " + " ".join(f"{p:>8s}" for p in ATTN_PHASES))
        for wg in range(2):
            t0 = a[5, wg, 0, 0]
            for w in range(4):
                print(f"{('first', 'last')[wg]:5s} {w:4d} " + " ".join(
                    f"{int(a[5, wg, w, i] - t0) if a[5, wg, w, i] else -1:8d}" for i in range(len(ATTN_PHASES))))
        ctx.close()
        return
    print(f"{model}: last launch of each kernel (last layer of the 16th step, T = {last}); shader clocks from"
          " wave 0's entry, latest wave (attention: head_dim 64 only)")
    for k, name in enumerate(GEMV_KINDS + ["attn"]):
        cols = ATTN_PHASES if name == "attn" else GEMV_PHASES
        print(f"{name:9s} {'wg':5s} " + " ".join(f"{p:>10s}" for p in cols))
        for wg in range(2):
            t0 = a[k, wg, 0, 0]
            vals = []
            for i in range(len(cols)):
                v = [int(a[k, wg, w, i] - t0) for w in range(N_WAVES) if a[k, wg, w, i]]
                vals.append(max(v) if v else -1)
            print(f"{name:9s} {('first', 'last')[wg]:5s} " + " ".join(f"{v:10d}" for v in vals))
    ctx.close()


if __name__ == "__main__":
    if len(sys.argv) not in (2, 3, 4) or sys.argv[1] not in ("build", "run") or (
            len(sys.argv) >= 3 and (sys.argv[1] != "run" or not sys.argv[2].isdigit())) or (
            len(sys.argv) == 4 and sys.argv[3] not in ("qwen2.5-0.5b", "qwen3", "real-formats")):
        sys.exit("usage: python phase_trace.py build | run [positions [qwen2.5-0.5b | qwen3 | real-formats]]")
    if sys.argv[1] == "build":
        print(build())
    else:
        run(int(sys.argv[2]) if len(sys.argv) >= 3 else 48, sys.argv[3] if len(sys.argv) == 4 else "qwen2.5-0.5b")
