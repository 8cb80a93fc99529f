"""ctypes front end of the C oracle (oracle/c2slm_oracle.c).

Test infrastructure only: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the reported CPU
baseline, never as the thing measured.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32P = C.POINTER(C.c_float)
U8P = C.POINTER(C.c_uint8)
I32P = C.POINTER(C.c_int32)


class OrcLayer(C.Structure):
    _fields_ = [(n, F32P) for n in ("attn_norm", "bq", "bk", "bv", "ffn_norm")] + \
               [(n, U8P) for n in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")] + \
               [(n, C.c_int32) for n in ("tq", "tk", "tv", "to", "tg", "tu", "td")] + \
               [(n, F32P) for n in ("q_norm", "k_norm")]


class OrcModel(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("n_layers", "n_embd", "n_heads", "n_kv_heads", "head_dim", "n_ff",
                                         "n_vocab", "max_ctx")] + \
               [("eps", C.c_float), ("theta", C.c_float), ("token_embd", U8P), ("embd_type", C.c_int32),
                ("output", U8P), ("output_type", C.c_int32), ("output_norm", F32P),
                ("layers", C.POINTER(OrcLayer)), ("n_threads", C.c_int32), ("simd_avx2", C.c_int32)]


def build():
    subprocess.run(["make", "-C", HERE, "-s"], check=True)


_libs: dict = {}


def lib(path: str | None = None):
    """The oracle library (another build of the same source with `path`)."""
    path = path or LIB_PATH
    if path not in _libs:
        if path == LIB_PATH and not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(path)
        sig = {
            "orc_fp16_simd": (C.c_float, [C.c_uint16]),
            "orc_fp16_tensor": (C.c_float, [C.c_uint16]),
            "orc_fp16_simd_bits": (C.c_uint32, [C.c_uint16]),
            "orc_fp16_tensor_bits": (C.c_uint32, [C.c_uint16]),
            "orc_quantize_row_q8k": (None, [F32P, U8P, C.c_int, C.c_long]),
            "orc_q4k_block_isums": (None, [U8P, U8P, I32P]),
            "orc_q6k_block_isum": (C.c_int32, [U8P, U8P]),
            "orc_dot_q4k_q8k": (C.c_float, [U8P, U8P, C.c_int]),
            "orc_dot_q6k_q8k": (C.c_float, [U8P, U8P, C.c_int]),
            "orc_dot_q8_0": (C.c_float, [U8P, F32P, C.c_int]),
            "orc_avx2_dot_q4k_q8k": (C.c_float, [U8P, U8P, C.c_int]),
            "orc_avx2_dot_q6k_q8k": (C.c_float, [U8P, U8P, C.c_int]),
            "orc_avx2_q6k_block_isum": (C.c_int32, [U8P, U8P]),
            "orc_avx2_dot_q8_0": (C.c_float, [U8P, F32P, C.c_int]),
            "orc_dot_q5_0": (C.c_float, [U8P, F32P, C.c_int]),
            "orc_dot_q4k_f32": (C.c_float, [U8P, F32P, C.c_int]),
            "orc_dot_q6k_f32": (C.c_float, [U8P, F32P, C.c_int]),
            "orc_dequant_row_q8_0": (None, [F32P, U8P, C.c_int]),
            "orc_rmsnorm": (None, [F32P, F32P, F32P, C.c_int, C.c_float]),
            "orc_rope_table": (None, [F32P, F32P, C.c_int, C.c_int, C.c_float]),
            "orc_rope_apply": (None, [F32P, C.c_int, C.c_int, C.c_int, F32P, F32P, C.c_int, C.c_int]),
            "orc_softmax": (None, [F32P, C.c_int]),
            "orc_attn_qk": (None, [F32P, F32P, C.c_int, C.c_int, C.c_float, F32P, C.c_int]),
            "orc_attn_av": (None, [F32P, F32P, C.c_int, C.c_int, F32P, C.c_int]),
            "orc_swiglu": (None, [F32P, F32P, F32P, C.c_int]),
            "orc_penalty_argmax": (C.c_int32, [F32P, C.c_int, I32P, C.c_int, C.c_int32, C.c_int32, C.c_float]),
            "orc_state_new": (C.c_void_p, [C.POINTER(OrcModel)]),
            "orc_state_free": (None, [C.c_void_p]),
            "orc_forward": (None, [C.c_void_p, C.c_int32, C.c_int, F32P]),
            "orc_compute_logits": (None, [C.c_void_p, F32P, F32P]),
            "orc_ingest_from": (C.c_int, [C.c_void_p, C.c_int, I32P, C.c_int, F32P]),
            "orc_generate": (C.c_int, [C.c_void_p, C.c_int, C.c_int32, C.c_int32, C.c_float, I32P]),
            "orc_state_logits": (F32P, [C.c_void_p]),
            "orc_state_normx": (F32P, [C.c_void_p]),
            "orc_state_kv": (F32P, [C.c_void_p]),
            "orc_state_token_ids": (I32P, [C.c_void_p]),
            "orc_state_seq_len": (C.c_int32, [C.c_void_p]),
            "orc_state_set_seq_len": (None, [C.c_void_p, C.c_int32]),
            "orc_state_trace": (None, [C.c_void_p, U8P, C.c_long]),
            "orc_state_trace_len": (C.c_long, [C.c_void_p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _libs[path] = L
    return _libs[path]


def ptr(a: np.ndarray, typ):
    return a.ctypes.data_as(typ)


# ---------------------------------------------------------- kernel wrappers


def quantize_row_q8k(x: np.ndarray, y_len: int | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    nb = len(x) // 256
    n = y_len if y_len is not None else nb * 292
    y = np.zeros(n, dtype=np.uint8)
    lib().orc_quantize_row_q8k(ptr(x, F32P), ptr(y, U8P), len(x), n)
    return y


def gemv(w: np.ndarray, ggml_type: int, rows: int, cols: int, x: np.ndarray | None = None,
         q8k: np.ndarray | None = None, float_x: bool = False) -> np.ndarray:
    """y = W·x for the reference's row functions (row stride with floor semantics).
    K-quants take the Q8_K row of x (GEMVQ*_K_Q8_K), or with float_x the f32
    x itself (GEMVQ4_K / GEMVQ6_K, engine/model.go:250-270 without a pool)."""
    from c2slm_amd import gguf as G
    L = lib()
    w = np.ascontiguousarray(w, dtype=np.uint8)
    rb = G.row_bytes(ggml_type, cols)
    y = np.empty(rows, dtype=np.float32)
    if ggml_type in (G.Q4_K, G.Q6_K) and float_x:
        x = np.ascontiguousarray(x, dtype=np.float32)
        fn = L.orc_dot_q4k_f32 if ggml_type == G.Q4_K else L.orc_dot_q6k_f32
        base = w.ctypes.data
        xp = ptr(x, F32P)
        for r in range(rows):
            y[r] = fn(C.cast(base + r * rb, U8P), xp, cols)
    elif ggml_type in (G.Q4_K, G.Q6_K):
        if q8k is None:
            q8k = quantize_row_q8k(x)
        q8k = np.ascontiguousarray(q8k, dtype=np.uint8)
        fn = L.orc_dot_q4k_q8k if ggml_type == G.Q4_K else L.orc_dot_q6k_q8k
        base = w.ctypes.data
        qp = ptr(q8k, U8P)
        for r in range(rows):
            y[r] = fn(C.cast(base + r * rb, U8P), qp, cols)
    else:
        x = np.ascontiguousarray(x, dtype=np.float32)
        fn = L.orc_dot_q8_0 if ggml_type == G.Q8_0 else L.orc_dot_q5_0
        base = w.ctypes.data
        xp = ptr(x, F32P)
        for r in range(rows):
            y[r] = fn(C.cast(base + r * rb, U8P), xp, cols)
    return y


# ------------------------------------------------------------------ model


class OracleEngine:
    """The reference's Engine state (model + KV cache + arena) over a GGUF file,
    computed by the oracle on the host CPU."""

    def __init__(self, gf, max_ctx: int = 1024, n_threads: int = 1, lib_path: str | None = None,
                 avx2_dots: bool = False):
        """avx2_dots: the GEMVs run the reference's AVX2 kernels as restated
        in oracle/c2slm_avx2.c (the CPU baseline) instead of the scalar
        restatement; the results are identical."""
        from c2slm_amd import gguf as G
        self._L = lib(lib_path)
        self.gf = gf
        md = gf
        def u32(k2, k3, dflt):
            v = md.get_u32(k2) or md.get_u32(k3)
            return v or dflt
        def f32(k2, k3, dflt):
            v = md.get_f32(k2) or md.get_f32(k3)
            return v or dflt
        E = u32("qwen2.embedding_length", "qwen3.embedding_length", 896)
        L = u32("qwen2.block_count", "qwen3.block_count", 24)
        H = u32("qwen2.attention.head_count", "qwen3.attention.head_count", 14)
        KVH = u32("qwen2.attention.head_count_kv", "qwen3.attention.head_count_kv", 2)
        F = u32("qwen2.feed_forward_length", "qwen3.feed_forward_length", 4864)
        theta = f32("qwen2.rope.freq_base", "qwen3.rope.freq_base", 1.0e6)
        eps = f32("qwen2.attention.layer_norm_rms_epsilon", "qwen3.attention.layer_norm_rms_epsilon", 1e-6)
        tm = gf.tensor_map
        emb = tm["token_embd.weight"]
        V = int(emb.dims[1])
        out = tm.get("output.weight", emb)
        self._keep = []

        def u8(ti):
            if ti is None:
                return C.cast(None, U8P)
            a = np.ascontiguousarray(ti.data)
            self._keep.append(a)
            return ptr(a, U8P)

        def fp(ti):
            if ti is None:
                return C.cast(None, F32P)
            a = np.ascontiguousarray(np.frombuffer(ti.data, dtype="<f4"))
            self._keep.append(a)
            return ptr(a, F32P)

        layers = (OrcLayer * L)()
        for i in range(L):
            g = lambda n: tm.get(f"blk.{i}.{n}")
            ly = layers[i]
            ly.attn_norm, ly.bq, ly.bk, ly.bv, ly.ffn_norm = (
                fp(g("attn_norm.weight")), fp(g("attn_q.bias")), fp(g("attn_k.bias")), fp(g("attn_v.bias")),
                fp(g("ffn_norm.weight")))
            ly.q_norm, ly.k_norm = fp(g("attn_q_norm.weight")), fp(g("attn_k_norm.weight"))
            for fld, nm in (("wq", "attn_q"), ("wk", "attn_k"), ("wv", "attn_v"), ("wo", "attn_output"),
                            ("wg", "ffn_gate"), ("wu", "ffn_up"), ("wd", "ffn_down")):
                ti = g(nm + ".weight")
                setattr(ly, fld, u8(ti))
                setattr(ly, "t" + fld[1], ti.ggml_type)
        self._layers = layers
        m = OrcModel()
        m.n_layers, m.n_embd, m.n_heads, m.n_kv_heads = L, E, H, KVH
        m.head_dim, m.n_ff, m.n_vocab, m.max_ctx = E // H, F, V, max_ctx
        m.eps, m.theta = eps, theta
        m.token_embd, m.embd_type = u8(emb), emb.ggml_type
        m.output, m.output_type = u8(out), out.ggml_type
        m.output_norm = fp(tm["output_norm.weight"])
        m.layers = layers
        m.n_threads = n_threads
        m.simd_avx2 = 1 if avx2_dots else 0
        self.model = m
        self.n_embd, self.n_vocab, self.max_ctx = E, V, max_ctx
        self.n_layers, self.n_kv_heads, self.head_dim = L, KVH, E // H
        self.state = self._L.orc_state_new(C.byref(m))
        if not self.state:
            raise MemoryError("oracle state allocation failed")

    def close(self):
        if self.state:
            self._L.orc_state_free(self.state)
            self.state = None

    def __del__(self):
        self.close()

    def forward(self, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.n_embd, dtype=np.float32)
        self._L.orc_forward(self.state, token, pos, ptr(out, F32P))
        return out

    def compute_logits(self, normx: np.ndarray | None = None) -> np.ndarray:
        L = self._L
        nx = np.ctypeslib.as_array(L.orc_state_normx(self.state), shape=(self.n_embd,)).copy() \
            if normx is None else np.ascontiguousarray(normx, dtype=np.float32)
        out = np.empty(self.n_vocab, dtype=np.float32)
        L.orc_compute_logits(self.state, ptr(nx, F32P), ptr(out, F32P))
        return out

    def ingest_from(self, pos: int, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty(self.n_embd, dtype=np.float32)
        self._L.orc_ingest_from(self.state, pos, ptr(t, I32P), len(t), ptr(out, F32P))
        return out

    def generate(self, max_new: int, im_end: int, eos: int, penalty: float = 1.15) -> np.ndarray:
        out = np.empty(max_new, dtype=np.int32)
        n = self._L.orc_generate(self.state, max_new, im_end, eos, penalty, ptr(out, I32P))
        return out[:n]

    @property
    def seq_len(self) -> int:
        return self._L.orc_state_seq_len(self.state)

    def token_ids(self) -> np.ndarray:
        return np.ctypeslib.as_array(self._L.orc_state_token_ids(self.state), shape=(self.max_ctx,)).copy()

    def kv(self) -> np.ndarray:
        return self.kv_view().copy()

    def kv_view(self) -> np.ndarray:
        """Writable view of the KV cache [2][L][KVH][max_ctx][HD] (for pre-filling)."""
        n = 2 * self.n_layers * self.n_kv_heads * self.max_ctx * self.head_dim
        a = np.ctypeslib.as_array(self._L.orc_state_kv(self.state), shape=(n,))
        return a.reshape(2, self.n_layers, self.n_kv_heads, self.max_ctx, self.head_dim)

    def set_token_ids(self, pos0: int, ids) -> None:
        ids = np.asarray(ids, np.int32)
        np.ctypeslib.as_array(self._L.orc_state_token_ids(self.state), shape=(self.max_ctx,))[pos0:pos0 + len(ids)] = ids

    def set_seq_len(self, n: int) -> None:
        self._L.orc_state_set_seq_len(self.state, n)

    def start_q8k_trace(self, cap: int = 1 << 24) -> None:
        """Record every Q8_K row the pooled GEMV quantises from now on."""
        self._trace = np.zeros(cap, np.uint8)
        self._L.orc_state_trace(self.state, ptr(self._trace, U8P), cap)

    def take_q8k_trace(self) -> np.ndarray:
        """The Q8_K bytes recorded since the last start/take, in call order."""
        n = self._L.orc_state_trace_len(self.state)
        if n > len(self._trace):
            raise RuntimeError("Q8_K trace truncated")
        out = self._trace[:n].copy()
        self._L.orc_state_trace(self.state, ptr(self._trace, U8P), len(self._trace))
        return out
