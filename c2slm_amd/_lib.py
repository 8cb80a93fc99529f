"""ctypes binding of libc2h.so (include/c2h.h).

Loading fails loudly when the library is missing: there is no CPU fallback
anywhere in this package.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# C2H_LIB selects another build of the same ABI (for example an instrumented one)
LIB_PATH = os.environ.get("C2H_LIB") or os.path.join(HERE, "libc2h.so")

C2H_OK = 0
NOALLOC_MAX_COLS = 16384  # C2H_NOALLOC_MAX_COLS
F32, Q5_0, Q8_0, Q4_K, Q6_K = 0, 6, 8, 12, 14

ROLE = dict(TOKEN_EMBD=0, OUTPUT=1, OUTPUT_NORM=2, ATTN_NORM=10, ATTN_Q=11, ATTN_Q_BIAS=12, ATTN_K=13,
            ATTN_K_BIAS=14, ATTN_V=15, ATTN_V_BIAS=16, ATTN_OUT=17, FFN_NORM=18, FFN_GATE=19, FFN_UP=20,
            FFN_DOWN=21, ATTN_Q_NORM=22, ATTN_K_NORM=23)

LAYER_TENSORS = {
    "attn_norm.weight": "ATTN_NORM", "attn_q.weight": "ATTN_Q", "attn_q.bias": "ATTN_Q_BIAS",
    "attn_k.weight": "ATTN_K", "attn_k.bias": "ATTN_K_BIAS", "attn_v.weight": "ATTN_V",
    "attn_v.bias": "ATTN_V_BIAS", "attn_output.weight": "ATTN_OUT", "ffn_norm.weight": "FFN_NORM",
    "attn_q_norm.weight": "ATTN_Q_NORM", "attn_k_norm.weight": "ATTN_K_NORM",
    "ffn_gate.weight": "FFN_GATE", "ffn_up.weight": "FFN_UP", "ffn_down.weight": "FFN_DOWN",
}


class ModelDesc(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("n_layers", "n_embd", "n_heads", "n_kv_heads", "head_dim", "n_ff",
                                         "n_vocab", "max_ctx")] + \
               [("rms_eps", C.c_float), ("rope_theta", C.c_float), ("reserved", C.c_int32 * 6)]


class C2hError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"c2h error {code}: {msg}")
        self.code = code


_lib = None

VP = C.c_void_p
I32 = C.c_int32
I64 = C.c_int64


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with c2slm_amd/build.py (no CPU fallback exists)")
        L = C.CDLL(LIB_PATH)
        sig = {
            "c2h_create": (C.c_int, [C.POINTER(ModelDesc), C.c_int, C.POINTER(VP)]),
            "c2h_destroy": (None, [VP]),
            "c2h_last_error": (C.c_char_p, [VP]),
            "c2h_upload_tensor": (C.c_int, [VP, I32, I32, I32, I64, I64, VP, C.c_size_t]),
            "c2h_set_token_ids": (C.c_int, [VP, I32, VP, I32]),
            "c2h_forward": (C.c_int, [VP, I32, I32, VP]),
            "c2h_prefill": (C.c_int, [VP, VP, I32, I32, VP]),
            "c2h_logits": (C.c_int, [VP, VP]),
            "c2h_step": (C.c_int, [VP, I32, C.c_float, I32, I32, C.POINTER(I32)]),
            "c2h_restore_normx": (C.c_int, [VP]),
            "c2h_get_normx": (C.c_int, [VP, VP]),
            "c2h_get_kv": (C.c_int, [VP, I32, I32, I32, I32, VP]),
            "c2h_set_kv": (C.c_int, [VP, I32, I32, I32, I32, I32, VP]),
            "c2h_set_seq": (C.c_int, [VP, I32]),
            "c2h_get_token_ids": (C.c_int, [VP, I32, I32, VP]),
            "c2h_get_seq": (C.c_int, [VP, C.POINTER(I32)]),
            "c2h_quantize_q8k": (C.c_int, [VP, VP, I32, VP]),
            "c2h_quantize_q8k_noalloc": (C.c_int, [VP, VP, I32, VP]),
            "c2h_time_layer_kernel": (C.c_int, [VP, I32, I32, I32, C.POINTER(C.c_float)]),
            "c2h_time_gemv": (C.c_int, [VP, I32, VP, VP, I32, I32, I32, I64, C.POINTER(C.c_float)]),
            "c2h_time_quantize_q8k": (C.c_int, [VP, VP, I32, I32, I64, C.POINTER(C.c_float)]),
            "c2h_gemv": (C.c_int, [VP, I32, VP, VP, I32, I32, VP, VP]),
            "c2h_packed_size": (C.c_size_t, [I32, I64, I64]),
            "c2h_pack_weights": (C.c_int, [I32, I64, I64, VP, C.c_size_t, VP, C.c_size_t]),
            "c2h_quantize_q8k_dev": (C.c_int, [VP, VP, I32, VP]),
            "c2h_gemv_dev": (C.c_int, [VP, I32, VP, VP, I32, I32, VP, VP]),
            "c2h_sync": (C.c_int, [VP]),
            "c2h_time_vocab": (C.c_int, [VP, I32, I32, I32, C.POINTER(C.c_float)]),
            "c2h_copy_bench": (C.c_int, [VP, C.c_int64, I32, C.POINTER(C.c_float)]),
            "c2h_launch_floor": (C.c_int, [VP, I32, I32, I32, C.POINTER(C.c_float)]),
            "c2h_time_producer_consumer": (C.c_int, [VP, I32, I32, I32, I32, I32, I32, C.POINTER(C.c_float),
                                                     C.POINTER(C.c_float)]),
            "c2h_check_rms_scale": (C.c_int, [VP, C.c_uint32, C.c_uint64, C.POINTER(C.c_uint64),
                                              C.POINTER(C.c_uint32)]),
            "c2h_time_steps": (C.c_int, [VP, I32, I32, C.c_float, I32, I32, C.POINTER(C.c_float)]),
            "c2h_gemv_f32": (C.c_int, [VP, I32, VP, VP, I32, I32, VP]),
            "c2h_gemv_f32_dev": (C.c_int, [VP, I32, VP, VP, I32, I32, VP]),
            "c2h_logits_ids": (C.c_int, [VP, VP, I32, VP]),
            "c2h_logits_ids_dev": (C.c_int, [VP, VP, I32, VP]),
            "c2h_time_dot_rows": (C.c_int, [VP, I32, VP, VP, I32, I32, VP, I32, I32, C.c_int64, VP,
                                            C.POINTER(C.c_float)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return C.c_void_p(a.ctypes.data)


class Ctx:
    """One c2h context (one device stream, its buffers)."""

    def __init__(self, desc: ModelDesc | None = None, device: int = 0):
        L = lib()
        h = VP()
        rc = L.c2h_create(C.byref(desc) if desc is not None else None, device, C.byref(h))
        if rc != C2H_OK:
            raise C2hError(rc, (L.c2h_last_error(None) or b"").decode())
        self.h = h
        self.desc = desc

    def _chk(self, rc: int):
        if rc != C2H_OK:
            raise C2hError(rc, (lib().c2h_last_error(self.h) or b"").decode())

    def close(self):
        if getattr(self, "h", None):
            lib().c2h_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # ---- model
    def upload(self, layer: int, role: str, ggml_type: int, rows: int, cols: int, data: np.ndarray):
        a = np.ascontiguousarray(data)
        self._chk(lib().c2h_upload_tensor(self.h, layer, ROLE[role], ggml_type, rows, cols, _p(a), a.nbytes))

    def set_token_ids(self, pos0: int, ids):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        self._chk(lib().c2h_set_token_ids(self.h, pos0, _p(a), len(a)))

    def forward(self, token: int, pos: int, want_normx: bool = True):
        out = np.empty(self.desc.n_embd, np.float32) if want_normx else None
        self._chk(lib().c2h_forward(self.h, token, pos, _p(out) if want_normx else None))
        return out

    def prefill(self, tokens, pos0: int, want_normx: bool = True):
        """Engine.IngestFrom's Forward loop for all tokens at once (batched)."""
        toks = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
        out = np.empty(self.desc.n_embd, np.float32) if want_normx else None
        self._chk(lib().c2h_prefill(self.h, _p(toks), len(toks), pos0, _p(out) if want_normx else None))
        return out

    def logits(self) -> np.ndarray:
        out = np.empty(self.desc.n_vocab, np.float32)
        self._chk(lib().c2h_logits(self.h, _p(out)))
        return out

    def logits_ids(self, ids, out: np.ndarray | None = None) -> np.ndarray:
        """engine.ComputeLogits with a target list: out[id] for each id in
        range; the other entries of out keep their values."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        if out is None:
            out = np.zeros(self.desc.n_vocab, np.float32)
        assert out.dtype == np.float32 and out.flags.c_contiguous and len(out) == self.desc.n_vocab
        self._chk(lib().c2h_logits_ids(self.h, _p(ids) if len(ids) else None, len(ids), _p(out)))
        return out

    def step(self, pos: int, penalty: float, im_end: int, eos: int) -> int:
        t = I32()
        self._chk(lib().c2h_step(self.h, pos, penalty, im_end, eos, C.byref(t)))
        return t.value

    def restore_normx(self):
        self._chk(lib().c2h_restore_normx(self.h))

    def sync(self):
        """Wait for all work queued on the context (a step's call returns with
        its token while the forward of that token still runs)."""
        self._chk(lib().c2h_sync(self.h))

    def normx(self) -> np.ndarray:
        out = np.empty(self.desc.n_embd, np.float32)
        self._chk(lib().c2h_get_normx(self.h, _p(out)))
        return out

    def kv(self, which: int, layer: int, kv_head: int, n: int) -> np.ndarray:
        out = np.empty((n, self.desc.head_dim), np.float32)
        self._chk(lib().c2h_get_kv(self.h, which, layer, kv_head, n, _p(out)))
        return out

    def set_kv(self, which: int, layer: int, kv_head: int, pos0: int, data: np.ndarray):
        a = np.ascontiguousarray(data, dtype=np.float32).reshape(-1, self.desc.head_dim)
        self._chk(lib().c2h_set_kv(self.h, which, layer, kv_head, pos0, a.shape[0], _p(a)))

    def token_ids(self, pos0: int, n: int) -> np.ndarray:
        out = np.empty(n, np.int32)
        self._chk(lib().c2h_get_token_ids(self.h, pos0, n, _p(out)))
        return out

    @property
    def seq_len(self) -> int:
        n = I32()
        self._chk(lib().c2h_get_seq(self.h, C.byref(n)))
        return n.value

    def set_seq(self, n: int):
        self._chk(lib().c2h_set_seq(self.h, n))

    def time_vocab(self, iters: int, pos: int, in_step: int = 1) -> float:
        ms = C.c_float()
        self._chk(lib().c2h_time_vocab(self.h, iters, pos, int(in_step), C.byref(ms)))
        return ms.value

    def copy_bench(self, nbytes: int, reps: int) -> float:
        ms = C.c_float()
        self._chk(lib().c2h_copy_bench(self.h, nbytes, reps, C.byref(ms)))
        return ms.value

    def launch_floor(self, n=240, grid=256, reps=5):
        """Device µs per kernel of a graph of n dependent empty launches."""
        us = C.c_float()
        self._chk(lib().c2h_launch_floor(self.h, n, grid, reps, C.byref(us)))
        return us.value

    def time_producer_consumer(self, n_prod: int, n_cons: int, work: int = 0, n_launch: int = 100,
                               reps: int = 5, proto: int = 0) -> tuple[float, float]:
        """(µs per fused producer->consumer launch, µs per split launch pair)
        (c2h_time_producer_consumer; proto 0 counters, 1 tagged outputs)."""
        f, sp = C.c_float(), C.c_float()
        self._chk(lib().c2h_time_producer_consumer(self.h, n_prod, n_cons, work, n_launch, reps, proto, C.byref(f),
                                                   C.byref(sp)))
        return f.value, sp.value

    def check_rms_scale(self, lo: int, hi: int) -> tuple[int, int]:
        """(mismatches, lowest mismatching bit pattern) of the kernels' RMSNorm
        scale against the IEEE sqrt and division over patterns [lo, hi)."""
        bad, first = C.c_uint64(), C.c_uint32()
        self._chk(lib().c2h_check_rms_scale(self.h, lo, hi, C.byref(bad), C.byref(first)))
        return bad.value, first.value

    def time_steps(self, pos: int, iters: int, penalty: float, im_end: int, eos: int) -> float:
        ms = C.c_float()
        self._chk(lib().c2h_time_steps(self.h, pos, iters, penalty, im_end, eos, C.byref(ms)))
        return ms.value

    KERNELS = ("qkv", "attn", "attn_out", "ffn_in", "ffn_out", "final_norm", "attn_block",
               "attn_oproj", "ffn_block")  # C2H_KERNEL_*

    def time_layer_kernel(self, kernel: str, iters: int, captured: bool = False) -> float:
        """ms per launch of one decoder-layer kernel (c2h_time_layer_kernel):
        eager launches back to back (paced by the GPU), or one captured graph."""
        ms = C.c_float()
        self._chk(lib().c2h_time_layer_kernel(self.h, self.KERNELS.index(kernel), iters, int(captured), C.byref(ms)))
        return ms.value

    def time_gemv(self, ggml_type: int, w: np.ndarray, xq: np.ndarray, rows: int, cols: int, iters: int,
                  rotate_bytes: int = 0) -> float:
        w = np.ascontiguousarray(w)
        xq = np.ascontiguousarray(xq)
        ms = C.c_float()
        self._chk(lib().c2h_time_gemv(self.h, ggml_type, _p(w), _p(xq), rows, cols, iters, rotate_bytes,
                                      C.byref(ms)))
        return ms.value

    def time_quantize_q8k(self, x: np.ndarray, iters: int, rotate_bytes: int = 0) -> float:
        x = np.ascontiguousarray(x, dtype=np.float32)
        ms = C.c_float()
        self._chk(lib().c2h_time_quantize_q8k(self.h, _p(x), len(x), iters, rotate_bytes, C.byref(ms)))
        return ms.value

    # ---- operators (host buffers)
    def quantize_q8k(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros((len(x) // 256) * 292, np.uint8)
        self._chk(lib().c2h_quantize_q8k(self.h, _p(x), len(x), _p(out)))
        return out

    def quantize_q8k_noalloc(self, x: np.ndarray) -> np.ndarray:
        """c2h_quantize_q8k through the entry point that allocates nothing."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros((len(x) // 256) * 292, np.uint8)
        self._chk(lib().c2h_quantize_q8k_noalloc(self.h, _p(x), len(x), _p(out)))
        return out

    def gemv(self, ggml_type: int, w: np.ndarray, xq: np.ndarray, rows: int, cols: int, want_isums: bool = False):
        w = np.ascontiguousarray(w)
        xq = np.ascontiguousarray(xq)
        y = np.empty(rows, np.float32)
        isums = None
        if want_isums and ggml_type == Q4_K:
            isums = np.empty((rows, cols // 256, 8), np.int32)
        elif want_isums and ggml_type == Q6_K:
            isums = np.empty((rows, cols // 256), np.int32)
        self._chk(lib().c2h_gemv(self.h, ggml_type, _p(w), _p(xq), rows, cols, _p(y),
                                 _p(isums) if isums is not None else None))
        return (y, isums) if want_isums else y


    def time_dot_rows(self, ggml_type: int, w: np.ndarray, x: np.ndarray, rows: int, cols: int, ids=None,
                      n: int | None = None, iters: int = 20, flush_bytes: int = 0):
        """(ms per launch, results) of the float-x row dots: rows 0..n-1, or
        the listed ids."""
        w = np.ascontiguousarray(w)
        x = np.ascontiguousarray(x, dtype=np.float32)
        if ids is not None:
            ids = np.ascontiguousarray(ids, dtype=np.int32)
            n = len(ids)
        n = rows if n is None else n
        y = np.empty(n, np.float32)
        ms = C.c_float()
        self._chk(lib().c2h_time_dot_rows(self.h, ggml_type, _p(w), _p(x), rows, cols,
                                          _p(ids) if ids is not None else None, n, iters, flush_bytes, _p(y),
                                          C.byref(ms)))
        return ms.value, y

    def gemv_f32(self, ggml_type: int, w: np.ndarray, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
        """engine.DispatchGEMV without a pool: y = W·x on f32 x."""
        w = np.ascontiguousarray(w)
        x = np.ascontiguousarray(x, dtype=np.float32)
        assert len(x) >= cols
        y = np.empty(rows, np.float32)
        self._chk(lib().c2h_gemv_f32(self.h, ggml_type, _p(w), _p(x), rows, cols, _p(y)))
        return y


def packed_size(ggml_type: int, rows: int, cols: int) -> int:
    return lib().c2h_packed_size(ggml_type, rows, cols)


def pack_weights(ggml_type: int, rows: int, cols: int, native: np.ndarray) -> np.ndarray:
    native = np.ascontiguousarray(native, dtype=np.uint8)
    out = np.zeros(packed_size(ggml_type, rows, cols), np.uint8)
    rc = lib().c2h_pack_weights(ggml_type, rows, cols, _p(native), native.nbytes, _p(out), out.nbytes)
    if rc != C2H_OK:
        raise C2hError(rc, "pack_weights")
    return out


def desc_from_gguf(gf, max_ctx: int = 16384) -> ModelDesc:
    """Dimensions as engine.LoadModel resolves them (engine/model.go:64-145):
    qwen2.* keys, then qwen3.*, then the Qwen2.5-0.5B defaults."""
    def u32(k2, k3, dflt):
        return gf.get_u32(k2) or gf.get_u32(k3) or dflt

    def f32(k2, k3, dflt):
        return gf.get_f32(k2) or gf.get_f32(k3) or dflt

    d = ModelDesc()
    d.n_embd = u32("qwen2.embedding_length", "qwen3.embedding_length", 896)
    d.n_layers = u32("qwen2.block_count", "qwen3.block_count", 24)
    d.n_heads = u32("qwen2.attention.head_count", "qwen3.attention.head_count", 14)
    d.n_kv_heads = u32("qwen2.attention.head_count_kv", "qwen3.attention.head_count_kv", 2)
    d.n_ff = u32("qwen2.feed_forward_length", "qwen3.feed_forward_length", 4864)
    d.rope_theta = f32("qwen2.rope.freq_base", "qwen3.rope.freq_base", 1.0e6)
    d.rms_eps = f32("qwen2.attention.layer_norm_rms_epsilon", "qwen3.attention.layer_norm_rms_epsilon", 1e-6)
    d.head_dim = d.n_embd // d.n_heads
    d.n_vocab = int(gf.tensor_map["token_embd.weight"].dims[1])
    d.max_ctx = max_ctx
    return d


def load_gguf_into(ctx: Ctx, gf) -> None:
    """Uploads every tensor engine/model.go:114-207 binds."""
    tm = gf.tensor_map

    def up(layer, role, ti):
        ctx.upload(layer, role, ti.ggml_type, ti.rows, ti.cols, np.asarray(ti.data))

    up(0, "TOKEN_EMBD", tm["token_embd.weight"])
    if "output.weight" in tm:
        up(0, "OUTPUT", tm["output.weight"])
    up(0, "OUTPUT_NORM", tm["output_norm.weight"])
    for i in range(ctx.desc.n_layers):
        for suffix, role in LAYER_TENSORS.items():
            ti = tm.get(f"blk.{i}.{suffix}")
            if ti is not None:
                up(i, role, ti)
