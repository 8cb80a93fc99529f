"""A float64 Qwen2 decoder written from the model's mathematics, for pinning
the oracle's composed functions (orc_forward / orc_ingest_from /
orc_generate / orc_compute_logits).

It shares no code with the oracle.  Weights are dequantised to float64 by
tests/refdequant.py (itself checked against the reference's C dequantisers);
every matrix product, norm, rotation, softmax and activation is float64:

  x    = embedding row of the token (an id outside [0, V) embeds id 0,
         engine/model.go:222-224)
  per layer:
    n    = x / sqrt(mean(x^2) + eps) * attn_norm
    q,k,v = Wq n + bq, Wk n + bk, Wv n + bv
    (Qwen3: no biases; every head of q and of k divided by its own
     sqrt(mean(head^2) + eps) and scaled by attn_q_norm / attn_k_norm,
     engine/forward.go:80-91)
    rotate-half RoPE on every head: pair (i, i + hd/2) turned by
         pos * theta^(-2i/hd)
    per query head h, KV head h // (H/KVH): softmax(q.K^T / sqrt(hd)) V
    x   += Wo attn
    n    = RMSNorm(x) * ffn_norm
    x   += Wd (silu(Wg n) * (Wu n))
  normX = RMSNorm(x) * output_norm;  logits = Wout normX

One property of the reference's arithmetic is part of its model and is
kept: a Q4_K / Q6_K matrix multiplies the Q8_K quantisation of its input
(engine/pool.go:123-125), the first floor(cols/256)*256 elements rounded
to int8 per 256-element block, q = trunc(x*(127/amax) +- 0.5) with
d = amax/127 (internal/simd/c2_quantize_q8_k_gen.go:22-90).  That rounding
changes results by ~1/127 of a block's amax, far above the 1e-3 tolerance
this reference is compared at, so it is applied here too (to the float64
activations rounded to f32).  Q5_0 / Q8_0 matrices take the f32 vector
itself (engine/model.go:250-270).
"""
from __future__ import annotations

import numpy as np

from c2slm_amd import gguf as G
from tests import refdequant as R


def _dequant_matrix(ti) -> np.ndarray:
    """[rows, used_cols] float64 of a quantised tensor: K-quants cover
    floor(cols/256) super-blocks per row, Q8_0/Q5_0 floor(cols/32) blocks."""
    cols, rows = int(ti.dims[0]), int(ti.dims[1])
    raw = np.frombuffer(ti.data, np.uint8)
    t = ti.ggml_type
    if t == G.Q4_K:
        nb = cols // 256
        return R.dequant_q4k_f64(raw[:rows * nb * 144]).reshape(rows, nb * 256)
    if t == G.Q6_K:
        nb = cols // 256
        return R.dequant_q6k_f64(raw[:rows * nb * 210]).reshape(rows, nb * 256)
    if t == G.Q8_0:
        nb = cols // 32
        return R.dequant_q8_0_f64(raw[:rows * nb * 34]).reshape(rows, nb * 32)
    if t == G.Q5_0:
        nb = cols // 32
        return R.dequant_q5_0_f64(raw[:rows * nb * 22]).reshape(rows, nb * 32)
    if t == G.F32:
        return np.frombuffer(ti.data, "<f4").astype(np.float64).reshape(rows, cols)
    raise ValueError(f"type {t}")


def q8k_round_trip(x: np.ndarray) -> np.ndarray:
    """The Q8_K quantisation of x (f32) dequantised: d*q per element over the
    whole 256-element blocks."""
    x = np.asarray(x, np.float32)
    nb = len(x) // 256
    out = np.zeros(nb * 256, np.float64)
    with np.errstate(all="ignore"):
        for b in range(nb):
            blk = x[b * 256:(b + 1) * 256]
            amax = np.fmax.reduce(np.abs(blk))  # NaN never wins the reference's '>' scan
            if not amax > 0:
                continue
            d = np.float32(amax / np.float32(127.0))
            isc = np.float32(np.float32(127.0) / amax)
            t = (blk * isc).astype(np.float32)
            r = (t + np.where(t >= 0, np.float32(0.5), np.float32(-0.5))).astype(np.float32)
            q = np.clip(np.trunc(r), -127, 127)
            out[b * 256:(b + 1) * 256] = np.float64(d) * q
    return out


class Qwen2F64:
    def __init__(self, gf: G.GGUFFile, max_ctx: int = 1024):
        arch = gf.metadata.get("general.architecture", "qwen2")
        u32 = lambda k: gf.get_u32(f"{arch}.{k}")
        self.E = u32("embedding_length")
        self.L = u32("block_count")
        self.H = u32("attention.head_count")
        self.KVH = u32("attention.head_count_kv")
        self.F = u32("feed_forward_length")
        self.theta = float(np.float32(gf.get_f32(f"{arch}.rope.freq_base")))
        self.eps = float(np.float32(gf.get_f32(f"{arch}.attention.layer_norm_rms_epsilon")))
        self.hd = self.E // self.H
        tm = gf.tensor_map
        self.types = {}

        def mat(name):
            ti = tm[name]
            self.types[name] = ti.ggml_type
            return _dequant_matrix(ti)

        def vec(name):
            ti = tm.get(name)
            return None if ti is None else np.frombuffer(ti.data, "<f4").astype(np.float64)

        self.emb = mat("token_embd.weight")
        self.V = self.emb.shape[0]
        out_name = "output.weight" if "output.weight" in tm else "token_embd.weight"
        self.out = mat(out_name)
        self.out_type = tm[out_name].ggml_type
        self.out_norm = vec("output_norm.weight")
        self.layers = []
        for i in range(self.L):
            p = f"blk.{i}."
            ly = {k: mat(p + k + ".weight") for k in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate",
                                                      "ffn_up", "ffn_down")}
            ly["types"] = {k: tm[p + k + ".weight"].ggml_type for k in ly}
            for k in ("attn_norm", "ffn_norm"):
                ly[k] = vec(p + k + ".weight")
            for k in ("attn_q", "attn_k", "attn_v"):
                ly[k + ".bias"] = vec(p + k + ".bias")
            for k in ("attn_q_norm", "attn_k_norm"):
                ly[k] = vec(p + k + ".weight")
            self.layers.append(ly)
        self.max_ctx = max_ctx
        kv = self.KVH * self.hd
        self.K = np.zeros((self.L, max_ctx, kv))
        self.Vc = np.zeros((self.L, max_ctx, kv))
        self.normx = np.zeros(self.E)

    # -- Q8_K rows supplied by the oracle (flip-free comparison)
    def feed_q8k(self, trace: np.ndarray) -> None:
        """Queue the oracle's Q8_K rows (in its call order).  Each K-quant
        matvec then takes the next row -- after checking that it is a correct
        Q8_K rounding of this model's own float64 activation: d = amax/127
        and every |q*d - x| <= d/2 (up to an f32/f64 difference of the
        activations of 1e-4 of the block's amax).  Only the direction of a rounding whose input sits
        within that difference of a .5 boundary is taken from the oracle;
        without this a single such flip moves the outputs by ~1e-3."""
        self._q8k = np.asarray(trace, np.uint8)
        self._q8k_off = 0
        self.q8k_checked = 0

    def q8k_left(self) -> int:
        return len(self._q8k) - self._q8k_off if getattr(self, "_q8k", None) is not None else 0

    def _q8k_row(self, x: np.ndarray, nb: int) -> np.ndarray:
        n = nb * 292
        if getattr(self, "_q8k", None) is None:
            return q8k_round_trip(x.astype(np.float32))
        if self._q8k_off + n > len(self._q8k):
            raise AssertionError("the oracle quantised fewer Q8_K rows than the model needs")
        raw = self._q8k[self._q8k_off:self._q8k_off + n].reshape(nb, 292)
        self._q8k_off += n
        d = raw[:, 0:4].copy().view("<f4")[:, 0].astype(np.float64)
        q = raw[:, 4:260].view(np.int8).astype(np.int64)
        bs = raw[:, 260:292].copy().view("<i2").astype(np.int64)
        xb = np.asarray(x, np.float64)[:nb * 256].reshape(nb, 256)
        amax = np.max(np.abs(xb), axis=1)
        for b in range(nb):
            if amax[b] == 0:
                assert d[b] == 0 and not q[b].any(), "zero block"
                continue
            if amax[b] < 1e-30:  # f32 underflow territory: contributes < 1e-28 to any output
                assert np.all(np.abs(q[b] * d[b] - xb[b]) <= 1e-30), ("negligible block", b)
                continue
            assert abs(d[b] - amax[b] / 127) <= 1e-4 * amax[b] / 127, ("Q8_K d", b, d[b], amax[b] / 127)
            err = np.abs(q[b] * d[b] - xb[b])
            # half a step, plus an f32/f64 drift of the activation up to 1e-4 of the block's amax
            assert np.all(err <= 0.5 * d[b] + 1e-4 * amax[b]), ("Q8_K rounding", b, err.max() / d[b])
            assert np.array_equal(bs[b], q[b].reshape(16, 16).sum(axis=1)), ("Q8_K bsums", b)
        self.q8k_checked += nb
        return (d[:, None] * q).reshape(-1)

    # -- building blocks, float64
    def _rmsnorm(self, x, w):
        return x / np.sqrt(np.mean(x * x) + self.eps) * w

    def _head_norm(self, v, w):
        hd = self.hd
        return np.concatenate([self._rmsnorm(v[i:i + hd], w) for i in range(0, len(v), hd)])

    def _matvec(self, w, t, x):
        if t in (G.Q4_K, G.Q6_K):
            return w @ self._q8k_row(x, w.shape[1] // 256)
        return w @ x.astype(np.float32).astype(np.float64)[:w.shape[1]]

    def _rope(self, v, pos):
        hd, half = self.hd, self.hd // 2
        i = np.arange(half, dtype=np.float64)
        ang = pos * self.theta ** (-2.0 * i / hd)
        c, s = np.cos(ang), np.sin(ang)
        v = v.reshape(-1, hd).copy()
        x0, x1 = v[:, :half].copy(), v[:, half:].copy()
        v[:, :half] = x0 * c - x1 * s
        v[:, half:] = x0 * s + x1 * c
        return v.reshape(-1)

    def forward(self, tok: int, pos: int) -> np.ndarray:
        E, H, KVH, hd = self.E, self.H, self.KVH, self.hd
        x = self.emb[tok if 0 <= tok < self.V else 0].copy()
        for li, ly in enumerate(self.layers):
            t = ly["types"]
            n = self._rmsnorm(x, ly["attn_norm"])
            q = self._matvec(ly["attn_q"], t["attn_q"], n)
            k = self._matvec(ly["attn_k"], t["attn_k"], n)
            v = self._matvec(ly["attn_v"], t["attn_v"], n)
            for name, arr in (("attn_q", q), ("attn_k", k), ("attn_v", v)):
                b = ly[name + ".bias"]
                if b is not None:
                    arr += b
            if ly["attn_q_norm"] is not None:
                q = self._head_norm(q, ly["attn_q_norm"])
            if ly["attn_k_norm"] is not None:
                k = self._head_norm(k, ly["attn_k_norm"])
            q, k = self._rope(q, pos), self._rope(k, pos)
            self.K[li, pos], self.Vc[li, pos] = k, v
            att = np.zeros(E)
            rep = H // KVH
            for h in range(H):
                g = h // rep
                Kh = self.K[li, :pos + 1, g * hd:(g + 1) * hd]
                Vh = self.Vc[li, :pos + 1, g * hd:(g + 1) * hd]
                sc = Kh @ q[h * hd:(h + 1) * hd] / np.sqrt(hd)
                p = np.exp(sc - sc.max())
                p /= p.sum()
                att[h * hd:(h + 1) * hd] = p @ Vh
            x = x + self._matvec(ly["attn_output"], t["attn_output"], att)
            n = self._rmsnorm(x, ly["ffn_norm"])
            g = self._matvec(ly["ffn_gate"], t["ffn_gate"], n)
            u = self._matvec(ly["ffn_up"], t["ffn_up"], n)
            with np.errstate(over="ignore"):  # exp(-g) = inf gives silu(g) = -0
                h_ = g / (1.0 + np.exp(-g)) * u
            x = x + self._matvec(ly["ffn_down"], t["ffn_down"], h_)
        self.normx = self._rmsnorm(x, self.out_norm)
        return self.normx

    def logits(self, normx=None) -> np.ndarray:
        nx = self.normx if normx is None else np.asarray(normx, np.float64)
        return self._matvec(self.out, self.out_type, nx)

    @staticmethod
    def penalise(logits: np.ndarray, window_ids, im_end: int, eos: int, penalty: float) -> np.ndarray:
        """c2slm.go:157-168: each occurrence of an id in the window divides a
        positive logit by the penalty and multiplies a non-positive one."""
        lg = np.array(logits, np.float64)
        for t in window_ids:
            if t < 0 or t >= len(lg) or t == im_end or t == eos:
                continue
            lg[t] = lg[t] / penalty if lg[t] > 0 else lg[t] * penalty
        return lg


# ------------------------------------------------------------ pin models

def pack_q4k_scales(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """The 12 scale bytes holding eight 6-bit scales and mins per block
    ([n,8] each), the inverse of the unpacking in
    c2_tensor_dot_q4_k_q8_k_gen.go:47-61."""
    sc = np.asarray(sc, np.int64)
    m = np.asarray(m, np.int64)
    out = np.zeros((len(sc), 12), np.uint8)
    for j in range(4):
        out[:, j] = (sc[:, j] & 63) | ((sc[:, j + 4] >> 4) << 6)
        out[:, j + 4] = (m[:, j] & 63) | ((m[:, j + 4] >> 4) << 6)
        out[:, j + 8] = (sc[:, j + 4] & 15) | ((m[:, j + 4] & 15) << 4)
    return out


def centered_q4_k(rng: np.random.Generator, n_blocks: int) -> np.ndarray:
    """Q4_K blocks whose weights d*sc*q - dmin*m are centred on zero: dmin = d
    and m = round(7.5*sc) for scales sc in [1, 8] (q is uniform on [0, 15])."""
    blk = rng.integers(0, 256, size=(n_blocks, 144), dtype=np.uint8)
    d = rng.uniform(0.002, 0.01, n_blocks).astype(np.float16).view(np.uint16)
    blk[:, 0:2] = d.view(np.uint8).reshape(n_blocks, 2)
    blk[:, 2:4] = blk[:, 0:2]
    sc = rng.integers(1, 9, size=(n_blocks, 8))
    blk[:, 4:16] = pack_q4k_scales(sc, np.rint(7.5 * sc).astype(np.int64))
    return blk.reshape(-1)


def write_pin_model(path: str, shape: G.ModelShape, seed: int, bias_std: float = 1.0,
                    norm_lo: float = 0.5, norm_hi: float = 1.5) -> None:
    """A random-init GGUF for pinning the composition: centred Q4_K weights
    (the bench's Q4_K draw is all-positive, mean weight ~ +1, so outputs are
    small differences of large sums), every norm weight vector distinct
    (U(norm_lo, norm_hi)), biases N(0, bias_std^2) comparable to the
    projections, so a swapped norm vector or a dropped bias shows.  A
    shape with arch "qwen3" has no biases and distinct attn_q_norm /
    attn_k_norm vectors (U(norm_lo, norm_hi), head_dim long)."""
    rng = np.random.default_rng(seed)
    E, F, V, L = shape.n_embd, shape.n_ff, shape.n_vocab, shape.n_layers
    KV = shape.n_kv_heads * shape.head_dim
    tensors = []
    synth = dict(G.SYNTH)
    synth[G.Q4_K] = centered_q4_k

    def quant(name, tt, rows, cols):
        dims = [cols, rows]
        size = G.tensor_byte_size(tt, dims)
        tensors.append((name, dims, tt, synth[tt](rng, size // G.BLOCK[tt][1])))

    def f32(name, values):
        tensors.append((name, [len(values)], G.F32, np.asarray(values, dtype="<f4").view(np.uint8)))

    qwen3 = shape.arch == "qwen3"
    quant("token_embd.weight", shape.t_embd, V, E)
    f32("output_norm.weight", rng.uniform(norm_lo, norm_hi, E))
    if shape.t_out is not None:
        quant("output.weight", shape.t_out, V, E)
    for i in range(L):
        f32(f"blk.{i}.attn_norm.weight", rng.uniform(norm_lo, norm_hi, E))
        quant(f"blk.{i}.attn_q.weight", shape.t_q, E, E)
        if not qwen3:
            f32(f"blk.{i}.attn_q.bias", rng.normal(0.0, bias_std, E))
        quant(f"blk.{i}.attn_k.weight", shape.t_k, KV, E)
        if not qwen3:
            f32(f"blk.{i}.attn_k.bias", rng.normal(0.0, bias_std, KV))
        quant(f"blk.{i}.attn_v.weight", shape.t_v, KV, E)
        if not qwen3:
            f32(f"blk.{i}.attn_v.bias", rng.normal(0.0, bias_std, KV))
        else:
            f32(f"blk.{i}.attn_q_norm.weight", rng.uniform(norm_lo, norm_hi, shape.head_dim))
            f32(f"blk.{i}.attn_k_norm.weight", rng.uniform(norm_lo, norm_hi, shape.head_dim))
        quant(f"blk.{i}.attn_output.weight", shape.t_o, E, E)
        f32(f"blk.{i}.ffn_norm.weight", rng.uniform(norm_lo, norm_hi, E))
        quant(f"blk.{i}.ffn_gate.weight", shape.t_gate, F, E)
        quant(f"blk.{i}.ffn_up.weight", shape.t_up, F, E)
        quant(f"blk.{i}.ffn_down.weight", shape.t_down, E, F)
    a = shape.arch
    md = [
        ("general.architecture", G.T_STR, a),
        ("general.alignment", G.T_U32, 32),
        (f"{a}.block_count", G.T_U32, L),
        (f"{a}.embedding_length", G.T_U32, E),
        (f"{a}.feed_forward_length", G.T_U32, F),
        (f"{a}.attention.head_count", G.T_U32, shape.n_heads),
        (f"{a}.attention.head_count_kv", G.T_U32, shape.n_kv_heads),
        (f"{a}.rope.freq_base", G.T_F32, shape.rope_theta),
        (f"{a}.attention.layer_norm_rms_epsilon", G.T_F32, shape.rms_eps),
        ("tokenizer.ggml.model", G.T_STR, "gpt2"),
        ("tokenizer.ggml.tokens", G.T_ARR, (G.T_STR, G.token_list(V))),
    ]
    G.write_gguf(path, md, tensors)
