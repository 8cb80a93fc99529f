"""GGUF v3 files for the decode path: a reader with the reference's parse rules
and a seeded writer for random-init Qwen2.5-0.5B-shaped models.

Reader rules follow gguf/reader.go: magic 0x46554747, versions 2-3 only
(:401-413), metadata value types (:308-392), default alignment 32 overridable
by general.alignment (:443-451), tensor data offset aligned (:491-495) and
payload sizes from tensorByteSize (:513-546), i.e. Q4_K (n/256)*144,
Q6_K (n/256)*210, Q8_0 (n/32)*34, F32 n*4 — floor division on the element
count, as the reference does.

The writer emits exactly what engine/model.go:58-210 binds (qwen2.* keys,
blk.N.* tensor names, dims [cols, rows]) plus the tokenizer token list that
tokenizer/bpe.go:30-33 requires.
"""
from __future__ import annotations

import dataclasses
import struct
from typing import Any, Dict, List, Optional, Tuple

import numpy as np

GGUF_MAGIC = 0x46554747

# ggml tensor types (gguf/reader.go:21-37)
F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 6, 8, 12, 14

# metadata value types (gguf/reader.go:73-87)
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)

BLOCK = {Q4_K: (256, 144), Q6_K: (256, 210), Q8_0: (32, 34), Q5_0: (32, 22), Q4_0: (32, 18)}


def tensor_byte_size(ggml_type: int, dims) -> int:
    """gguf/reader.go:513-546."""
    if len(dims) == 0:
        return 0
    n = 1
    for d in dims:
        n *= int(d)
    if ggml_type == F32:
        return n * 4
    if ggml_type == F16:
        return n * 2
    if ggml_type in BLOCK:
        qk, bs = BLOCK[ggml_type]
        return (n // qk) * bs
    return n * 4


def row_bytes(ggml_type: int, cols: int) -> int:
    """Row stride the reference uses for a quantized row of `cols` inputs:
    (cols / QK) * blockSize with integer division (tensor/ops.go:26,78,121,183)."""
    qk, bs = BLOCK[ggml_type]
    return (cols // qk) * bs


@dataclasses.dataclass
class TensorInfo:
    name: str
    dims: List[int]
    ggml_type: int
    offset: int
    data: Optional[np.ndarray] = None  # uint8 view of the payload

    @property
    def cols(self) -> int:
        return int(self.dims[0])

    @property
    def rows(self) -> int:
        n = 1
        for d in self.dims[1:]:
            n *= int(d)
        return n


class GGUFFile:
    """Memory-mapped GGUF file parsed like gguf/reader.go:394-510."""

    def __init__(self, path: str):
        self.path = path
        self.mm = np.memmap(path, dtype=np.uint8, mode="r")
        self.metadata: Dict[str, Any] = {}
        self.tensors: List[TensorInfo] = []
        self.tensor_map: Dict[str, TensorInfo] = {}
        self._parse()

    # -- low-level reads ----------------------------------------------------
    def _rd(self, fmt: str):
        size = struct.calcsize(fmt)
        if self.pos + size > len(self.mm):
            raise EOFError("unexpected EOF")
        v = struct.unpack_from(fmt, self.mm, self.pos)[0]
        self.pos += size
        return v

    def _rd_str(self) -> str:
        n = self._rd("<Q")
        if self.pos + n > len(self.mm):
            raise EOFError("unexpected EOF")
        s = bytes(self.mm[self.pos:self.pos + n]).decode("utf-8", errors="surrogateescape")
        self.pos += n
        return s

    def _rd_value(self, vt: int):
        scalar = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i",
                  T_F32: "<f", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}
        if vt in scalar:
            return self._rd(scalar[vt])
        if vt == T_BOOL:
            return self._rd("<B") != 0
        if vt == T_STR:
            return self._rd_str()
        if vt == T_ARR:
            et = self._rd("<I")
            cnt = self._rd("<Q")
            return [self._rd_value(et) for _ in range(cnt)]
        raise ValueError(f"unknown metadata value type: {vt}")

    def _parse(self):
        self.pos = 0
        magic = self._rd("<I")
        if magic != GGUF_MAGIC:
            raise ValueError(f"invalid GGUF magic: 0x{magic:08x}")
        version = self._rd("<I")
        if version < 2 or version > 3:
            raise ValueError(f"unsupported GGUF version {version} (only v2/v3 supported)")
        self.version = version
        n_tensors = self._rd("<Q")
        n_kv = self._rd("<Q")
        for _ in range(n_kv):
            key = self._rd_str()
            vt = self._rd("<I")
            self.metadata[key] = self._rd_value(vt)
        align = 32
        a = self.metadata.get("general.alignment")
        if isinstance(a, int) and not isinstance(a, bool):
            align = a
        for _ in range(n_tensors):
            name = self._rd_str()
            nd = self._rd("<I")
            dims = [self._rd("<Q") for _ in range(nd)]
            tt = self._rd("<I")
            off = self._rd("<Q")
            ti = TensorInfo(name, dims, tt, off)
            self.tensors.append(ti)
            self.tensor_map[name] = ti
        pad = self.pos % align
        if pad:
            self.pos += align - pad
        self.data_offset = self.pos
        for ti in self.tensors:
            start = self.data_offset + ti.offset
            size = tensor_byte_size(ti.ggml_type, ti.dims)
            if start + size > len(self.mm):
                raise ValueError(f"tensor[{ti.name}] data out of range")
            ti.data = self.mm[start:start + size]

    def get_u32(self, key: str) -> int:
        v = self.metadata.get(key)
        return int(v) if isinstance(v, int) and not isinstance(v, bool) else 0

    def get_f32(self, key: str) -> float:
        v = self.metadata.get(key)
        return float(v) if isinstance(v, float) else 0.0


# ---------------------------------------------------------------- writer


def _w_str(buf: bytearray, s: str):
    b = s.encode("utf-8")
    buf += struct.pack("<Q", len(b))
    buf += b


def _w_kv(buf: bytearray, key: str, vt: int, value):
    _w_str(buf, key)
    buf += struct.pack("<I", vt)
    if vt == T_U32:
        buf += struct.pack("<I", value)
    elif vt == T_F32:
        buf += struct.pack("<f", value)
    elif vt == T_STR:
        _w_str(buf, value)
    elif vt == T_ARR:
        et, items = value
        buf += struct.pack("<IQ", et, len(items))
        if et == T_STR:
            for it in items:
                _w_str(buf, it)
        elif et == T_I32:
            buf += np.asarray(items, dtype="<i4").tobytes()
        elif et == T_F32:
            buf += np.asarray(items, dtype="<f4").tobytes()
        else:
            raise ValueError("unsupported array element type")
    else:
        raise ValueError("unsupported metadata type")


def write_gguf(path: str, metadata: List[tuple], tensors: List[tuple], alignment: int = 32):
    """metadata: [(key, vt, value)], tensors: [(name, dims, ggml_type, payload_bytes)]."""
    head = bytearray()
    head += struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), len(metadata))
    for key, vt, value in metadata:
        _w_kv(head, key, vt, value)
    offsets = []
    off = 0
    for name, dims, tt, payload in tensors:
        size = tensor_byte_size(tt, dims)
        if len(payload) != size:
            raise ValueError(f"{name}: payload {len(payload)} != {size}")
        off = (off + alignment - 1) // alignment * alignment
        offsets.append(off)
        off += size
    for (name, dims, tt, _), o in zip(tensors, offsets):
        _w_str(head, name)
        head += struct.pack("<I", len(dims))
        for d in dims:
            head += struct.pack("<Q", d)
        head += struct.pack("<IQ", tt, o)
    pad = (-len(head)) % alignment
    head += b"\0" * pad
    with open(path, "wb") as f:
        f.write(head)
        pos = 0
        for (name, dims, tt, payload), o in zip(tensors, offsets):
            if o > pos:
                f.write(b"\0" * (o - pos))
                pos = o
            mv = memoryview(np.ascontiguousarray(payload)).cast("B")
            f.write(mv)
            pos += len(mv)


# ------------------------------------------------------- synthetic weights


def _fp16_bits(x: np.ndarray) -> np.ndarray:
    return x.astype(np.float16).view(np.uint16)


def synth_q4_k(rng: np.random.Generator, n_blocks: int) -> np.ndarray:
    """Q4_K super-blocks: d, dmin fp16 U(0,0.01); 12 scale bytes uniform, so the
    six-bit scales and mins are U[0,63]; 4-bit quants U[0,15]."""
    blk = rng.integers(0, 256, size=(n_blocks, 144), dtype=np.uint8)
    d = _fp16_bits(rng.uniform(0.0, 0.01, n_blocks))
    dmin = _fp16_bits(rng.uniform(0.0, 0.01, n_blocks))
    blk[:, 0:2] = d.view(np.uint8).reshape(n_blocks, 2)
    blk[:, 2:4] = dmin.view(np.uint8).reshape(n_blocks, 2)
    return blk.reshape(-1)


def synth_q6_k(rng: np.random.Generator, n_blocks: int) -> np.ndarray:
    """Q6_K super-blocks: ql/qh uniform bytes, int8 scales U[-63,63], d fp16 U(0,0.01)."""
    blk = rng.integers(0, 256, size=(n_blocks, 210), dtype=np.uint8)
    blk[:, 192:208] = rng.integers(-63, 64, size=(n_blocks, 16), dtype=np.int8).view(np.uint8)
    d = _fp16_bits(rng.uniform(0.0, 0.01, n_blocks))
    blk[:, 208:210] = d.view(np.uint8).reshape(n_blocks, 2)
    return blk.reshape(-1)


def synth_q8_0(rng: np.random.Generator, n_blocks: int) -> np.ndarray:
    """Q8_0 blocks: d fp16 U(0,0.02), int8 quants U[-127,127]."""
    blk = np.empty((n_blocks, 34), dtype=np.uint8)
    blk[:, 2:] = rng.integers(-127, 128, size=(n_blocks, 32), dtype=np.int8).view(np.uint8)
    d = _fp16_bits(rng.uniform(0.0, 0.02, n_blocks))
    blk[:, 0:2] = d.view(np.uint8).reshape(n_blocks, 2)
    return blk.reshape(-1)


def synth_q5_0(rng: np.random.Generator, n_blocks: int) -> np.ndarray:
    """Q5_0 blocks: d fp16 U(0,0.02), the 32 high bits and the 16 nibble
    bytes uniform (5-bit quants U[0,31], offset -16)."""
    blk = rng.integers(0, 256, size=(n_blocks, 22), dtype=np.uint8)
    d = _fp16_bits(rng.uniform(0.0, 0.02, n_blocks))
    blk[:, 0:2] = d.view(np.uint8).reshape(n_blocks, 2)
    return blk.reshape(-1)


SYNTH = {Q4_K: synth_q4_k, Q6_K: synth_q6_k, Q8_0: synth_q8_0, Q5_0: synth_q5_0}


@dataclasses.dataclass
class ModelShape:
    n_layers: int = 24
    n_embd: int = 896
    n_heads: int = 14
    n_kv_heads: int = 2
    n_ff: int = 4864
    n_vocab: int = 151936
    rope_theta: float = 1.0e6
    rms_eps: float = 1.0e-6
    # Q4_K_M-style mix: Q4_K projections, Q6_K attn_v/ffn_down, Q8_0 embedding
    t_q: int = Q4_K
    t_k: int = Q4_K
    t_v: int = Q6_K
    t_o: int = Q4_K
    t_gate: int = Q4_K
    t_up: int = Q4_K
    t_down: int = Q6_K
    # per-layer ffn_down types, layer i taking entry i (None: t_down on every
    # layer), as a Q4_K_M file keeps Q6_K on some layers and Q4_K on others
    t_down_layers: Optional[Tuple[int, ...]] = None
    t_embd: int = Q8_0
    t_out: Optional[int] = None  # an untied output.weight of this type (None: tied to token_embd)
    # Qwen3 files: qwen3.* metadata keys, per-head attn_q_norm / attn_k_norm
    # weights (engine/forward.go:80-91) and no q/k/v biases
    arch: str = "qwen2"

    @property
    def head_dim(self) -> int:
        return self.n_embd // self.n_heads


QWEN05B = ModelShape()

# Qwen3-1.7B's dimensions (engine/model_config_test.go:18-33: 28 layers,
# 16/8 heads, head_dim 2048/16 = 128; FFN 6144, tied embedding) in the
# Q4_K_M mix of the other shapes.
QWEN3_1_7B = ModelShape(n_layers=28, n_embd=2048, n_heads=16, n_kv_heads=8, n_ff=6144, arch="qwen3")

# Qwen2.5-1.5B and Qwen2.5-3B dimensions (hidden 1536 / 2048, 12 / 16 query
# heads and 2 KV heads of 128, FFN 8960 / 11008, q/k/v biases, tied
# embedding), read by LoadModel's qwen2.* keys like the 0.5B
# (engine/model.go:64-145; head_dim = n_embd / n_heads), in the Q4_K_M mix.
QWEN25_1_5B = ModelShape(n_layers=28, n_embd=1536, n_heads=12, n_kv_heads=2, n_ff=8960)
QWEN25_3B = ModelShape(n_layers=36, n_embd=2048, n_heads=16, n_kv_heads=2, n_ff=11008)

# The published Qwen2.5-0.5B-Instruct Q4_K_M file's format mix: 896-column
# matrices cannot hold K-quant super-blocks whole, so q/k/o/gate/up are Q5_0
# and attn_v is Q8_0; ffn_down (4864 columns) stays a K-quant
# (tensor/real_tensor_test.go:26-33,55-66).
QWEN05B_REAL_FORMATS = ModelShape(t_q=Q5_0, t_k=Q5_0, t_v=Q8_0, t_o=Q5_0, t_gate=Q5_0, t_up=Q5_0, t_down=Q6_K)

# Qwen special ids (tokenizer/bpe_test.go:31-36)
SPECIAL_TOKENS = {151643: "<|endoftext|>", 151644: "<|im_start|>", 151645: "<|im_end|>"}


def token_list(n_vocab: int) -> List[str]:
    toks = [f"t{i}" for i in range(n_vocab)]
    for i, s in SPECIAL_TOKENS.items():
        if i < n_vocab:
            toks[i] = s
    if n_vocab <= 151645:
        # small test vocabularies still carry the three control tokens
        toks[n_vocab - 3:] = ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]
    return toks


def write_synthetic_model(path: str, shape: ModelShape = QWEN05B, seed: int = 20261201,
                          bias_std: float = 0.02) -> None:
    """Random-init GGUF v3 of the given shape.  numpy PCG64 seeded with `seed`;
    tensors are drawn in file order, so a given (shape, seed) always yields
    the same bytes."""
    rng = np.random.default_rng(seed)
    E, F, V, L = shape.n_embd, shape.n_ff, shape.n_vocab, shape.n_layers
    KV = shape.n_kv_heads * shape.head_dim
    tensors = []

    def quant(name, tt, rows, cols):
        dims = [cols, rows]
        size = tensor_byte_size(tt, dims)
        qk, bs = BLOCK[tt]
        data = SYNTH[tt](rng, size // bs)
        tensors.append((name, dims, tt, data))

    def f32(name, values):
        tensors.append((name, [len(values)], F32, np.asarray(values, dtype="<f4").view(np.uint8)))

    quant("token_embd.weight", shape.t_embd, V, E)
    f32("output_norm.weight", np.ones(E, np.float32))
    if shape.t_out is not None:
        quant("output.weight", shape.t_out, V, E)
    qwen3 = shape.arch == "qwen3"
    for i in range(L):
        f32(f"blk.{i}.attn_norm.weight", np.ones(E, np.float32))
        quant(f"blk.{i}.attn_q.weight", shape.t_q, E, E)
        if not qwen3:
            f32(f"blk.{i}.attn_q.bias", rng.normal(0.0, bias_std, E).astype(np.float32))
        quant(f"blk.{i}.attn_k.weight", shape.t_k, KV, E)
        if not qwen3:
            f32(f"blk.{i}.attn_k.bias", rng.normal(0.0, bias_std, KV).astype(np.float32))
        quant(f"blk.{i}.attn_v.weight", shape.t_v, KV, E)
        if not qwen3:
            f32(f"blk.{i}.attn_v.bias", rng.normal(0.0, bias_std, KV).astype(np.float32))
        else:  # per-head QK-norm weights near 1, distinct for q and k
            f32(f"blk.{i}.attn_q_norm.weight", rng.uniform(0.5, 1.5, shape.head_dim).astype(np.float32))
            f32(f"blk.{i}.attn_k_norm.weight", rng.uniform(0.5, 1.5, shape.head_dim).astype(np.float32))
        quant(f"blk.{i}.attn_output.weight", shape.t_o, E, E)
        f32(f"blk.{i}.ffn_norm.weight", np.ones(E, np.float32))
        quant(f"blk.{i}.ffn_gate.weight", shape.t_gate, F, E)
        quant(f"blk.{i}.ffn_up.weight", shape.t_up, F, E)
        quant(f"blk.{i}.ffn_down.weight", shape.t_down_layers[i] if shape.t_down_layers else shape.t_down, E, F)

    a = shape.arch
    md = [
        ("general.architecture", T_STR, a),
        ("general.name", T_STR, "synthetic-qwen3-shape" if qwen3 else "synthetic-qwen2.5-0.5b-shape"),
        ("general.alignment", T_U32, 32),
        (f"{a}.block_count", T_U32, L),
        (f"{a}.context_length", T_U32, 40960 if qwen3 else 32768),
        (f"{a}.embedding_length", T_U32, E),
        (f"{a}.feed_forward_length", T_U32, F),
        (f"{a}.attention.head_count", T_U32, shape.n_heads),
        (f"{a}.attention.head_count_kv", T_U32, shape.n_kv_heads),
        (f"{a}.rope.freq_base", T_F32, shape.rope_theta),
        (f"{a}.attention.layer_norm_rms_epsilon", T_F32, shape.rms_eps),
        ("tokenizer.ggml.model", T_STR, "gpt2"),
        ("tokenizer.ggml.tokens", T_ARR, (T_STR, token_list(V))),
    ]
    write_gguf(path, md, tensors)


def special_token_ids(gf: GGUFFile):
    """(im_start, im_end, eos) as tokenizer/bpe.go:284-289 resolves them:
    0 when a token is absent."""
    toks = gf.metadata.get("tokenizer.ggml.tokens") or []
    ids = {}
    for i, s in enumerate(toks):
        if s.startswith("<|") and s.endswith("|>"):
            ids[s] = i
    return ids.get("<|im_start|>", 0), ids.get("<|im_end|>", 0), ids.get("<|endoftext|>", 0)
