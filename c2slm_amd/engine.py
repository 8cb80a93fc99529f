"""Host side of the decode path over the C ABI, mirroring the reference's
engine API (c2slm.go:12-226): NewEngine, Close, IngestFrom,
GenerateStream, GenerateStreamSession and the generate loop, with the same
argument meaning, clamping and error behaviour.

The device owns the step: c2h_step runs logits -> repetition penalty ->
greedy argmax -> Forward(best, pos) and returns only the chosen id.  Token
text, the stop-string check and the on_token callback stay here, as in the
reference.  Prompts are token ids (the reference's BPE Encode,
tokenizer/bpe.go:85-189, is not part of this path); Decode follows
tokenizer/bpe.go:191-229 on the GGUF vocabulary and returns bytes, which is
what the reference's Go strings hold.
"""
from __future__ import annotations

from typing import Callable, Iterable, Optional, Sequence

import numpy as np

from . import _lib as H
from . import gguf as G

MAX_CONTEXT_LEN = 16384  # engine.MaxContextLen (engine/kvcache.go:11)
PENALTY = 1.15           # c2slm.go:165,167


class EngineError(RuntimeError):
    """The errors the reference's Generate* entry guards return
    (c2slm.go:66-72,125-131)."""


def _bytes_to_unicode():
    """GPT-2 byte <-> unicode table (tokenizer/bpe.go:244-281)."""
    bs = list(range(ord("!"), ord("~") + 1)) + list(range(ord("¡"), ord("¬") + 1)) + \
        list(range(ord("®"), ord("ÿ") + 1))
    cs = list(bs)
    n = 0
    for b in range(256):
        if b not in bs:
            bs.append(b)
            cs.append(256 + n)
            n += 1
    return {b: chr(c) for b, c in zip(bs, cs)}


class VocabDecoder:
    """Tokenizer.Decode (tokenizer/bpe.go:191-229) over tokenizer.ggml.tokens:
    out-of-range ids are skipped, special tokens (<|...|>) are copied
    verbatim, other tokens map their characters back to bytes through the
    GPT-2 table; characters outside it are written as UTF-8."""

    def __init__(self, gf):
        self.tokens = list(gf.metadata.get("tokenizer.ggml.tokens") or [])
        self.special = {s for s in self.tokens if s.startswith("<|") and s.endswith("|>")}
        self.u2b = {u: b for b, u in _bytes_to_unicode().items()}

    def decode(self, ids: Iterable[int]) -> bytes:
        out = bytearray()
        for i in ids:
            if i < 0 or i >= len(self.tokens):
                continue
            s = self.tokens[i]
            if s in self.special:
                out += s.encode("utf-8")
                continue
            for ch in s:
                b = self.u2b.get(ch)
                out += bytes([b]) if b is not None else ch.encode("utf-8")
        return bytes(out)


class Engine:
    """c2slm.Engine (c2slm.go:12-17) on one GPU: the model and KV cache live
    in a c2h context; SeqLen is the context's (c2h_get_seq / c2h_set_seq).
    The reference sizes the cache and its guards with engine.MaxContextLen;
    here both are the context's max_ctx (16384 by default)."""

    def __init__(self, ctx: H.Ctx, gf, decoder=None):
        self.ctx = ctx
        self.gf = gf
        self.decoder = decoder if decoder is not None else VocabDecoder(gf)
        self.im_start, self.im_end, self.eos = G.special_token_ids(gf)
        self.max_tokens = ctx.desc.max_ctx  # KVCache.MaxTokens
        self.n_vocab = ctx.desc.n_vocab

    @classmethod
    def new(cls, model_path: str, max_ctx: int = MAX_CONTEXT_LEN, device: int = 0, decoder=None) -> "Engine":
        """NewEngine (c2slm.go:20-42): load the GGUF, upload every tensor
        LoadModel binds, allocate the KV cache of max_ctx positions."""
        gf = G.GGUFFile(model_path)
        if not gf.metadata.get("tokenizer.ggml.tokens"):
            raise EngineError("load tokenizer: tokenizer.ggml.tokens missing or empty")
        ctx = H.Ctx(H.desc_from_gguf(gf, max_ctx=max_ctx), device)
        try:
            H.load_gguf_into(ctx, gf)
        except Exception:
            ctx.close()
            raise
        return cls(ctx, gf, decoder)

    def close(self) -> None:
        """Engine.Close (c2slm.go:44-55); idempotent."""
        if self.ctx is not None:
            self.ctx.close()
            self.ctx = None

    @property
    def seq_len(self) -> int:
        return self.ctx.seq_len

    def ingest_from(self, pos: int, tokens: Sequence[int]) -> Optional[np.ndarray]:
        """Engine.IngestFrom (c2slm.go:92-117): pos clamped to [0, SeqLen],
        the cache rewound to pos, tokens past MaxTokens dropped; returns the
        last token's normX (None for no tokens).  The batch runs as one
        c2h_prefill, bit-identical to the reference's Forward loop."""
        toks = np.asarray(tokens, dtype=np.int32)
        if len(toks) == 0:
            return None
        seq = self.ctx.seq_len
        pos = min(max(pos, 0), seq)
        if pos < seq:
            self.ctx.set_seq(pos)  # KVCache.Rewind
        toks = toks[: max(0, self.max_tokens - pos)]
        if len(toks) == 0:
            return None
        return self.ctx.prefill(toks, pos)

    def generate_stream(self, prompt_tokens: Sequence[int], max_new_tokens: int,
                        stop_strings: Sequence[bytes] = (),
                        on_token: Optional[Callable[[bytes], bool]] = None) -> bytes:
        """Engine.GenerateStream (c2slm.go:64-82) after tokenisation: reset
        the cache, ingest the whole prompt, generate."""
        toks = np.asarray(prompt_tokens, dtype=np.int32)
        if len(toks) == 0:
            raise EngineError("empty prompt tokens")
        if len(toks) >= self.max_tokens:
            raise EngineError(f"prompt ({len(toks)}) exceeds max context ({self.max_tokens})")
        self.ctx.set_seq(0)  # KVCache.Reset
        last = self.ingest_from(0, toks)
        max_new_tokens = min(max_new_tokens, self.max_tokens - self.ctx.seq_len)
        return self._generate(last, self.ctx.seq_len, max_new_tokens, stop_strings, on_token)

    def generate(self, prompt_tokens: Sequence[int], max_new_tokens: int, stop_strings: Sequence[bytes] = ()) -> bytes:
        """Engine.Generate (c2slm.go:58-60)."""
        return self.generate_stream(prompt_tokens, max_new_tokens, stop_strings, None)

    def generate_stream_session(self, new_prompt_tokens: Sequence[int], max_new_tokens: int,
                                stop_strings: Sequence[bytes] = (),
                                on_token: Optional[Callable[[bytes], bool]] = None) -> bytes:
        """Engine.GenerateStreamSession (c2slm.go:119-138): append to the
        cached conversation without recomputing it."""
        toks = np.asarray(new_prompt_tokens, dtype=np.int32)
        if len(toks) == 0:
            raise EngineError("empty prompt tokens")
        seq = self.ctx.seq_len
        if seq + len(toks) >= self.max_tokens:
            raise EngineError(f"session prompt ({seq + len(toks)}) exceeds max context ({self.max_tokens})")
        last = self.ingest_from(seq, toks)
        max_new_tokens = min(max_new_tokens, self.max_tokens - self.ctx.seq_len)
        return self._generate(last, self.ctx.seq_len, max_new_tokens, stop_strings, on_token)

    def _generate(self, last_normx, current_pos: int, max_new_tokens: int, stop_strings, on_token) -> bytes:
        """The generate loop (c2slm.go:144-226).  c2h_step forwards the chosen
        token at once (TokenIDs and SeqLen included), which is what the
        reference does on every branch except a stop-string match; there the
        step is undone: the previous normX is restored and SeqLen stays, so
        the forwarded K/V entry is past the cursor and the next ingest
        overwrites it."""
        text = bytearray()
        stops = [s.encode("utf-8") if isinstance(s, str) else bytes(s) for s in stop_strings]
        for _ in range(max_new_tokens):
            if current_pos >= self.max_tokens:
                break
            best = self.ctx.step(current_pos, PENALTY, self.im_end, self.eos)
            if best in (self.im_end, self.eos):
                break  # forwarded and recorded, SeqLen = current_pos + 1
            piece = self.decoder.decode([best])
            text += piece
            if on_token is not None and not on_token(piece):
                break  # forwarded and recorded, as c2slm.go:196-201
            if any(s in text for s in stops):
                self.ctx.restore_normx()
                self.ctx.set_seq(current_pos)
                break
            current_pos += 1
        return bytes(text)
