"""Host logic of c2slm_amd.engine (the c2slm.go session API) on a scripted
context: clamping and rewinds of IngestFrom (c2slm.go:92-117), the entry
guards (c2slm.go:66-72,125-131), the generate loop's EOS / callback /
stop-string branches (c2slm.go:144-226) and Tokenizer.Decode
(tokenizer/bpe.go:191-229).  No GPU: the device calls are recorded."""
from types import SimpleNamespace

import numpy as np
import pytest

from c2slm_amd import engine as E

IM_END, EOS = 9, 8
TOKENS = ["<|x|>", "a", "Ġhello", "Ċ", "Ã©", "中", "b", "stop", "<|endoftext|>", "<|im_end|>", "c"]


class ScriptedCtx:
    """The c2h calls the engine makes, with c2h_step returning scripted ids."""

    def __init__(self, script=(), max_ctx=64, seq=0):
        self.desc = SimpleNamespace(max_ctx=max_ctx, n_vocab=len(TOKENS), n_embd=4)
        self.seq = seq
        self.script = list(script)
        self.calls = []
        self.ids = {}

    @property
    def seq_len(self):
        return self.seq

    def set_seq(self, n):
        assert 0 <= n <= self.desc.max_ctx
        self.calls.append(("set_seq", n))
        self.seq = n

    def prefill(self, toks, pos):
        self.calls.append(("prefill", pos, list(map(int, toks))))
        for i, t in enumerate(toks):
            self.ids[pos + i] = int(t)
        self.seq = pos + len(toks)
        return np.full(4, self.seq, np.float32)

    def step(self, pos, penalty, im_end, eos):
        assert penalty == E.PENALTY and (im_end, eos) == (IM_END, EOS)
        t = self.script.pop(0)
        self.calls.append(("step", pos, t))
        self.ids[pos] = t
        self.seq = pos + 1
        return t

    def restore_normx(self):
        self.calls.append(("restore",))


def engine(ctx):
    gf = SimpleNamespace(metadata={"tokenizer.ggml.tokens": TOKENS})
    return E.Engine(ctx, gf)


def test_decode_follows_the_gpt2_byte_table():
    d = engine(ScriptedCtx()).decoder
    assert d.decode([2]) == b" hello"
    assert d.decode([3]) == b"\n"
    assert d.decode([4]) == "é".encode("utf-8")       # bytes C3 A9 written through the table
    assert d.decode([5]) == "中".encode("utf-8")      # outside the table: the rune itself
    assert d.decode([9, 0]) == b"<|im_end|><|x|>"    # special tokens verbatim
    assert d.decode([-1, 99, 1]) == b"a"              # out-of-range ids skipped


def test_special_ids():
    e = engine(ScriptedCtx())
    assert (e.im_end, e.eos) == (IM_END, EOS)


def test_ingest_clamps_and_rewinds():
    ctx = ScriptedCtx(seq=10)
    e = engine(ctx)
    assert e.ingest_from(3, []) is None and ctx.calls == []
    e.ingest_from(15, [1, 2])                     # ahead of the cursor: clamped to SeqLen
    assert ctx.calls[-1] == ("prefill", 10, [1, 2]) and ctx.seq == 12
    e.ingest_from(4, [6])                         # behind: rewind, then ingest
    assert ctx.calls[-2:] == [("set_seq", 4), ("prefill", 4, [6])] and ctx.seq == 5
    e.ingest_from(-7, [1])                        # negative: 0
    assert ctx.calls[-2:] == [("set_seq", 0), ("prefill", 0, [1])]


def test_ingest_stops_at_capacity():
    ctx = ScriptedCtx(max_ctx=16, seq=14)
    e = engine(ctx)
    e.ingest_from(14, [1, 2, 3, 4, 5])
    assert ctx.calls[-1] == ("prefill", 14, [1, 2]) and ctx.seq == 16
    assert e.ingest_from(16, [1]) is None


def test_generate_eos_is_forwarded_and_counted():
    ctx = ScriptedCtx([1, 2, EOS, 1])
    e = engine(ctx)
    out = e.generate_stream([1, 6, 10], 10)
    assert out == b"a hello"
    assert ctx.calls[0] == ("set_seq", 0)
    assert [c for c in ctx.calls if c[0] == "step"] == [("step", 3, 1), ("step", 4, 2), ("step", 5, EOS)]
    assert ctx.seq == 6 and ctx.ids[5] == EOS


def test_generate_callback_false_keeps_the_token():
    ctx = ScriptedCtx([1, 2, 6, 6])
    e = engine(ctx)
    seen = []
    out = e.generate_stream([1], 10, on_token=lambda p: seen.append(p) or len(seen) < 2)
    assert out == b"a hello" and seen == [b"a", b" hello"]
    assert ctx.seq == 3  # both tokens forwarded (c2slm.go:196-201)


def test_generate_stop_string_drops_the_token():
    ctx = ScriptedCtx([1, 7, 6])
    e = engine(ctx)
    out = e.generate_stream([10, 10], 10, stop_strings=[b"astop"])
    assert out == b"astop"
    # the matching token was not forwarded in the reference: SeqLen stays,
    # normX goes back to the one before it
    assert ctx.calls[-2:] == [("restore",), ("set_seq", 3)]
    assert ctx.seq == 3


def test_max_new_tokens_clamped_to_capacity():
    ctx = ScriptedCtx([1] * 10, max_ctx=16)
    e = engine(ctx)
    e.generate_stream(list(range(1, 11)) + [1, 1, 1, 1], 10)
    assert len([c for c in ctx.calls if c[0] == "step"]) == 2 and ctx.seq == 16


def test_session_appends_without_reset():
    ctx = ScriptedCtx([1, 2, 6, 10], max_ctx=64)
    e = engine(ctx)
    e.generate_stream([1, 1], 2)
    assert ctx.seq == 4
    e.generate_stream_session([6, 6, 6], 2)
    assert ("set_seq", 0) not in ctx.calls[1:]
    assert ("prefill", 4, [6, 6, 6]) in ctx.calls and ctx.seq == 9


def test_entry_guards():
    e = engine(ScriptedCtx(max_ctx=16, seq=10))
    with pytest.raises(E.EngineError, match="empty prompt"):
        e.generate_stream([], 4)
    with pytest.raises(E.EngineError, match="exceeds max context"):
        e.generate_stream([1] * 16, 4)
    with pytest.raises(E.EngineError, match="empty prompt"):
        e.generate_stream_session([], 4)
    with pytest.raises(E.EngineError, match="session prompt"):
        e.generate_stream_session([1] * 6, 4)   # 10 + 6 >= 16
