"""Long-context decode: the KV cache pre-filled with N(0,1) keys and values
at 512 / 4096 / 32768 positions (GQA 14/2, head_dim 64), then engine.Forward
and greedy steps through libc2h.so against the oracle on the same cache.

Past the split length (1024 attended positions by default; C2H_ATT_SPLIT
moves it) decode and prefill attend with the long-context kernels
(k_attn_scores -> k_attn_softmax -> k_attn_av); both forms reproduce
engine/forward.go:143-155 bit for bit, so every comparison is exact."""
import os

import numpy as np
import pytest

from c2slm_amd import _lib as H
from c2slm_amd import gguf as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu

PENALTY = 1.15


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def open_pair(path, max_ctx, split=None):
    gf = G.GGUFFile(path)
    desc = H.desc_from_gguf(gf, max_ctx=max_ctx)
    old = os.environ.get("C2H_ATT_SPLIT")
    if split is not None:
        os.environ["C2H_ATT_SPLIT"] = str(split)
    try:
        ctx = H.Ctx(desc)
    finally:
        if split is not None:
            if old is None:
                del os.environ["C2H_ATT_SPLIT"]
            else:
                os.environ["C2H_ATT_SPLIT"] = old
    H.load_gguf_into(ctx, gf)
    orc = O.OracleEngine(gf, max_ctx=max_ctx, n_threads=16)
    _, im_end, eos = G.special_token_ids(gf)
    return gf, ctx, orc, im_end, eos


def fill_cache(ctx, orc, n, seed):
    """Positions [0, n) of every layer's K and V ~ N(0,1), the same values in
    both caches; token ids uniform; SeqLen = n."""
    rng = np.random.default_rng(seed)
    view = orc.kv_view()
    L, KVH = view.shape[1], view.shape[2]
    for which in (0, 1):
        for layer in range(L):
            for h in range(KVH):
                a = rng.standard_normal((n, 64), dtype=np.float32)
                view[which, layer, h, :n] = a
                ctx.set_kv(which, layer, h, 0, a)
    ids = rng.integers(0, ctx.desc.n_vocab, n).astype(np.int32)
    ctx.set_token_ids(0, ids)
    orc.set_token_ids(0, ids)
    ctx.set_seq(n)
    orc.set_seq_len(n)


def check_decode(ctx, orc, pos, im_end, eos, steps, full_len=False):
    """Forward(11, pos) as ingest does it, then greedy steps: normX, logits
    and the stream equal the oracle's (full_len: all `steps` steps ran, no
    EOS / im_end ended the stream early)."""
    tok = np.array([11], np.int32)
    got = ctx.forward(int(tok[0]), pos)
    want = orc.ingest_from(pos, tok)
    assert np.array_equal(bits(got), bits(want)), f"normX at pos {pos}"
    assert np.array_equal(bits(ctx.logits()), bits(orc.compute_logits(want)))
    stream = []
    p = pos + 1
    for _ in range(steps):
        t = ctx.step(p, PENALTY, im_end, eos)
        stream.append(t)
        p += 1
        if t in (im_end, eos):
            break
    ref = orc.generate(steps, im_end, eos, PENALTY)
    assert np.array_equal(np.array(stream, np.int32), ref)
    if full_len:
        assert len(stream) == steps
    nx = np.ctypeslib.as_array(O.lib().orc_state_normx(orc.state), shape=(ctx.desc.n_embd,))
    assert np.array_equal(bits(ctx.normx()), bits(nx))


# ---- the short-context forms of k_attn_core: prefetch sized for up to 128
# and up to 256 attended positions, and the general form; decode crosses
# each boundary mid-stream (tiny model, default split)

@pytest.mark.parametrize("n0", [124, 252])
def test_core_forms_cross_their_limits(tiny_model_path, n0):
    gf, ctx, orc, im_end, eos = open_pair(tiny_model_path, max_ctx=1024)
    fill_cache(ctx, orc, n0, seed=n0)
    check_decode(ctx, orc, n0, im_end, eos, steps=8)  # T = n0+1 .. n0+9
    ctx.close()
    orc.close()


# ---- the long-context kernels at small sizes (tiny model, split moved down)

def test_long_kernels_decode_small_split(tiny_model_path):
    gf, ctx, orc, im_end, eos = open_pair(tiny_model_path, max_ctx=2048, split=64)
    fill_cache(ctx, orc, 300, seed=31)   # 301 positions: 2 score blocks, 2 AV chunks
    check_decode(ctx, orc, 300, im_end, eos, steps=6)
    ctx.close()
    orc.close()


def test_long_kernels_cross_the_split(tiny_model_path):
    # decode starts below the split (k_attn_core) and crosses it mid-stream
    gf, ctx, orc, im_end, eos = open_pair(tiny_model_path, max_ctx=1024, split=40)
    fill_cache(ctx, orc, 30, seed=32)
    check_decode(ctx, orc, 30, im_end, eos, steps=24)
    ctx.close()
    orc.close()


def test_long_kernels_prefill(tiny_model_path):
    # 40 prompt tokens after 300 cached positions: long-form attention in
    # sub-batches of 16 tokens, KV and normX equal to sequential ingest
    gf, ctx, orc, im_end, eos = open_pair(tiny_model_path, max_ctx=2048, split=64)
    fill_cache(ctx, orc, 300, seed=33)
    rng = np.random.default_rng(34)
    toks = rng.integers(0, 4096, 40).astype(np.int32)
    got = ctx.prefill(toks, 300)
    want = orc.ingest_from(300, toks)
    assert np.array_equal(bits(got), bits(want))
    kv = orc.kv()
    for which in (0, 1):
        for layer in (0, 1):
            for h in (0, 1):
                assert np.array_equal(bits(ctx.kv(which, layer, h, 340)), bits(kv[which, layer, h, :340]))
    assert ctx.seq_len == 340
    ctx.close()
    orc.close()


def test_long_kernels_nan_score_zero(tiny_model_path):
    # a NaN in K row 0 makes score[0] NaN for every head of its group: the
    # max is NaN (tensor/ops.go:320-326) and so is every probability; the
    # other group stays finite.  Both forms must agree with the oracle.
    for split in (4096, 64):
        gf, ctx, orc, im_end, eos = open_pair(tiny_model_path, max_ctx=2048, split=split)
        fill_cache(ctx, orc, 200, seed=35)
        row = np.full((1, 64), np.nan, np.float32)
        ctx.set_kv(0, 1, 0, 0, row)
        orc.kv_view()[0, 1, 0, 0] = row[0]
        got = ctx.forward(5, 200)
        want = orc.forward(5, 200)
        assert np.array_equal(bits(got), bits(want)), split
        ctx.close()
        orc.close()


# ---- config 3: the full Qwen2.5-0.5B-shaped model

@pytest.mark.parametrize("n_ctx", [512, 4096, 32768])
def test_full_model_long_context(full_model_path, n_ctx):
    # Forward at pos = n_ctx - 65 after pos cached positions, then 64 greedy
    # steps (c2slm.go:144-226): the last step forwards its token at
    # n_ctx - 1 and attends all n_ctx positions.  The 64-token stream, the
    # final normX and the logits at pos equal the oracle's bit for bit.
    gf, ctx, orc, im_end, eos = open_pair(full_model_path, max_ctx=32768)
    steps = 64
    pos = n_ctx - 1 - steps
    fill_cache(ctx, orc, pos, seed=n_ctx)
    check_decode(ctx, orc, pos, im_end, eos, steps=steps, full_len=True)
    assert ctx.seq_len == n_ctx
    ctx.close()
    orc.close()


def test_seq_len_tracking(tiny_model_path):
    gf, ctx, orc, im_end, eos = open_pair(tiny_model_path, max_ctx=256)
    assert ctx.seq_len == 0
    ctx.forward(3, 0)
    assert ctx.seq_len == 1
    ctx.prefill(np.arange(10, dtype=np.int32), 1)
    assert ctx.seq_len == 11
    ctx.step(11, PENALTY, im_end, eos)
    assert ctx.seq_len == 12
    ctx.set_seq(4)                   # KVCache.Rewind
    assert ctx.seq_len == 4
    ctx.set_seq(0)                   # KVCache.Reset
    assert ctx.seq_len == 0
    with pytest.raises(H.C2hError):
        ctx.set_seq(257)
    with pytest.raises(H.C2hError):
        ctx.set_kv(0, 0, 0, 250, np.zeros((10, 64), np.float32))
    ctx.close()
    orc.close()
