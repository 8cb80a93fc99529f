"""Batched prefill (c2h_prefill) against the oracle's sequential ingest
(c2slm.go:92-117: engine.Forward per token).  Every token's arithmetic is
the reference's, so the KV cache, the final normX and the greedy stream that
follows must be bit-identical."""
import numpy as np
import pytest

from c2slm_amd import _lib as H
from c2slm_amd import gguf as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu

PENALTY = 1.15


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def tiny(tiny_model_path):
    gf = G.GGUFFile(tiny_model_path)
    desc = H.desc_from_gguf(gf, max_ctx=512)
    ctx = H.Ctx(desc)
    H.load_gguf_into(ctx, gf)
    _, im_end, eos = G.special_token_ids(gf)
    yield gf, ctx, im_end, eos
    ctx.close()


def check_kv(ctx, orc, n, layers=(0, 1)):
    kv = orc.kv()
    for which in (0, 1):
        for layer in layers:
            for h in range(2):
                got = ctx.kv(which, layer, h, n)
                assert np.array_equal(bits(got), bits(kv[which, layer, h, :n])), (which, layer, h)


def test_prefill_matches_sequential_ingest(tiny):
    gf, ctx, _, _ = tiny
    rng = np.random.default_rng(5)
    toks = rng.integers(0, 4096, 37).astype(np.int32)  # not a multiple of the 64-token tile
    toks[4] = -3          # invalid ids embed row 0 (engine/model.go:222-224)
    toks[20] = 99999
    got = ctx.prefill(toks, 0)
    orc = O.OracleEngine(gf, max_ctx=512, n_threads=16)
    want = orc.ingest_from(0, toks)
    assert np.array_equal(bits(got), bits(want))
    check_kv(ctx, orc, len(toks))
    orc.close()


def test_prefill_continues_a_cached_prefix(tiny):
    # the second batch attends to positions the first one stored
    gf, ctx, _, _ = tiny
    rng = np.random.default_rng(6)
    a = rng.integers(0, 4096, 20).astype(np.int32)
    b = rng.integers(0, 4096, 150).astype(np.int32)  # > 128: the attention stages V in two chunks
    ctx.prefill(a, 0, want_normx=False)
    got = ctx.prefill(b, 20)
    orc = O.OracleEngine(gf, max_ctx=512, n_threads=16)
    orc.ingest_from(0, a)
    want = orc.ingest_from(20, b)
    assert np.array_equal(bits(got), bits(want))
    check_kv(ctx, orc, 170)
    orc.close()


def test_prefill_equals_device_forward_loop(tiny):
    gf, ctx, _, _ = tiny
    rng = np.random.default_rng(7)
    toks = rng.integers(0, 4096, 70).astype(np.int32)
    for p, t in enumerate(toks):
        seq = ctx.forward(int(t), p)
    kv_seq = [ctx.kv(w, l, h, 70) for w in (0, 1) for l in (0, 1) for h in (0, 1)]
    got = ctx.prefill(toks, 0)
    assert np.array_equal(bits(got), bits(seq))
    kv_pf = [ctx.kv(w, l, h, 70) for w in (0, 1) for l in (0, 1) for h in (0, 1)]
    for x, y in zip(kv_seq, kv_pf):
        assert np.array_equal(bits(x), bits(y))


def test_prefill_then_greedy_stream(tiny):
    gf, ctx, im_end, eos = tiny
    rng = np.random.default_rng(8)
    prompt = rng.integers(0, 4096, 96).astype(np.int32)
    ctx.prefill(prompt, 0, want_normx=False)
    got = []
    pos = len(prompt)
    for _ in range(48):
        t = ctx.step(pos, PENALTY, im_end, eos)
        got.append(t)
        pos += 1
        if t in (im_end, eos):
            break
    orc = O.OracleEngine(gf, max_ctx=512, n_threads=16)
    orc.ingest_from(0, prompt)
    want = orc.generate(48, im_end, eos, PENALTY)
    assert np.array_equal(np.array(got, np.int32), want)
    orc.close()


def test_prefill_bounds(tiny):
    gf, ctx, _, _ = tiny
    with pytest.raises(H.C2hError):
        ctx.prefill(np.zeros(10, np.int32), 505)  # past max_ctx
    with pytest.raises(H.C2hError):
        ctx.prefill(np.zeros(3, np.int32), -1)
