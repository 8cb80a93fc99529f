"""Larger Qwen2.5 shapes that the reference's LoadModel reads with the same
qwen2.* keys (engine/model.go:64-145; head_dim = n_embd / n_heads):
Qwen2.5-1.5B (hidden 1536 = 6 Q8_K super-blocks, 12 query / 2 KV heads of
128, FFN 8960 = 35 super-blocks, q/k/v biases, a vocab row of 48 Q8_0
blocks) and Qwen2.5-3B (hidden 2048, 16 / 2 heads of 128, FFN 11008 = 43
super-blocks).  Head_dim 128 without the Qwen3 QK-norm, and 6 or 8 query
heads per KV head.  Two-layer models with each shape's layers and a 4,096-id
vocabulary, against the oracle bit for bit: normX after every forward, the
K and V rows, the logits, a 48-step greedy stream, and an ingest of 20
tokens through c2h_prefill."""
import numpy as np
import pytest

from c2slm_amd import _lib as H
from c2slm_amd import gguf as G
from oracle import oracle as O
from tests.test_gpu_model import bits, gpu_generate, open_pair, oracle_generate

pytestmark = pytest.mark.gpu

SHAPES = {
    "qwen2.5-1.5b": G.ModelShape(n_layers=2, n_embd=1536, n_heads=12, n_kv_heads=2, n_ff=8960, n_vocab=4096),
    "qwen2.5-3b": G.ModelShape(n_layers=2, n_embd=2048, n_heads=16, n_kv_heads=2, n_ff=11008, n_vocab=4096),
}


@pytest.fixture(scope="module", params=sorted(SHAPES))
def shape_path(request, tmp_path_factory):
    p = str(tmp_path_factory.mktemp("shapes") / f"{request.param}.gguf")
    G.write_synthetic_model(p, SHAPES[request.param], seed=311)
    return request.param, p


def orc_normx(orc, n):
    return np.ctypeslib.as_array(O.lib().orc_state_normx(orc.state), shape=(n,)).copy()


def test_shape_desc(shape_path):
    name, path = shape_path
    s = SHAPES[name]
    d = H.desc_from_gguf(G.GGUFFile(path), max_ctx=512)
    assert (d.n_embd, d.n_heads, d.n_kv_heads, d.head_dim, d.n_ff) == (s.n_embd, s.n_heads, s.n_kv_heads, 128, s.n_ff)


def test_shape_forward_kv_logits_bitexact(shape_path):
    name, path = shape_path
    gf, ctx, orc, im_end, eos = open_pair(path, max_ctx=512)
    E = ctx.desc.n_embd
    try:
        toks = np.random.default_rng(12).integers(0, 4096, 24).tolist() + [-3]  # an invalid id embeds row 0
        print(f"{name}: forward of {len(toks)} tokens", flush=True)
        for p, t in enumerate(toks):
            got = ctx.forward(int(t), p)
            want = orc.forward(int(t), p)
            assert np.array_equal(bits(got), bits(want)), (name, p)
        kv = orc.kv()
        for which in (0, 1):
            for layer in (0, 1):
                for h in (0, 1):
                    assert np.array_equal(bits(ctx.kv(which, layer, h, len(toks))),
                                          bits(kv[which, layer, h, :len(toks)])), (which, layer, h)
        assert np.array_equal(bits(ctx.logits()), bits(orc.compute_logits(orc_normx(orc, E))))
    finally:
        ctx.close()
        orc.close()


def test_shape_greedy_stream_and_prefill(shape_path):
    name, path = shape_path
    gf, ctx, orc, im_end, eos = open_pair(path, max_ctx=512)
    E = ctx.desc.n_embd
    try:
        prompt = np.random.default_rng(13).integers(0, 4096, 20).astype(np.int32)
        print(f"{name}: 20-token prompt, 48 steps", flush=True)
        got = gpu_generate(ctx, prompt, 48, im_end, eos)
        want = oracle_generate(orc, prompt, 48, im_end, eos)
        assert np.array_equal(got, want)
        assert np.array_equal(bits(ctx.normx()), bits(orc_normx(orc, E)))
        # the same prompt through c2h_prefill equals the oracle's ingest
        ctx.set_token_ids(0, prompt)
        nx = ctx.prefill(prompt, 0)
        want_nx = orc.ingest_from(0, prompt)
        assert np.array_equal(bits(nx), bits(want_nx))
        assert ctx.seq_len == len(prompt)
    finally:
        ctx.close()
        orc.close()
