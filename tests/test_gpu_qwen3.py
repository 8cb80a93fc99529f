"""Qwen3 on the GPU against the oracle: head_dim 128 (engine/model.go:137),
per-head QK-RMSNorm before RoPE and no q/k/v biases
(engine/forward.go:66-91), hidden 2048 (eight Q8_K super-blocks per row),
FFN 6144 (24), and the tied Q8_0 vocab projection of 64 blocks per row.

Two models: a 2-layer model with Qwen3-1.7B's layer shapes (16/8 heads,
vocab 4096) for the forward / KV / logits / long-context cases, and the
full Qwen3-1.7B shape (28 layers, vocab 151936;
engine/model_config_test.go:18-33) for the 64-step stream.  Everything is
compared bit for bit: normX after every forward, the K and V rows, the
logits and the greedy stream (the oracle itself is pinned to a float64
Qwen3 decoder by tests/test_oracle_model.py)."""
import numpy as np
import pytest

from c2slm_amd import _lib as H
from c2slm_amd import gguf as G
from oracle import oracle as O
from tests.test_gpu_model import bits, gpu_generate, open_pair, oracle_generate

pytestmark = pytest.mark.gpu

QWEN3_TINY = G.ModelShape(n_layers=2, n_embd=2048, n_heads=16, n_kv_heads=8, n_ff=6144, n_vocab=4096,
                          arch="qwen3")


@pytest.fixture(scope="module")
def qwen3_tiny_path(tmp_path_factory):
    p = str(tmp_path_factory.mktemp("qwen3") / "qwen3_tiny.gguf")
    G.write_synthetic_model(p, QWEN3_TINY, seed=77)
    return p


def orc_normx(orc, n):
    return np.ctypeslib.as_array(O.lib().orc_state_normx(orc.state), shape=(n,)).copy()


def check_kv(ctx, orc, n, layers, heads):
    kv = orc.kv()
    for which in (0, 1):
        for layer in layers:
            for h in heads:
                got = ctx.kv(which, layer, h, n)
                assert np.array_equal(bits(got), bits(kv[which, layer, h, :n])), (which, layer, h)


def test_qwen3_desc(qwen3_tiny_path):
    gf = G.GGUFFile(qwen3_tiny_path)
    d = H.desc_from_gguf(gf, max_ctx=2048)
    assert (d.n_embd, d.n_heads, d.n_kv_heads, d.head_dim, d.n_ff) == (2048, 16, 8, 128, 6144)


def test_qwen3_forward_kv_logits_bitexact(qwen3_tiny_path):
    gf, ctx, orc, im_end, eos = open_pair(qwen3_tiny_path, max_ctx=2048)
    rng = np.random.default_rng(5)
    toks = rng.integers(0, 4096, 40).tolist() + [4096 + 9]  # an id past the vocabulary embeds id 0
    print("qwen3 tiny: forward of 41 tokens", flush=True)
    for p, t in enumerate(toks):
        got = ctx.forward(int(t), p)
        want = orc.forward(int(t), p)
        assert np.array_equal(bits(got), bits(want)), p
    check_kv(ctx, orc, len(toks), (0, 1), range(8))
    lg = ctx.logits()
    want_lg = orc.compute_logits(orc_normx(orc, 2048))
    assert np.array_equal(bits(lg), bits(want_lg))
    ctx.close()
    orc.close()


def test_qwen3_greedy_64_steps(qwen3_tiny_path):
    gf, ctx, orc, im_end, eos = open_pair(qwen3_tiny_path, max_ctx=512)
    rng = np.random.default_rng(6)
    prompt = rng.integers(0, 4096, 24).astype(np.int32)
    print("qwen3 tiny: 24-token prompt, 64 steps", flush=True)
    got = gpu_generate(ctx, prompt, 64, im_end, eos)
    want = oracle_generate(orc, prompt, 64, im_end, eos)
    assert len(want) == 64 and np.array_equal(got, want)
    assert np.array_equal(bits(ctx.normx()), bits(orc_normx(orc, 2048)))
    ctx.close()
    orc.close()


def test_qwen3_prefill_past_1024_then_steps(qwen3_tiny_path):
    # c2h_prefill runs one forward graph per token at head_dim 128; past
    # 1024 attended positions the softmax sum takes the long exact chain
    gf, ctx, orc, im_end, eos = open_pair(qwen3_tiny_path, max_ctx=1200)
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, 4096, 1100).astype(np.int32)
    print("qwen3 tiny: prefill 1100 tokens, 8 steps", flush=True)
    got_nx = ctx.prefill(prompt, 0)
    want_nx = orc.ingest_from(0, prompt)
    assert np.array_equal(bits(got_nx), bits(want_nx))
    check_kv(ctx, orc, 1100, (1,), (0, 7))
    got = [ctx.step(1100 + i, 1.15, im_end, eos) for i in range(8)]
    want = orc.generate(8, im_end, eos, 1.15)
    assert np.array_equal(np.array(got, np.int32), want)
    ctx.close()
    orc.close()


def test_qwen3_1_7b_shape_greedy_64_steps(tmp_path):
    path = str(tmp_path / "qwen3_1_7b_synth.gguf")
    print("qwen3-1.7b shape: writing the synthetic file", flush=True)
    G.write_synthetic_model(path, G.QWEN3_1_7B, seed=20261202)
    gf = G.GGUFFile(path)
    d = H.desc_from_gguf(gf, max_ctx=1024)
    assert (d.n_layers, d.n_kv_heads, d.head_dim, d.n_heads) == (28, 8, 128, 16)  # model_config_test.go:24-31
    _, im_end, eos = G.special_token_ids(gf)
    assert (im_end, eos) == (151645, 151643)
    ctx = H.Ctx(d)
    H.load_gguf_into(ctx, gf)
    orc = O.OracleEngine(gf, max_ctx=1024, n_threads=16)
    rng = np.random.default_rng(20261202)
    prompt = rng.integers(0, 151936, 16).astype(np.int32)
    print("qwen3-1.7b shape: 16-token prompt, 64 steps", flush=True)
    got = gpu_generate(ctx, prompt, 64, im_end, eos)
    want = oracle_generate(orc, prompt, 64, im_end, eos)
    print("first tokens", got[:8], flush=True)
    assert len(want) == 64 and len(got) == 64
    assert np.array_equal(got, want)
    nx = orc_normx(orc, 2048)
    assert np.array_equal(bits(ctx.normx()), bits(nx))
    check_kv(ctx, orc, 80, (0, 27), (0, 7))
    lg = ctx.logits()
    assert np.array_equal(bits(lg), bits(orc.compute_logits(nx)))
    ctx.close()
    orc.close()
