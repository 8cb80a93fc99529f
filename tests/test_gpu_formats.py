"""The real-model format mix (the published Qwen2.5-0.5B-Instruct Q4_K_M
file: Q5_0 q/k/o/gate/up, Q8_0 attn_v, K-quant ffn_down; engine/model.go:
250-270 multiplies Q5_0/Q8_0 with the f32 input) through the decode path,
bit for bit against the oracle."""
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
def real_tiny(tmp_path_factory):
    p = str(tmp_path_factory.mktemp("models") / "tiny_real.gguf")
    shape = G.ModelShape(n_layers=2, n_vocab=4096, t_q=G.Q5_0, t_k=G.Q5_0, t_v=G.Q8_0, t_o=G.Q5_0,
                         t_gate=G.Q5_0, t_up=G.Q5_0, t_down=G.Q6_K)
    G.write_synthetic_model(p, shape, seed=77)
    return p


def open_pair(path, max_ctx):
    gf = G.GGUFFile(path)
    ctx = H.Ctx(H.desc_from_gguf(gf, max_ctx=max_ctx))
    H.load_gguf_into(ctx, gf)
    orc = O.OracleEngine(gf, max_ctx=max_ctx, n_threads=16)
    _, im_end, eos = G.special_token_ids(gf)
    return gf, ctx, orc, im_end, eos


def test_real_formats_forward_and_kv(real_tiny):
    gf, ctx, orc, _, _ = open_pair(real_tiny, 256)
    rng = np.random.default_rng(78)
    toks = rng.integers(0, 4093, 12)
    toks[5] = -2
    for p, t in enumerate(toks):
        got = ctx.forward(int(t), p)
        want = orc.forward(int(t), p)
        assert np.array_equal(bits(got), bits(want)), p
    kv = orc.kv()
    for which in (0, 1):
        for layer in (0, 1):
            for h in (0, 1):
                assert np.array_equal(bits(ctx.kv(which, layer, h, 12)), bits(kv[which, layer, h, :12]))
    assert np.array_equal(bits(ctx.logits()), bits(orc.compute_logits(want)))
    ctx.close()
    orc.close()


def test_real_formats_greedy_stream(real_tiny):
    gf, ctx, orc, im_end, eos = open_pair(real_tiny, 256)
    rng = np.random.default_rng(79)
    prompt = rng.integers(0, 4093, 20).astype(np.int32)
    ctx.set_token_ids(0, prompt)
    for p, t in enumerate(prompt):
        ctx.forward(int(t), p, want_normx=False)
    got = []
    pos = len(prompt)
    for _ in range(40):
        t = ctx.step(pos, PENALTY, im_end, eos)
        got.append(t)
        pos += 1
        if t in (im_end, eos):
            break
    orc.ingest_from(0, prompt)
    want = orc.generate(40, im_end, eos, PENALTY)
    assert np.array_equal(np.array(got, np.int32), want)
    ctx.close()
    orc.close()


def test_real_formats_batched_prefill(real_tiny):
    # Q5_0 / Q8_0 projections of a token batch (k_pf_gemm_q50, k_pf_gemm_f;
    # 37 and 21 tokens: partial 16-token tiles) with the K-quant ffn_down on
    # MFMA: KV and normX equal sequential ingest
    gf, ctx, orc, _, _ = open_pair(real_tiny, 256)
    rng = np.random.default_rng(81)
    a = rng.integers(0, 4093, 37).astype(np.int32)
    b = rng.integers(0, 4093, 21).astype(np.int32)
    ctx.prefill(a, 0, want_normx=False)
    got = ctx.prefill(b, 37)
    orc.ingest_from(0, a)
    want = orc.ingest_from(37, b)
    assert np.array_equal(bits(got), bits(want))
    kv = orc.kv()
    for which in (0, 1):
        for layer in (0, 1):
            for h in (0, 1):
                assert np.array_equal(bits(ctx.kv(which, layer, h, 58)), bits(kv[which, layer, h, :58]))
    ctx.close()
    orc.close()


def test_real_formats_prefill_300_tokens(real_tiny):
    # 300 tokens from position 0: nineteen 16-token tiles of k_pf_gemm_q50
    # (the last partial, 12 tokens: both staged halves hold padding), attn_v
    # through k_pf_gemm_f at 4 tokens per workgroup, and the 8-token blocks
    # of k_pf_attn up to 300 positions
    gf, ctx, orc, _, _ = open_pair(real_tiny, 512)
    toks = np.random.default_rng(83).integers(0, 4093, 300).astype(np.int32)
    got = ctx.prefill(toks, 0)
    want = orc.ingest_from(0, toks)
    assert np.array_equal(bits(got), bits(want))
    kv = orc.kv()
    for which in (0, 1):
        for layer in (0, 1):
            for h in (0, 1):
                assert np.array_equal(bits(ctx.kv(which, layer, h, 300)), bits(kv[which, layer, h, :300]))
    ctx.close()
    orc.close()


def test_full_model_real_formats_64_steps(tmp_path_factory):
    p = str(tmp_path_factory.mktemp("models") / "qwen05b_real.gguf")
    G.write_synthetic_model(p, G.QWEN05B_REAL_FORMATS, seed=20261202)
    gf, ctx, orc, im_end, eos = open_pair(p, 1024)
    rng = np.random.default_rng(80)
    prompt = rng.integers(0, 151936, 32).astype(np.int32)
    ctx.prefill(prompt, 0, want_normx=False)  # batched: Q5_0 / Q8_0 / Q6_K projections of 32 tokens
    got = []
    pos = len(prompt)
    for _ in range(64):
        t = ctx.step(pos, PENALTY, im_end, eos)
        got.append(t)
        pos += 1
        if t in (im_end, eos):
            break
    orc.ingest_from(0, prompt)
    want = orc.generate(64, im_end, eos, PENALTY)
    assert np.array_equal(np.array(got, np.int32), want)
    nx = np.ctypeslib.as_array(O.lib().orc_state_normx(orc.state), shape=(896,))
    assert np.array_equal(bits(ctx.normx()), bits(nx))
    ctx.close()
    orc.close()
