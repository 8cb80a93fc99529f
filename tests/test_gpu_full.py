"""Full-size parity: the Qwen2.5-0.5B-shaped model (24 layers, vocab
151936), 32-token random prompt, 64 greedy steps with the reference's
penalty — the token stream, final normX and logits must be identical to the
oracle's."""
import numpy as np
import pytest

from c2slm_amd import _lib as H
from c2slm_amd import gguf as G
from oracle import oracle as O
from tests.test_gpu_model import gpu_generate, oracle_generate, bits

pytestmark = pytest.mark.gpu


def test_full_model_greedy_64_steps(full_model_path):
    gf = G.GGUFFile(full_model_path)
    _, im_end, eos = G.special_token_ids(gf)
    assert (im_end, eos) == (151645, 151643)
    ctx = H.Ctx(H.desc_from_gguf(gf, max_ctx=1024))
    H.load_gguf_into(ctx, gf)
    orc = O.OracleEngine(gf, max_ctx=1024, n_threads=16)
    rng = np.random.default_rng(20261201)
    prompt = rng.integers(0, 151936, 32).astype(np.int32)
    got = gpu_generate(ctx, prompt, 64, im_end, eos)
    print("first tokens", got[:8])
    want = oracle_generate(orc, prompt, 64, im_end, eos)
    # north star: an identical greedy stream for at least 64 steps (no early EOS on either side)
    assert len(want) == 64 and len(got) == 64
    assert np.array_equal(got, want)
    nx = np.ctypeslib.as_array(O.lib().orc_state_normx(orc.state), shape=(896,)).copy()
    assert np.array_equal(bits(ctx.normx()), bits(nx))
    lg = ctx.logits()
    want_lg = orc.compute_logits(nx)
    assert np.array_equal(bits(lg), bits(want_lg))
    # north-star tolerance, for the record: relative max-abs <= 1e-3
    assert np.max(np.abs(lg - want_lg)) <= 1e-3 * np.max(np.abs(want_lg))
    ctx.close()
    orc.close()


def test_full_model_prefill_512_then_128_steps(full_model_path):
    # batched prefill of a 512-token prompt (int8 MFMA GEMMs), then 128 greedy
    # steps: KV, normX and the stream equal the oracle's sequential ingest
    gf = G.GGUFFile(full_model_path)
    _, im_end, eos = G.special_token_ids(gf)
    ctx = H.Ctx(H.desc_from_gguf(gf, max_ctx=1024))
    H.load_gguf_into(ctx, gf)
    orc = O.OracleEngine(gf, max_ctx=1024, n_threads=16)
    rng = np.random.default_rng(4)
    prompt = rng.integers(0, 151936, 512).astype(np.int32)
    got_nx = ctx.prefill(prompt, 0)
    want_nx = orc.ingest_from(0, prompt)
    assert np.array_equal(bits(got_nx), bits(want_nx))
    kv = orc.kv()
    for which in (0, 1):
        for layer in (0, 11, 23):
            for h in (0, 1):
                assert np.array_equal(bits(ctx.kv(which, layer, h, 512)), bits(kv[which, layer, h, :512]))
    got = []
    pos = 512
    for _ in range(128):
        t = ctx.step(pos, 1.15, im_end, eos)
        got.append(t)
        pos += 1
        if t in (im_end, eos):
            break
    want = orc.generate(128, im_end, eos, 1.15)
    assert len(want) == 128 and len(got) == 128
    assert np.array_equal(np.array(got, np.int32), want)
    ctx.close()
    orc.close()
