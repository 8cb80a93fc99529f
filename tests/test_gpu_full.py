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
    assert len(got) == len(want) and np.array_equal(got, want)
    nx = np.ctypeslib.as_array(O.lib().orc_state_normx(orc.state), shape=(896,)).copy()
    assert np.array_equal(bits(ctx.normx()), bits(nx))
    lg = ctx.logits()
    want_lg = orc.compute_logits(nx)
    assert np.array_equal(bits(lg), bits(want_lg))
    # north-star tolerance, for the record: relative max-abs <= 1e-3
    assert np.max(np.abs(lg - want_lg)) <= 1e-3 * np.max(np.abs(want_lg))
    ctx.close()
    orc.close()
