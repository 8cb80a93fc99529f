"""The decode step's launch forms on the GPU against the oracle, bit for bit.

A layer past 0 runs q|k|v, attention and the o-projection as one launch
(k_attn_block, or k_attn_block_f for Q5_0 / Q8_0 projections), layer 0 as
q|k|v then attention + o-projection (k_attn_oproj); with K-quant gate/up and
a Q6_K down projection the FFN is one launch too (k_ffn_block: the down
projection split by super-block, its terms folded in block order).
C2H_NO_FUSE, read when a context is created, selects the separate forms
("qkv": q|k|v on its own, "ffn": the FFN's two launches apart, "1": every
kernel on its own), which models without the fused instances run.
Each form: a 20-token ingest, normX after every forward, every K and V row,
then a 40-step greedy stream (positions 20..59, crossing the 32- and
64-position attention tiers), on the Qwen2.5-0.5B layer shape with the
synthetic K-quant mix and with the published file's format mix; and two
corners of the FFN's residual add moving to the next launch: a one-layer
model (layer 0's FFN leaves it to the final norm), K-quant attention with
Q5_0 gate/up (the float-input FFN launch leaves it to k_attn_block), and
ffn_down Q6_K / Q4_K / Q6_K by layer, as a Q4_K_M file mixes it (the FFN as
one launch on layers 0 and 2, as two on layer 1)."""
import numpy as np
import pytest

from c2slm_amd import _lib as H
from c2slm_amd import gguf as G
from oracle import oracle as O
from tests.test_gpu_model import PENALTY, bits

pytestmark = pytest.mark.gpu

FORMS = ["1", "qkv", "ffn", ""]  # separate, attention + o-projection only, the FFN apart, all fused


@pytest.fixture(scope="module", params=["k-quants", "real-formats", "one-layer", "q50-ffn", "mixed-down"])
def model(request, tmp_path_factory):
    p = str(tmp_path_factory.mktemp("forms") / f"{request.param}.gguf")
    shape = G.ModelShape(n_layers=2, n_vocab=4096)
    if request.param == "real-formats":
        shape = G.ModelShape(n_layers=2, n_vocab=4096, t_q=G.Q5_0, t_k=G.Q5_0, t_v=G.Q8_0, t_o=G.Q5_0,
                             t_gate=G.Q5_0, t_up=G.Q5_0, t_down=G.Q6_K)
    elif request.param == "one-layer":
        shape = G.ModelShape(n_layers=1, n_vocab=4096)
    elif request.param == "q50-ffn":
        shape = G.ModelShape(n_layers=2, n_vocab=4096, t_gate=G.Q5_0, t_up=G.Q5_0, t_down=G.Q6_K)
    elif request.param == "mixed-down":  # the FFN one launch on layers 0 and 2, two on layer 1
        shape = G.ModelShape(n_layers=3, n_vocab=4096, t_down_layers=(G.Q6_K, G.Q4_K, G.Q6_K))
    G.write_synthetic_model(p, shape, seed=77)
    gf = G.GGUFFile(p)
    _, im_end, eos = G.special_token_ids(gf)
    prompt = np.random.default_rng(78).integers(0, 4096, 20).astype(np.int32)
    orc = O.OracleEngine(gf, max_ctx=256, n_threads=16)
    nx = [orc.forward(int(t), i).copy() for i, t in enumerate(prompt)]
    kv = orc.kv()[:, :, :, :len(prompt)].copy()
    orc.close()
    orc = O.OracleEngine(gf, max_ctx=256, n_threads=16)
    orc.ingest_from(0, prompt)
    stream = orc.generate(40, im_end, eos, PENALTY)
    orc.close()
    return request.param, gf, prompt, nx, kv, stream, im_end, eos


@pytest.mark.parametrize("form", FORMS)
def test_launch_form_bitexact(model, form, monkeypatch):
    name, gf, prompt, nx, kv, stream, im_end, eos = model
    if form:
        monkeypatch.setenv("C2H_NO_FUSE", form)
    else:
        monkeypatch.delenv("C2H_NO_FUSE", raising=False)
    print(f"{name}: C2H_NO_FUSE={form!r}", flush=True)
    ctx = H.Ctx(H.desc_from_gguf(gf, max_ctx=256))
    try:
        H.load_gguf_into(ctx, gf)
        ctx.set_token_ids(0, prompt)
        for i, t in enumerate(prompt):
            assert np.array_equal(bits(ctx.forward(int(t), i)), bits(nx[i])), (name, form, i)
        for which in (0, 1):
            for layer in range(kv.shape[1]):  # [K|V][layer][kv head][position][dim]
                for h in range(2):
                    assert np.array_equal(bits(ctx.kv(which, layer, h, len(prompt))),
                                          bits(kv[which, layer, h])), (name, form, which, layer, h)
        out, pos = [], len(prompt)
        for _ in range(40):
            t = ctx.step(pos, PENALTY, im_end, eos)
            out.append(t)
            pos += 1
            if t in (im_end, eos):
                break
        ctx.sync()
        assert np.array_equal(np.array(out, np.int32), stream), (name, form)
    finally:
        ctx.close()
