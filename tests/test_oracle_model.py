"""Pins of the oracle's composed functions -- orc_forward, orc_ingest_from
(a rewind and a clamp), orc_compute_logits and orc_generate
(oracle/c2slm_oracle.c, restating engine/forward.go:54-191 and
c2slm.go:92-226) -- against the float64 Qwen2 decoder of
tests/qwen2_f64.py, which is written from the model's mathematics.

The float64 model takes each Q8_K activation row from the oracle's trace
only after checking that it is a correct rounding of its own float64
activation (tests/qwen2_f64.py, Qwen2F64.feed_q8k), and it must consume
exactly the rows the oracle produced: the count and order of the
quantised GEMVs are checked too.  What remains between the two is float32
against float64 arithmetic.

Tolerance: north_star's 1e-3 relative max-abs (max|a-b| / max|b|) for
normX, K/V and logits.  The greedy stream is compared step by step with the
float64 model fed the oracle's tokens: wherever the float64 top-2 margin
after the penalty exceeds that tolerance, the oracle's token must be the
float64 argmax.

The pin models (tests/qwen2_f64.py, write_pin_model) carry distinct norm
weight vectors and biases comparable to the projections, so a swapped norm
vector, a dropped bias, a wrong RoPE pairing or GQA head map, a missing
residual or a penalty on the wrong ids moves these outputs by far more than
the tolerance; float32 rounding moves them by ~1e-6.  The Qwen3 case
(engine/forward.go:80-91) adds per-head QK-norm vectors of their own, so a
skipped or swapped QK-norm shows the same way.  The bench's own
synthetic draw (all-positive Q4_K weights) is checked as well."""
import numpy as np
import pytest

from c2slm_amd import gguf as G
from oracle import oracle as O
from tests.qwen2_f64 import Qwen2F64, write_pin_model

TOL = 1e-3
PENALTY = 1.15
V = 4096


def rel_err(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


SHAPES = {
    # Q4_K projections, Q6_K attn_v / ffn_down, tied Q8_0 embedding
    "q4k_mix": G.ModelShape(n_layers=2, n_vocab=V),
    # the published file's mix: Q5_0 / Q8_0 projections on the f32 input
    "real_formats": G.ModelShape(n_layers=2, n_vocab=V, t_q=G.Q5_0, t_k=G.Q5_0, t_v=G.Q8_0, t_o=G.Q5_0,
                                 t_gate=G.Q5_0, t_up=G.Q5_0, t_down=G.Q6_K),
    # untied K-quant output.weight (the vocab projection on the Q8_K row)
    "untied_q6k": G.ModelShape(n_layers=2, n_vocab=V, t_out=G.Q6_K),
    "untied_q4k": G.ModelShape(n_layers=2, n_vocab=V, t_out=G.Q4_K),
    # Qwen3: head_dim 128, per-head QK-norm before RoPE, no biases
    "qwen3_hd128": G.ModelShape(n_layers=2, n_embd=512, n_heads=4, n_kv_heads=2, n_ff=768, n_vocab=V,
                                arch="qwen3"),
    # Qwen2.5-1.5B / 3B layout: head_dim 128 with q/k/v biases and no
    # QK-norm, 6 query heads per KV head (smaller widths, same structure)
    "qwen25_hd128": G.ModelShape(n_layers=2, n_embd=768, n_heads=6, n_kv_heads=1, n_ff=1024, n_vocab=V),
}
CASES = sorted(SHAPES) + ["bench_draw"]


@pytest.fixture(scope="module", params=CASES)
def pair(request, tmp_path_factory):
    path = str(tmp_path_factory.mktemp("f64") / f"{request.param}.gguf")
    if request.param == "bench_draw":  # the bench's distributions (gguf.write_synthetic_model)
        G.write_synthetic_model(path, G.ModelShape(n_layers=2, n_vocab=V), seed=31)
    else:
        write_pin_model(path, SHAPES[request.param], seed=31)
    gf = G.GGUFFile(path)
    orc = O.OracleEngine(gf, max_ctx=256, n_threads=4)
    orc.start_q8k_trace()
    ref = Qwen2F64(gf, max_ctx=256)
    yield gf, orc, ref
    orc.close()


def oracle_kv_close(orc, ref, n):
    kv = orc.kv()
    for layer in range(ref.L):
        for g in range(ref.KVH):
            sl = slice(g * ref.hd, (g + 1) * ref.hd)
            assert rel_err(kv[0, layer, g, :n], ref.K[layer, :n, sl]) <= TOL, ("K", layer, g)
            assert rel_err(kv[1, layer, g, :n], ref.Vc[layer, :n, sl]) <= TOL, ("V", layer, g)


def test_forward_kv_logits_match_float64(pair):
    gf, orc, ref = pair
    rng = np.random.default_rng(5)
    toks = rng.integers(0, V, 34).tolist() + [V + 17]  # an id past the vocabulary embeds id 0
    orc.take_q8k_trace()
    worst = 0.0
    for p, t in enumerate(toks):
        got = orc.forward(int(t), p)
        ref.feed_q8k(orc.take_q8k_trace())
        want = ref.forward(int(t), p)
        assert ref.q8k_left() == 0, "the oracle quantised more Q8_K rows than the model needs"
        e = rel_err(got, want)
        worst = max(worst, e)
        assert e <= TOL, (p, e)
    oracle_kv_close(orc, ref, len(toks))
    lg = orc.compute_logits(got)
    ref.feed_q8k(orc.take_q8k_trace())
    want_lg = ref.logits()
    assert ref.q8k_left() == 0
    assert rel_err(lg, want_lg) <= TOL
    print(f"worst normX error over {len(toks)} positions {worst:.1e}; logits {rel_err(lg, want_lg):.1e}")


def test_ingest_rewind_and_clamp_match_float64(pair):
    gf, orc, ref = pair
    rng = np.random.default_rng(6)
    a = rng.integers(0, V, 24).astype(np.int32)
    b = rng.integers(0, V, 20).astype(np.int32)
    c = rng.integers(0, V, 2).astype(np.int32)
    orc.set_seq_len(0)
    orc.take_q8k_trace()
    # (tokens, position the reference's IngestFrom starts at after its clamp)
    for seg, pos_in, pos0 in ((a, 0, 0), (b, 16, 16), (c, 1000, 36)):
        nx = orc.ingest_from(pos_in, seg)
        ref.feed_q8k(orc.take_q8k_trace())
        for i, t in enumerate(seg):
            want = ref.forward(int(t), pos0 + i)
        assert ref.q8k_left() == 0
        assert orc.seq_len == pos0 + len(seg)
        assert rel_err(nx, want) <= TOL
    assert np.array_equal(orc.token_ids()[:38], np.concatenate([a[:16], b, c]))
    oracle_kv_close(orc, ref, 38)


def test_generate_matches_float64_where_decided(pair):
    gf, orc, ref = pair
    _, im_end, eos = G.special_token_ids(gf)
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, V, 32).astype(np.int32)
    prompt[[3, 9, 20]] = prompt[1]  # one id four times in the penalty window
    prompt[30] = im_end             # exempt from the penalty (c2slm.go:163)
    orc.set_seq_len(0)
    orc.take_q8k_trace()
    orc.ingest_from(0, prompt)
    ref.feed_q8k(orc.take_q8k_trace())
    for p, t in enumerate(prompt):
        ref.forward(int(t), p)
    toks = orc.generate(64, im_end, eos, PENALTY)
    ref.feed_q8k(orc.take_q8k_trace())
    ids = list(int(t) for t in prompt)
    decided = 0
    for s, t in enumerate(toks):
        pos = len(ids)
        lg = Qwen2F64.penalise(ref.logits(), ids[max(0, pos - 64):pos], im_end, eos, PENALTY)
        top2 = np.sort(lg)[-2:]
        if top2[1] - top2[0] > TOL * np.max(np.abs(lg)):
            decided += 1
            assert int(np.argmax(lg)) == int(t), (s, int(np.argmax(lg)), int(t))
        ref.forward(int(t), pos)
        ids.append(int(t))
    assert ref.q8k_left() == 0
    assert len(toks) == 64 or toks[-1] in (im_end, eos)
    assert decided >= 0.9 * len(toks), (decided, len(toks))
    print(f"{decided} of {len(toks)} steps decided by a margin above {TOL}")


def check_exemption_and_repeats(orc, ref, seed: int = 8):
    """orc_generate's penalty on the composed path (c2slm.go:157-180): the
    float64 top token t1, placed three times in the window, wins when it is
    the im_end id (exempt) and loses to the float64 winner once its
    occurrences compound past the runner-up."""
    rng = np.random.default_rng(seed)
    prompt = rng.integers(0, V, 8).astype(np.int32)
    orc.set_seq_len(0)
    orc.take_q8k_trace()
    nx = orc.ingest_from(0, prompt)
    ref.feed_q8k(orc.take_q8k_trace())
    for p, t in enumerate(prompt):
        ref.forward(int(t), p)
    orc.compute_logits(nx)  # (an untied K-quant output quantises normX)
    ref.feed_q8k(orc.take_q8k_trace())
    base = ref.logits()
    order = np.argsort(base)[::-1]
    t1 = int(order[0])
    assert base[t1] > 0
    no_id = -1  # an im_end / eos that matches no token
    # (window with t1 at positions 1, 4, 6; im_end), float64 expectation
    for k, im_end in ((3, t1), (None, no_id)):
        win = prompt.copy()
        reps = [1, 4, 6] if k else []
        if k is None:  # enough occurrences of t1 that the runner-up wins
            reps = [1]
            while base[t1] / PENALTY ** len(reps) > base[order[1]] and len(reps) < 7:
                reps.append(len(reps) + 1)
        win[reps] = t1
        orc.set_token_ids(0, win)
        want = Qwen2F64.penalise(base, list(win), im_end, no_id, PENALTY)
        top2 = np.sort(want)[-2:]
        assert top2[1] - top2[0] > TOL * np.max(np.abs(want)), "test logits too close to decide"
        nx_before = ref.normx.copy()
        got = orc.generate(1, im_end, no_id, PENALTY)
        assert int(got[0]) == int(np.argmax(want)), (k, int(got[0]), int(np.argmax(want)))
        assert (int(got[0]) == t1) == (im_end == t1)
        # restore the state the next case starts from
        orc.set_seq_len(0)
        orc.ingest_from(0, prompt)
        orc.take_q8k_trace()
        ref.normx = nx_before


def test_generate_exemption_and_repeats(pair):
    gf, orc, ref = pair
    check_exemption_and_repeats(orc, ref)
