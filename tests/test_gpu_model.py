"""Model-level parity on the GPU: engine.Forward, ComputeLogits and the
greedy generate loop through libc2h.so against the oracle on the same
synthetic GGUF weights.  Everything is compared bit for bit; the greedy
stream must be identical."""
import numpy as np
import pytest

from c2slm_amd import _lib as H
from c2slm_amd import gguf as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu

PENALTY = 1.15  # c2slm.go:165,167


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def open_pair(path, max_ctx, threads=16):
    gf = G.GGUFFile(path)
    desc = H.desc_from_gguf(gf, max_ctx=max_ctx)
    ctx = H.Ctx(desc)
    H.load_gguf_into(ctx, gf)
    orc = O.OracleEngine(gf, max_ctx=max_ctx, n_threads=threads)
    _, im_end, eos = G.special_token_ids(gf)
    return gf, ctx, orc, im_end, eos


@pytest.fixture(scope="module")
def tiny(tiny_model_path):
    gf, ctx, orc, im_end, eos = open_pair(tiny_model_path, 512)
    yield gf, ctx, orc, im_end, eos
    ctx.close()
    orc.close()


def test_forward_bitexact_with_kv(tiny):
    gf, ctx, orc, _, _ = tiny
    rng = np.random.default_rng(1)
    toks = rng.integers(0, 4096, 12)
    toks[3] = -5      # invalid ids embed row 0 (engine/model.go:222-224)
    toks[7] = 99999
    for p, t in enumerate(toks):
        got = ctx.forward(int(t), p)
        want = orc.forward(int(t), p)
        assert np.array_equal(bits(got), bits(want)), p
    kv = orc.kv()
    n = len(toks)
    for which in (0, 1):
        for layer in range(2):
            for h in range(2):
                assert np.array_equal(bits(ctx.kv(which, layer, h, n)), bits(kv[which, layer, h, :n]))


def test_logits_bitexact(tiny):
    gf, ctx, orc, _, _ = tiny
    ctx.forward(17, 0)
    nx = orc.forward(17, 0)
    assert np.array_equal(bits(ctx.normx()), bits(nx))
    assert np.array_equal(bits(ctx.logits()), bits(orc.compute_logits(nx)))


def test_logits_ids_bitexact(tiny):
    # engine.ComputeLogits with a target list (engine/forward.go:171-183):
    # only the listed ids in range are written
    gf, ctx, orc, _, _ = tiny
    ctx.forward(29, 0)
    nx = orc.forward(29, 0)
    full = orc.compute_logits(nx)
    V = ctx.desc.n_vocab
    ids = np.array([5, 0, V - 1, 17, 17, -3, V, 2 ** 30, 1234 % V], np.int32)
    out = np.full(V, 7.25, np.float32)
    got = ctx.logits_ids(ids, out)
    valid = ids[(ids >= 0) & (ids < V)]
    assert np.array_equal(bits(got[valid]), bits(full[valid]))
    rest = np.ones(V, bool)
    rest[valid] = False
    assert np.all(got[rest] == 7.25)
    # a long list (every 7th id) and the empty list (the whole vocabulary)
    many = np.arange(0, V, 7, dtype=np.int32)[::-1].copy()
    got = ctx.logits_ids(many, np.zeros(V, np.float32))
    assert np.array_equal(bits(got[many]), bits(full[many]))
    assert np.array_equal(bits(ctx.logits_ids([], np.zeros(V, np.float32))), bits(full))


def gpu_generate(ctx, prompt, max_new, im_end, eos, penalty=PENALTY):
    """The c2slm.go:92-117 ingest and :144-226 loop over the C ABI."""
    ctx.set_token_ids(0, prompt)
    for p, t in enumerate(prompt):
        ctx.forward(int(t), p, want_normx=False)
    out = []
    pos = len(prompt)
    for _ in range(max_new):
        best = ctx.step(pos, penalty, im_end, eos)
        out.append(best)
        pos += 1
        if best in (im_end, eos):
            break
    return np.array(out, np.int32)


def oracle_generate(orc, prompt, max_new, im_end, eos, penalty=PENALTY):
    orc.ingest_from(0, prompt)
    return orc.generate(max_new, im_end, eos, penalty)


def test_greedy_stream_tiny(tiny):
    gf, ctx, orc, im_end, eos = tiny
    rng = np.random.default_rng(32)
    prompt = rng.integers(0, 4096, 32).astype(np.int32)
    got = gpu_generate(ctx, prompt, 64, im_end, eos)
    orc2 = O.OracleEngine(gf, max_ctx=512, n_threads=16)
    want = oracle_generate(orc2, prompt, 64, im_end, eos)
    assert np.array_equal(got, want)
    want_nx = np.ctypeslib.as_array(O.lib().orc_state_normx(orc2.state), shape=(896,)).copy()
    assert np.array_equal(bits(ctx.normx()), bits(want_nx))
    orc2.close()


def test_device_fed_steps_match_host_loop(tiny):
    # c2h_time_steps copies the state once and lets each step's final norm
    # advance it; its tokens, KV and normX must equal those of c2h_step
    # calls, and c2h_step must continue from where it stopped
    gf, ctx, orc, im_end, eos = tiny
    prompt = np.random.default_rng(33).integers(0, 4096, 32).astype(np.int32)

    def ingest():
        ctx.set_token_ids(0, prompt)
        for p, t in enumerate(prompt):
            ctx.forward(int(t), p, want_normx=False)

    ingest()
    host = [ctx.step(32 + i, PENALTY, im_end, eos) for i in range(24)]
    ctx.sync()
    want_ids = ctx.token_ids(32, 24)
    want_kv = [ctx.kv(w, l, h, 56) for w in (0, 1) for l in range(2) for h in range(2)]
    want_nx = ctx.normx()
    assert np.array_equal(want_ids, np.array(host, np.int32))
    ingest()
    ctx.time_steps(32, 20, PENALTY, im_end, eos)
    tail = [ctx.step(52 + i, PENALTY, im_end, eos) for i in range(4)]
    ctx.sync()
    assert tail == host[20:]
    assert np.array_equal(ctx.token_ids(32, 24), want_ids)
    for got, want in zip([ctx.kv(w, l, h, 56) for w in (0, 1) for l in range(2) for h in range(2)], want_kv):
        assert np.array_equal(bits(got), bits(want))
    assert np.array_equal(bits(ctx.normx()), bits(want_nx))


def test_device_fed_steps_then_step_on_fresh_context(tiny_model_path, tiny):
    # A fresh context's first c2h_step after c2h_time_steps(iters=3): the
    # step numbers the device-fed graphs publish must not be one the next
    # c2h_step waits for, or it would return a token of the earlier steps
    _, ctx_h, _, im_end, eos = tiny
    prompt = np.random.default_rng(35).integers(0, 4096, 32).astype(np.int32)

    def ingest(c):
        c.set_token_ids(0, prompt)
        for p, t in enumerate(prompt):
            c.forward(int(t), p, want_normx=False)

    ingest(ctx_h)
    host = [ctx_h.step(32 + i, PENALTY, im_end, eos) for i in range(6)]
    ctx_h.sync()
    gf = G.GGUFFile(tiny_model_path)
    ctx = H.Ctx(H.desc_from_gguf(gf, max_ctx=512))
    try:
        H.load_gguf_into(ctx, gf)
        ingest(ctx)
        ctx.time_steps(32, 3, PENALTY, im_end, eos)
        tail = [ctx.step(35 + i, PENALTY, im_end, eos) for i in range(3)]
        ctx.sync()
        assert tail == host[3:]
        assert np.array_equal(ctx.token_ids(32, 6), np.array(host, np.int32))
    finally:
        ctx.close()


def test_layer_kernel_timing_leaves_state(tiny):
    # c2h_time_layer_kernel writes KV only at SeqLen and restores X and the
    # normX buffer its final norm writes: a step after it, and after
    # c2h_restore_normx, equals one without it
    gf, ctx, orc, im_end, eos = tiny
    prompt = np.random.default_rng(36).integers(0, 4096, 16).astype(np.int32)
    ctx.set_token_ids(0, prompt)
    for p, t in enumerate(prompt):
        ctx.forward(int(t), p, want_normx=False)
    nx0 = ctx.normx()
    ctx.restore_normx()
    prev = ctx.normx()
    ctx.forward(int(prompt[-1]), 15, want_normx=False)
    for k in H.Ctx.KERNELS:
        ctx.time_layer_kernel(k, 4)
    assert np.array_equal(bits(ctx.normx()), bits(nx0))
    ctx.restore_normx()
    assert np.array_equal(bits(ctx.normx()), bits(prev))
    ctx.forward(int(prompt[-1]), 15, want_normx=False)
    a = ctx.step(16, PENALTY, im_end, eos)
    ctx.sync()
    orc.ingest_from(0, prompt)
    assert a == int(orc.generate(1, im_end, eos, PENALTY)[0])
    ctx.set_seq(512)
    with pytest.raises(H.C2hError):
        ctx.time_layer_kernel("qkv", 4)
    ctx.set_seq(17)


def test_session_differential_ingestion(tiny):
    # c2slm_test.go:60-105: prefix then suffix == one shot, bit for bit
    gf, ctx, orc, _, _ = tiny
    toks = np.arange(100, 120, dtype=np.int32)
    for p, t in enumerate(toks):
        ctx.forward(int(t), p, want_normx=False)
    ref = ctx.logits()
    for p, t in enumerate(toks[:10]):
        ctx.forward(int(t), p, want_normx=False)
    for p, t in enumerate(toks[10:], start=10):
        ctx.forward(int(t), p, want_normx=False)
    assert np.array_equal(bits(ctx.logits()), bits(ref))


def test_position_bounds_rejected(tiny):
    gf, ctx, orc, _, _ = tiny
    with pytest.raises(H.C2hError):
        ctx.forward(1, 512)
    with pytest.raises(H.C2hError):
        ctx.forward(1, -1)


@pytest.mark.parametrize("t_out", [G.Q6_K, G.Q4_K, G.Q5_0])
def test_untied_output_formats(tmp_path, t_out):
    """An untied output.weight in a K-quant or Q5_0: the full projection as
    ParallelGEMV computes it (K-quants on the Q8_K row of normX), the penalty
    and argmax after it, and the restricted logits through the float-x dots
    (computeSingleTokenLogit), all against the oracle."""
    path = str(tmp_path / f"out{t_out}.gguf")
    G.write_synthetic_model(path, G.ModelShape(n_layers=2, n_vocab=4096, t_out=t_out), seed=99)
    gf, ctx, orc, im_end, eos = open_pair(path, 256)
    try:
        nx = orc.forward(3, 0)
        ctx.forward(3, 0)
        full = orc.compute_logits(nx)
        assert np.array_equal(bits(ctx.logits()), bits(full))
        V = ctx.desc.n_vocab
        ids = np.array([0, 9, V - 1, 2048, -1], np.int32)
        got = ctx.logits_ids(ids, np.zeros(V, np.float32))
        w = np.asarray(gf.tensor_map["output.weight"].data)
        rb = G.row_bytes(t_out, ctx.desc.n_embd)
        for t in ids[:4]:
            want = O.gemv(w[t * rb:(t + 1) * rb], t_out, 1, ctx.desc.n_embd, x=nx, float_x=True)[0]
            assert bits(got[t]) == bits(want), t
        prompt = np.array([5, 77, 300, 5, 77], np.int32)
        a = gpu_generate(ctx, prompt, 20, im_end, eos)
        b = oracle_generate(orc, prompt, 20, im_end, eos)
        assert np.array_equal(a, b)
    finally:
        ctx.close()
        orc.close()
