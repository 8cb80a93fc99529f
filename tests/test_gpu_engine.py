"""The session API (c2slm_amd.engine, c2slm.go:20-226) on the GPU against the
same host logic driven by the oracle: text, SeqLen, the token fingerprint
and normX agree over a multi-turn conversation with a stop string, and the
differential-ingestion property of c2slm_test.go:42-108 holds bit for bit."""
import numpy as np
import pytest

from c2slm_amd import _lib as H
from c2slm_amd import engine as E
from c2slm_amd import gguf as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


class OracleCtx:
    """The c2h calls of the engine, answered by the oracle."""

    def __init__(self, orc, desc):
        self.orc = orc
        self.desc = desc
        self.prev = None

    def _normx(self):
        return np.ctypeslib.as_array(O.lib().orc_state_normx(self.orc.state), shape=(self.desc.n_embd,))

    @property
    def seq_len(self):
        return self.orc.seq_len

    def set_seq(self, n):
        self.orc.set_seq_len(n)

    def prefill(self, toks, pos):
        return self.orc.ingest_from(pos, toks)

    def step(self, pos, penalty, im_end, eos):
        self.prev = self._normx().copy()
        self.orc.set_seq_len(pos)
        return int(self.orc.generate(1, im_end, eos, penalty)[0])

    def restore_normx(self):
        self._normx()[:] = self.prev

    def normx(self):
        return self._normx().copy()


@pytest.fixture(scope="module")
def engines(tiny_model_path):
    gpu = E.Engine.new(tiny_model_path, max_ctx=512)
    gf = G.GGUFFile(tiny_model_path)
    orc = O.OracleEngine(gf, max_ctx=512, n_threads=16)
    ref = E.Engine(OracleCtx(orc, gpu.ctx.desc), gf)
    yield gpu, ref, orc
    gpu.close()
    orc.close()


def run_conversation(e, turns, stops):
    out = []
    first = True
    for toks, n_new in turns:
        if first:
            out.append(e.generate_stream(toks, n_new, stops))
            first = False
        else:
            out.append(e.generate_stream_session(toks, n_new, stops))
        out.append(e.seq_len)
    return out


def test_session_matches_oracle(engines):
    gpu, ref, orc = engines
    rng = np.random.default_rng(21)
    turns = [(rng.integers(0, 4093, 24), 12), (rng.integers(0, 4093, 9), 10), (rng.integers(0, 4093, 5), 8)]
    # a stop string that the second turn produces: its third piece
    pieces = []
    ref.generate_stream(turns[0][0], turns[0][1])
    ref.generate_stream_session(turns[1][0], turns[1][1], on_token=lambda p: pieces.append(p) or True)
    stop = pieces[2] if len(pieces) > 2 else b"\xff"
    want = run_conversation(ref, turns, [stop])
    got = run_conversation(gpu, turns, [stop])
    assert got == want, (got, want)
    n = gpu.seq_len
    assert np.array_equal(gpu.ctx.token_ids(0, n), orc.token_ids()[:n])
    assert np.array_equal(bits(gpu.ctx.normx()), bits(ref.ctx.normx()))


def test_differential_ingestion(engines):
    # c2slm_test.go:42-108 on the synthetic model: one-shot and chunked
    # ingestion give the same normX and logits, the fingerprint records the
    # prompt, and a session turn grows the cache
    gpu, _, _ = engines
    rng = np.random.default_rng(22)
    toks = rng.integers(0, 4093, 33).astype(np.int32)
    gpu.ctx.set_seq(0)
    nx_ref = gpu.ingest_from(0, toks)
    lg_ref = gpu.ctx.logits()
    gpu.ctx.set_seq(0)
    split = len(toks) // 2
    gpu.ingest_from(0, toks[:split])
    nx_chunk = gpu.ingest_from(split, toks[split:])
    assert gpu.seq_len == len(toks)
    assert np.array_equal(gpu.ctx.token_ids(0, len(toks)), toks)
    assert np.array_equal(bits(nx_chunk), bits(nx_ref))
    assert np.array_equal(bits(gpu.ctx.logits()), bits(lg_ref))
    before = gpu.seq_len
    gpu.generate_stream_session(rng.integers(0, 4093, 6), 4)
    assert before < gpu.seq_len <= gpu.max_tokens
