"""The composed-function pins of tests/test_oracle_model.py catch plausible
mistakes.  Each case plants one mistake in a copy of the oracle's source
(compiled into a temporary directory with the oracle's own flags; the
oracle itself is untouched) and checks that a pin fails on it, while the
unmodified copy passes."""
import os
import subprocess

import numpy as np
import pytest

from c2slm_amd import gguf as G
from oracle import oracle as O
from tests import test_oracle_model as T
from tests.qwen2_f64 import Qwen2F64, write_pin_model

SRC = os.path.join(os.path.dirname(O.__file__), "c2slm_oracle.c")
AVX2_SRC = os.path.join(os.path.dirname(O.__file__), "c2slm_avx2.c")  # linked unchanged
CFLAGS = ["-O1", "-fPIC", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-mavx2", "-mfma", "-fopenmp",
          "-shared"]

# (name, text in oracle/c2slm_oracle.c, replacement, pin expected to fail)
MUTANTS = [
    ("k bias dropped", "if (L->bk) orc_add_bias(s->k, L->bk, KV);", "", "forward"),
    ("GQA head map h % KVH", "int kvh = h / qpkv;", "int kvh = h % m->n_kv_heads;", "forward"),
    ("RoPE of K skipped", "orc_rope_apply(s->k, KV, m->n_kv_heads, pos, s->cosb, s->sinb, m->max_ctx, hd);", "",
     "forward"),
    ("ffn RMSNorm with attn_norm", "orc_rmsnorm(s->normx, s->x, L->ffn_norm, E, m->eps);",
     "orc_rmsnorm(s->normx, s->x, L->attn_norm, E, m->eps);", "forward"),
    ("attention residual dropped", "for (int i = 0; i < E; ++i) s->x[i] = s->x[i] + s->down[i];",
     "for (int i = 0; i < E; ++i) s->x[i] = s->down[i];", "forward"),
    ("attention scale 1/hd", "float scale = (float)(1.0 / sqrt((double)hd));", "float scale = (float)(1.0 / hd);",
     "forward"),
    ("ingest clamp dropped", "if (pos > s->seq_len) pos = s->seq_len;", "", "ingest"),
    ("im_end not exempt", "t != im_end && t != eos", "t != eos", "penalty"),
    ("penalty window one short", "int start = pos - 64;", "int start = pos - 63;", "penalty_window"),
    ("k QK-norm skipped", "if (L->k_norm)\n", "if (0)\n", "forward_qwen3"),
    ("q QK-norm with the k weights", "orc_rmsnorm(s->q + h * hd, s->q + h * hd, L->q_norm, hd, m->eps)",
     "orc_rmsnorm(s->q + h * hd, s->q + h * hd, L->k_norm, hd, m->eps)", "forward_qwen3"),
]


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    out = {}
    for key, shape in (("qwen2", "q4k_mix"), ("qwen3", "qwen3_hd128")):
        path = str(tmp_path_factory.mktemp("mut") / f"{key}.gguf")
        write_pin_model(path, T.SHAPES[shape], seed=31)
        out[key] = G.GGUFFile(path)
    return out


def build_variant(tmp, name, old, new):
    text = open(SRC).read()
    if old is not None:
        assert text.count(old) >= 1, f"mutation site of '{name}' not found"
        text = text.replace(old, new, 1)
    d = tmp / name.replace(" ", "_").replace("%", "mod").replace("/", "_")
    d.mkdir()
    (d / "o.c").write_text(text)
    so = str(d / "liboracle_variant.so")
    subprocess.run(["gcc", *CFLAGS, "-o", so, str(d / "o.c"), AVX2_SRC, "-lm"], check=True)
    return so


def run_pin(gf, so, which):
    orc = O.OracleEngine(gf, max_ctx=256, n_threads=4, lib_path=so)
    orc.start_q8k_trace()
    ref = Qwen2F64(gf, max_ctx=256)
    try:
        if which in ("forward", "forward_qwen3"):
            rng = np.random.default_rng(5)
            for p, t in enumerate(rng.integers(0, T.V, 6)):
                got = orc.forward(int(t), p)
                ref.feed_q8k(orc.take_q8k_trace())
                assert T.rel_err(got, ref.forward(int(t), p)) <= T.TOL
        elif which == "ingest":
            T.test_ingest_rewind_and_clamp_match_float64((gf, orc, ref))
        elif which == "penalty":
            T.check_exemption_and_repeats(orc, ref)
        elif which == "penalty_window":
            check_window_edge(gf, orc, ref)
    finally:
        orc.close()


def check_window_edge(gf, orc, ref):
    """The penalty window is exactly [pos-64, pos) (c2slm.go:157-162): the
    float64 top token placed at pos-64 alone is penalised out of first place."""
    rng = np.random.default_rng(9)
    prompt = rng.integers(0, T.V, 70).astype(np.int32)
    orc.set_seq_len(0)
    orc.take_q8k_trace()
    nx = orc.ingest_from(0, prompt)
    ref.feed_q8k(orc.take_q8k_trace())
    for p, t in enumerate(prompt):
        ref.forward(int(t), p)
    orc.compute_logits(nx)
    ref.feed_q8k(orc.take_q8k_trace())
    base = ref.logits()
    order = np.argsort(base)[::-1]
    t1 = int(order[0])
    win = prompt.copy()
    win[win == t1] = (t1 + 1) % T.V
    win[70 - 64] = t1
    orc.set_token_ids(0, win)
    want = Qwen2F64.penalise(base, list(win[6:70]), -1, -1, T.PENALTY)
    top2 = np.sort(want)[-2:]
    assert top2[1] - top2[0] > T.TOL * np.max(np.abs(want)), "test logits too close to decide"
    got = orc.generate(1, -1, -1, T.PENALTY)
    assert int(got[0]) == int(np.argmax(want))


def model_for(models, which):
    return models["qwen3" if which.endswith("qwen3") else "qwen2"]


def test_unmodified_copy_passes_every_pin(models, tmp_path):
    so = build_variant(tmp_path, "unmodified", None, None)
    for which in ("forward", "ingest", "penalty", "penalty_window", "forward_qwen3"):
        run_pin(model_for(models, which), so, which)


@pytest.mark.parametrize("name,old,new,which", MUTANTS, ids=[m[0] for m in MUTANTS])
def test_pin_catches_planted_mistake(models, tmp_path, name, old, new, which):
    so = build_variant(tmp_path, name, old, new)
    with pytest.raises(AssertionError):
        run_pin(model_for(models, which), so, which)
