"""The CPU baseline's kernels (oracle/c2slm_avx2.c: the reference's AVX2
GEMV branches restated with VPMADDUBSW / VPMADDWD and 8-lane float vectors)
against the scalar oracle they must equal bit for bit: the Q4_K and Q6_K
integer sums and dots on random and extreme blocks, the Q8_0 dot on the
8-lane order's known answers, and a whole greedy stream of an engine that
runs them."""
import numpy as np

from c2slm_amd import gguf as G
from oracle import oracle as O

L = O.lib()
U8P, F32P = O.U8P, O.F32P


def q8k_of(x):
    return O.quantize_row_q8k(np.asarray(x, np.float32))


def test_q4k_q6k_dots_equal_the_scalar_oracle():
    rng = np.random.default_rng(41)
    for cols in (256, 896, 4864):
        nb = cols // 256
        for case in range(12):
            x = rng.normal(size=cols).astype(np.float32) * (10.0 ** rng.integers(-3, 3))
            if case == 0:
                x[:] = 1.0  # every quant 127
            if case == 1:
                x[:] = -1.0  # every quant -127
            q8 = q8k_of(x)
            for t, synth, bs in ((G.Q4_K, G.synth_q4_k, 144), (G.Q6_K, G.synth_q6_k, 210)):
                w = synth(rng, nb)
                if case in (0, 1):  # the largest products: every nibble 15 / every q6 0 and 63
                    for b in range(nb):
                        blk = w[b * bs:(b + 1) * bs]
                        if t == G.Q4_K:
                            blk[16:144] = 0xFF
                        else:
                            blk[0:192] = 0xFF if case == 0 else 0x00
                scalar = L.orc_dot_q4k_q8k if t == G.Q4_K else L.orc_dot_q6k_q8k
                avx2 = L.orc_avx2_dot_q4k_q8k if t == G.Q4_K else L.orc_avx2_dot_q6k_q8k
                a = scalar(O.ptr(w, U8P), O.ptr(q8, U8P), cols)
                b = avx2(O.ptr(w, U8P), O.ptr(q8, U8P), cols)
                assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), (t, cols, case)
                if t == G.Q6_K:
                    for blk in range(nb):
                        wp = O.ptr(w[blk * 210:], U8P)
                        qp = O.ptr(q8[blk * 292:], U8P)
                        assert L.orc_q6k_block_isum(wp, qp) == L.orc_avx2_q6k_block_isum(wp, qp)


def test_q8_0_dot_equals_the_scalar_oracle():
    rng = np.random.default_rng(42)
    for cols in (32, 96, 896):
        nb = cols // 32
        for case in range(20):
            w = G.synth_q8_0(rng, nb)
            x = rng.normal(size=cols).astype(np.float32) * np.float32(10.0 ** rng.integers(-4, 4))
            if case == 0:  # values whose sums round differently under another association
                x[:] = np.float32(1.0) + np.float32(2 ** -22) * np.arange(cols, dtype=np.float32)
            a = L.orc_dot_q8_0(O.ptr(w, U8P), O.ptr(x, F32P), cols)
            b = L.orc_avx2_dot_q8_0(O.ptr(w, U8P), O.ptr(x, F32P), cols)
            assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), (cols, case)


def test_engine_with_avx2_dots_equals_the_scalar_engine(tiny_model_path):
    gf = G.GGUFFile(tiny_model_path)
    _, im_end, eos = G.special_token_ids(gf)
    prompt = np.random.default_rng(43).integers(0, 4096, 12).astype(np.int32)
    out = []
    for avx2 in (False, True):
        orc = O.OracleEngine(gf, max_ctx=128, n_threads=4, avx2_dots=avx2)
        try:
            nx = orc.ingest_from(0, prompt)
            toks = orc.generate(12, im_end, eos, 1.15)
            lg = orc.compute_logits(nx)
            out.append((np.asarray(nx, np.float32).copy(), np.asarray(toks).copy(), np.asarray(lg, np.float32).copy()))
        finally:
            orc.close()
    (n0, t0, l0), (n1, t1, l1) = out
    assert np.array_equal(n0.view(np.uint32), n1.view(np.uint32))
    assert np.array_equal(t0, t1)
    assert np.array_equal(l0.view(np.uint32), l1.view(np.uint32))
