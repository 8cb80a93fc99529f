"""GPU parity at the edges of the greedy step and of the fp16 decode, against
the oracle, through the C ABI.

Greedy step (c2slm.go:153-180, the fused vocab kernel and the argmax
reduction in layer 0's prologue), on a 2-layer model with the full
151,936-row vocabulary so the vocab grid is the bench's (475 workgroups
walking 4,748 tiles of 32 rows):
  ties      copies of the winning row at lower ids -- in its tile, in the
            tile 475 before (the same workgroup), in the tile before (another
            workgroup) and in tile 1 -- the lowest id wins;
  NaN at 0  a NaN scale in row 0 makes logits[0] NaN: the step returns 0;
  NaN/Inf   NaN rows never win; -Inf rows never win; of two +Inf rows in
            different workgroups the lower id wins;
  window    the penalty per occurrence over TokenIDs[pos-64, pos), the
            im_end and eos exemptions, and the window's first position.
Each case first checks on the oracle that it decides what it is meant to
test, then compares the device's tokens with the oracle's.

fp16 decode, all 65,536 patterns as block scales: Q8_0 rows through
c2h_gemv (k_gemv_f) and c2h_gemv_f32 (k_dot_rows) -- the simd lookup table,
-0 -> +0 (c2_tensor_dot_q8_0_gen.go:16-70) -- Q4_K d and dmin and Q6_K d
through c2h_gemv, and a model whose tied embedding holds every pattern:
the embedding (tensor.FP16ToF32, -0 kept, tensor/fp16.go:16-50) through
c2h_forward's normX and the vocab kernel through c2h_logits.  Results are
bit-exact; NaN results are compared as NaN (a Q8_0 NaN scale's payload may
differ: the device converts with the hardware instruction)."""
import os
import shutil

import numpy as np
import pytest

from c2slm_amd import _lib as H
from c2slm_amd import gguf as G
from oracle import oracle as O
from tests import refdequant as R
from tests.qwen2_f64 import pack_q4k_scales
from tests.test_gpu_model import bits, open_pair

pytestmark = pytest.mark.gpu

PENALTY = 1.15
V = 151936
E = 896
ROW = 28 * 34  # native Q8_0 row bytes at 896 columns
P0 = 70        # prompt length: decoding at pos 70 reads the window [6, 70)


def nan_equal(a, b) -> bool:
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(bits(a[~na]), bits(b[~nb])))


# ------------------------------------------------------------ step edges

@pytest.fixture(scope="module")
def base(tmp_path_factory):
    d = tmp_path_factory.mktemp("edges")
    path = str(d / "base.gguf")
    G.write_synthetic_model(path, G.ModelShape(n_layers=2, n_vocab=V), seed=41)
    prompt = np.random.default_rng(41).integers(100000, 150000, P0).astype(np.int32)
    return path, prompt, d


def emb_row(gf, r: int) -> np.ndarray:
    return np.array(gf.tensor_map["token_embd.weight"].data[r * ROW:(r + 1) * ROW])


def write_patched(src: str, dst: str, rows: dict) -> None:
    shutil.copyfile(src, dst)
    gf = G.GGUFFile(src)
    base = gf.data_offset + gf.tensor_map["token_embd.weight"].offset
    mm = np.memmap(dst, dtype=np.uint8, mode="r+")
    for r, row in rows.items():
        mm[base + r * ROW:base + (r + 1) * ROW] = row
    mm.flush()
    del mm


def oracle_after_prompt(path, prompt):
    gf = G.GGUFFile(path)
    orc = O.OracleEngine(gf, max_ctx=128, n_threads=16)
    nx = orc.ingest_from(0, prompt)
    return gf, orc, nx


def penalised_f32(lg, window, im_end, eos):
    lg = np.array(lg, np.float32)
    p = np.float32(PENALTY)
    for t in window:
        if 0 <= t < len(lg) and t != im_end and t != eos:
            lg[t] = lg[t] / p if lg[t] > 0 else lg[t] * p
    return lg


def run_steps(path, prompt, n, im_end=None, eos=None, token_ids=None):
    """(device tokens, oracle tokens) of n greedy steps after the prompt;
    token_ids optionally replaces TokenIDs[0, P0) (the penalty window)
    after the ingest on both sides."""
    gf, ctx, orc, im0, eos0 = open_pair(path, 128)
    im_end = im0 if im_end is None else im_end
    eos = eos0 if eos is None else eos
    try:
        nx = ctx.prefill(prompt, 0)
        want_nx = orc.ingest_from(0, prompt)
        assert np.array_equal(bits(nx), bits(want_nx))
        if token_ids is not None:
            ctx.set_token_ids(0, token_ids)
            orc.set_token_ids(0, token_ids)
        want = orc.generate(n, im_end, eos, PENALTY)
        got = []
        for i in range(n):
            t = ctx.step(P0 + i, PENALTY, im_end, eos)
            got.append(t)
            if t in (im_end, eos):
                break
        return np.array(got, np.int32), want
    finally:
        ctx.close()
        orc.close()


def tie_case(path, prompt):
    """(rows to patch, expected winner): copies of the winning row at lower ids."""
    gf, orc, nx = oracle_after_prompt(path, prompt)
    _, im_end, eos = G.special_token_ids(gf)
    lg = penalised_f32(orc.compute_logits(nx), prompt[P0 - 64:], im_end, eos)
    orc.close()
    taken = set(prompt.tolist())
    r = int(np.argmax(lg))
    assert r not in taken and r % 32 >= 2 and r >= 32 * 476, "pick another seed: winner unsuited"
    row = emb_row(gf, r)
    copies = []
    for c in (r - 1, r - 32 * 475, r - 32, 32 + 5):
        while c in taken:
            c -= 1
        copies.append(c)
    return {c: row for c in copies}, min(copies)


def test_argmax_ties_lowest_id_across_tiles_and_workgroups(base):
    path, prompt, d = base
    rows, winner = tie_case(path, prompt)
    p = str(d / "ties.gguf")
    write_patched(path, p, rows)
    got, want = run_steps(p, prompt, 6)
    assert int(want[0]) == winner  # the oracle resolves the tie to the lowest id
    assert np.array_equal(got, want)


@pytest.mark.parametrize("pattern", [0x7E00, 0x7C01, 0xFE00])
def test_nan_logit_at_id_0_returns_0(base, pattern):
    path, prompt, d = base
    gf = G.GGUFFile(path)
    row = emb_row(gf, 0)
    row[0:2] = np.frombuffer(np.uint16(pattern).tobytes(), np.uint8)
    p = str(d / f"nan0_{pattern:x}.gguf")
    write_patched(path, p, {0: row})
    got, want = run_steps(p, prompt, 3)
    assert list(want) == [0, 0, 0]
    assert np.array_equal(got, want)


def inf_row(row, nx, sign):
    """Block 0 of the row scaled by +Inf with quants of the sign of
    sign*x[0:32]: every lane's partial sum has that sign, the logit is
    sign*Inf."""
    out = row.copy()
    out[0:2] = np.frombuffer(np.uint16(0x7C00).tobytes(), np.uint8)
    q = np.where(sign * np.asarray(nx[:32]) >= 0, 127, -127).astype(np.int8)
    out[2:34] = q.view(np.uint8)
    return out


def test_nan_and_minus_inf_rows_never_win(base):
    path, prompt, d = base
    gf, orc, nx = oracle_after_prompt(path, prompt)
    _, im_end, eos = G.special_token_ids(gf)
    lg = penalised_f32(orc.compute_logits(nx), prompt[P0 - 64:], im_end, eos)
    orc.close()
    top = [int(i) for i in np.argsort(lg)[::-1][:4]]
    rows = {}
    for i, r in enumerate(top[:3]):  # the three best rows: NaN, NaN, -Inf
        row = emb_row(gf, r)
        if i < 2:
            row[0:2] = np.frombuffer(np.uint16(0x7E00 if i == 0 else 0xFD00).tobytes(), np.uint8)
            rows[r] = row
        else:
            rows[r] = inf_row(row, nx, -1.0)
    p = str(d / "naninf.gguf")
    write_patched(path, p, rows)
    got, want = run_steps(p, prompt, 4)
    assert int(want[0]) == top[3]
    assert np.array_equal(got, want)


def test_plus_inf_rows_lowest_id_wins(base):
    path, prompt, d = base
    gf, orc, nx = oracle_after_prompt(path, prompt)
    orc.close()
    i1, i2 = 32 * 474 + 3, 32 * 475 + 3  # tiles 474 and 475: different workgroups
    rows = {i1: inf_row(emb_row(gf, i1), nx, 1.0), i2: inf_row(emb_row(gf, i2), nx, 1.0)}
    p = str(d / "pinf.gguf")
    write_patched(path, p, rows)
    got, want = run_steps(p, prompt, 3)
    assert int(want[0]) == i1
    assert np.array_equal(got, want)


def window_case(path, prompt):
    """(t1, t2, k): the top two raw logits (both positive) and the fewest
    occurrences of t1 that let t2 win."""
    gf, orc, nx = oracle_after_prompt(path, prompt)
    lg = np.array(orc.compute_logits(nx), np.float32)
    orc.close()
    order = [int(i) for i in np.argsort(lg)[::-1]]
    t1, t2 = order[0], order[1]
    assert lg[t1] > 0 and lg[t2] > 0
    v, k = lg[t1], 0
    while v >= lg[t2]:
        v = v / np.float32(PENALTY)
        k += 1
    assert 1 <= k <= 6, k
    return t1, t2, k


@pytest.mark.parametrize("case", ["penalised", "im_end_exempt", "eos_exempt", "outside_window", "window_start"])
def test_penalty_window_and_exemptions(base, case):
    path, prompt, d = base
    gf = G.GGUFFile(path)
    _, im_end, eos = G.special_token_ids(gf)
    t1, t2, k = window_case(path, prompt)
    # the window [6, 70) without t1 and t2, then k occurrences of t1
    ids = np.where(np.isin(prompt, [t1, t2]), 100000, prompt).astype(np.int32)
    if case == "outside_window":
        ids[6 - k:6] = t1    # the k positions just before the window's first (6)
    elif case == "window_start":
        ids[6:6 + k] = t1    # from the window's first position on
    else:
        ids[30:30 + k] = t1
    kw = {}
    if case == "im_end_exempt":
        kw["im_end"] = t1
    if case == "eos_exempt":
        kw["eos"] = t1
    got, want = run_steps(path, prompt, 2, token_ids=ids, **kw)
    expect_t1 = case in ("im_end_exempt", "eos_exempt", "outside_window")
    assert (int(want[0]) == t1) == expect_t1, (case, int(want[0]), t1, t2, k)
    assert np.array_equal(got, want)


# ------------------------------------------------------------ fp16 decode

ALL = np.arange(65536, dtype=np.uint32)


def q8_0_onehot_rows(patterns) -> np.ndarray:
    """One 32-column Q8_0 block per row: scale = pattern, quants (1, 0, ..)."""
    w = np.zeros((len(patterns), 34), np.uint8)
    w[:, 0:2] = np.asarray(patterns, np.uint16).view(np.uint8).reshape(-1, 2)
    w[:, 2] = 1
    return w.reshape(-1)


def simd_lut(patterns) -> np.ndarray:
    """The simd kernels' table: IEEE half -> float, both zeros to +0."""
    f = np.asarray(patterns, np.uint16).view(np.float16).astype(np.float32)
    return np.where(f == 0, np.float32(0), f)


def test_fp16_all_patterns_q8_0_gemvs():
    w = q8_0_onehot_rows(ALL)
    x = np.zeros(32, np.float32)
    x[0] = 1.0
    want = O.gemv(w, G.Q8_0, 65536, 32, x=x)
    assert nan_equal(want[~np.isnan(want)], simd_lut(ALL)[~np.isnan(want)])  # the oracle is the table
    with H.Ctx(None) as ctx:
        assert nan_equal(ctx.gemv(G.Q8_0, w, x, 65536, 32), want)
        assert nan_equal(ctx.gemv_f32(G.Q8_0, w, x, 65536, 32), want)


def q4k_onehot_rows(d, dmin) -> np.ndarray:
    """One super-block per row: d, dmin; scale and min of sub-block 0 are 1,
    the quant of element 0 is 1, every other quant 0."""
    n = len(d)
    w = np.zeros((n, 144), np.uint8)
    w[:, 0:2] = np.asarray(d, np.uint16).view(np.uint8).reshape(-1, 2)
    w[:, 2:4] = np.asarray(dmin, np.uint16).view(np.uint8).reshape(-1, 2)
    sc = np.zeros((n, 8), np.int64)
    sc[:, 0] = 1
    w[:, 4:16] = pack_q4k_scales(sc, sc)
    w[:, 16] = 1
    return w.reshape(-1)


def q6k_onehot_rows(d) -> np.ndarray:
    """One super-block per row: scale d, every 6-bit quant 32 (weight 0)
    except element 0's 33, every int8 sub-block scale 1."""
    n = len(d)
    w = np.zeros((n, 210), np.uint8)
    w[:, 0] = 1                 # ql: element 0's low nibble 1, the rest 0
    w[:, 128:192] = 0xAA        # qh: high bits 2 for every element (16 + ...)
    w[:, 192:208] = 1
    w[:, 208:210] = np.asarray(d, np.uint16).view(np.uint8).reshape(-1, 2)
    return w.reshape(-1)


@pytest.mark.parametrize("which", ["q4k_d", "q4k_dmin", "q6k_d"])
def test_fp16_all_patterns_k_quant_scales(which):
    xq = R.q8k_onehot(0)
    if which == "q4k_d":
        t, w = G.Q4_K, q4k_onehot_rows(ALL, np.zeros(65536))
    elif which == "q4k_dmin":
        t, w = G.Q4_K, q4k_onehot_rows(np.zeros(65536), ALL)
    else:
        t, w = G.Q6_K, q6k_onehot_rows(ALL)
    want = O.gemv(w, t, 65536, 256, q8k=xq)
    with H.Ctx(None) as ctx:
        got = ctx.gemv(t, w, xq, 65536, 256)
    assert nan_equal(got, want)
    f = ALL.astype(np.uint16).view(np.float16).astype(np.float32)
    fin = np.isfinite(f)
    expect = {"q4k_d": f, "q4k_dmin": -f, "q6k_d": f}[which]
    assert np.array_equal(np.abs(want[fin]), np.abs(expect[fin]))  # the decode itself, up to the sign of zero


def embedding_model(path) -> tuple:
    """1 layer, all projection weights zero, so normX = RMSNorm(embedding):
    rows of the tied Q8_0 embedding hold all 65,536 fp16 patterns as block
    scales with quants (1, 0, ..): the finite ones 28 to a row in order of
    magnitude, each Inf/NaN pattern alone in its row."""
    pats = ALL.astype(np.uint16)
    f = pats.view(np.float16).astype(np.float32)
    fin = pats[np.isfinite(f)]
    fin = fin[np.lexsort((fin >> 15, np.abs(fin.view(np.float16).astype(np.float32))))]
    special = pats[~np.isfinite(f)]
    n_fin_rows = -(-len(fin) // 28)
    rows = []
    for i in range(n_fin_rows):
        blk = fin[i * 28:(i + 1) * 28]
        rows.append(np.concatenate([blk, np.full(28 - len(blk), 0x3C00, np.uint16)]))
    for s in special:
        r = np.zeros(28, np.uint16)
        r[0] = s
        rows.append(r)
    nv = len(rows) + 4
    for _ in range(4):
        rows.append(np.full(28, 0x3C00, np.uint16))
    scales = np.stack(rows)                         # [nv, 28]
    emb = np.zeros((nv, 28, 34), np.uint8)
    emb[:, :, 0:2] = scales.view(np.uint8).reshape(nv, 28, 2)
    emb[:, :, 2] = 1
    shape = G.ModelShape(n_layers=1, n_vocab=nv)
    KV = shape.n_kv_heads * shape.head_dim
    F = shape.n_ff
    t = []

    def zero_quant(name, tt, r, c):
        t.append((name, [c, r], tt, np.zeros(G.tensor_byte_size(tt, [c, r]), np.uint8)))

    def f32(name, v):
        t.append((name, [len(v)], G.F32, np.asarray(v, "<f4").view(np.uint8)))

    t.append(("token_embd.weight", [E, nv], G.Q8_0, emb.reshape(-1)))
    f32("output_norm.weight", np.ones(E))
    f32("blk.0.attn_norm.weight", np.ones(E))
    zero_quant("blk.0.attn_q.weight", G.Q4_K, E, E)
    f32("blk.0.attn_q.bias", np.zeros(E))
    zero_quant("blk.0.attn_k.weight", G.Q4_K, KV, E)
    f32("blk.0.attn_k.bias", np.zeros(KV))
    zero_quant("blk.0.attn_v.weight", G.Q6_K, KV, E)
    f32("blk.0.attn_v.bias", np.zeros(KV))
    zero_quant("blk.0.attn_output.weight", G.Q4_K, E, E)
    f32("blk.0.ffn_norm.weight", np.ones(E))
    zero_quant("blk.0.ffn_gate.weight", G.Q4_K, F, E)
    zero_quant("blk.0.ffn_up.weight", G.Q4_K, F, E)
    zero_quant("blk.0.ffn_down.weight", G.Q6_K, E, F)
    md = [("general.architecture", G.T_STR, "qwen2"), ("general.alignment", G.T_U32, 32),
          ("qwen2.block_count", G.T_U32, 1), ("qwen2.embedding_length", G.T_U32, E),
          ("qwen2.feed_forward_length", G.T_U32, F), ("qwen2.attention.head_count", G.T_U32, 14),
          ("qwen2.attention.head_count_kv", G.T_U32, 2), ("qwen2.rope.freq_base", G.T_F32, 1.0e6),
          ("qwen2.attention.layer_norm_rms_epsilon", G.T_F32, 1.0e-6),
          ("tokenizer.ggml.model", G.T_STR, "gpt2"), ("tokenizer.ggml.tokens", G.T_ARR, (G.T_STR, G.token_list(nv)))]
    G.write_gguf(path, md, t)
    return nv, n_fin_rows


def test_fp16_all_patterns_embedding_and_vocab_kernel(tmp_path):
    path = str(tmp_path / "fp16.gguf")
    nv, n_fin_rows = embedding_model(path)
    gf, ctx, orc, _, _ = open_pair(path, 8)
    try:
        bad = []
        for tok in range(nv):
            got = ctx.forward(tok, 0)
            want = orc.forward(tok, 0)
            if not nan_equal(got, want):
                bad.append(tok)
        assert not bad, bad[:10]
        # the vocab kernel over every pattern, on the normX of a row of scales near 1
        tok = int(n_fin_rows * 0.75)  # scales of magnitude ~2^8
        nx = orc.forward(tok, 0)
        ctx.forward(tok, 0)
        assert nan_equal(ctx.logits(), orc.compute_logits(nx))
    finally:
        ctx.close()
        orc.close()
