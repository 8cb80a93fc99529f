"""Float-x row dots on the GPU -- engine.DispatchGEMV without a worker pool
(engine/model.go:250-270) and the restricted-token logits
(engine/forward.go:171-212) -- against the oracle, bit for bit, through the
C ABI (c2h_gemv_f32, c2h_logits_ids)."""
import numpy as np
import pytest

from c2slm_amd import _lib as H
from c2slm_amd import gguf as G
from oracle import oracle as O
from tests import refdequant as R

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = H.Ctx(None)
    yield c
    c.close()


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


SYNTH = {H.Q4_K: (G.synth_q4_k, 256), H.Q6_K: (G.synth_q6_k, 256), H.Q8_0: (G.synth_q8_0, 32),
         H.Q5_0: (G.synth_q5_0, 32)}

CASES = [
    (H.Q4_K, 4864, 896),   # 896 columns: three whole super-blocks, the tail ignored
    (H.Q4_K, 896, 4864),
    (H.Q4_K, 33, 1000),
    (H.Q6_K, 896, 4864),
    (H.Q6_K, 128, 896),
    (H.Q6_K, 31, 300),
    (H.Q8_0, 4096, 896),
    (H.Q8_0, 70, 4864),    # 152 blocks per row
    (H.Q8_0, 5, 40),
    (H.Q5_0, 896, 896),
    (H.Q5_0, 41, 4864),
    (H.Q5_0, 3, 96),
    (H.Q4_K, 9, 16384),
    (H.Q6_K, 5, 32768),    # the largest row the kernels stage
    (H.Q8_0, 3, 32768),
]


@pytest.mark.parametrize("typ,rows,cols", CASES)
def test_gemv_f32_bitexact(ctx, typ, rows, cols):
    synth, qk = SYNTH[typ]
    rng = np.random.default_rng(rows * 31 + cols + typ)
    w = synth(rng, rows * (cols // qk))
    x = (rng.normal(size=cols) * rng.uniform(0.1, 10)).astype(np.float32)
    got = ctx.gemv_f32(typ, w, x, rows, cols)
    want = O.gemv(w, typ, rows, cols, x=x, float_x=True)
    assert np.array_equal(bits(got), bits(want))


def test_gemv_f32_rejects_rows_beyond_the_lds_limit(ctx):
    with pytest.raises(H.C2hError):
        ctx.gemv_f32(H.Q8_0, np.zeros(3 * 1026 * 34, np.uint8), np.zeros(32832, np.float32), 3, 32832)


def test_gemv_f32_zero_fallbacks(ctx):
    x = np.ones(128, np.float32)
    # fewer than 256 columns: no whole super-block, every dot is 0
    assert np.array_equal(ctx.gemv_f32(H.Q4_K, np.zeros(144, np.uint8), x, 3, 128), np.zeros(3, np.float32))
    assert np.array_equal(ctx.gemv_f32(H.Q6_K, np.zeros(210, np.uint8), x, 2, 128), np.zeros(2, np.float32))
    # a type DispatchGEMV has no float row function for: zeros
    assert np.array_equal(ctx.gemv_f32(H.F32, np.zeros(512, np.uint8), x, 4, 128), np.zeros(4, np.float32))


def test_gemv_f32_order_known_answers(ctx):
    from tests.test_oracle import q4k_ones_block, q6k_ones_block
    big = float(2 ** 24)
    q4 = q4k_ones_block()
    q6 = q6k_ones_block()
    cases = [
        (H.Q4_K, q4, {0: big, 8: 1, 16: 1, 24: 1}, big + 2),
        (H.Q4_K, q4, {0: big, **{i: 1 for i in range(1, 8)}}, big),
        (H.Q4_K, q4, {0: big, 32: 1, 64: 1}, big),
        (H.Q4_K, q4, {32: big, 40: 1, 48: 1, 56: 1}, big + 2),
        (H.Q6_K, q6, {0: big, 16: 1, 24: 1}, big + 2),
        (H.Q6_K, q6, {0: big, 8: 1, 16: 1}, big),
        (H.Q6_K, q6, {0: big, 32: 1, 64: 1, 96: 1}, big + 2),
        (H.Q6_K, q6, {0: big, **{i: 1 for i in range(1, 8)}}, big),
    ]
    for typ, blk, xs, want in cases:
        x = np.zeros(256, np.float32)
        for k, v in xs.items():
            x[k] = v
        assert ctx.gemv_f32(typ, blk, x, 1, 256)[0] == want, (typ, xs)
    # rounding of the min term and of (q*(d*sc))*x
    blk = q4k_ones_block(dmin_bits=0x3C00, nib=0x33)
    blk[4:16] = 1
    x = np.zeros(256, np.float32)
    x[0] = np.float32(1 + 2 ** -23)
    assert ctx.gemv_f32(H.Q4_K, blk, x, 1, 256)[0] == np.float32(np.float32(3) * x[0]) - x[0]
    blk = q6k_ones_block()
    blk[0:128] = 0x33
    blk[192:208] = 3
    assert ctx.gemv_f32(H.Q6_K, blk, x, 1, 256)[0] == np.float32(np.float32(9) * x[0])


@pytest.mark.skipif(not (R.ref_available("q4_k") and R.ref_available("q6_k")), reason="oracle/_ref not built")
def test_gemv_f32_unit_vectors_vs_reference_c_oracle(ctx):
    from tests.test_oracle import hostile_blocks, q4k_fixture_block, q6k_fixture_block
    sets = [(H.Q4_K, "q4_k", [q4k_fixture_block()] + hostile_blocks(144, [(0, [0x00, 0x3C]), (2, [0x00, 0x38])])),
            (H.Q6_K, "q6_k", [q6k_fixture_block()] + hostile_blocks(210, [(208, [0x00, 0x3C])]))]
    eye = np.eye(256, dtype=np.float32)
    for typ, name, blocks in sets:
        for blk in blocks:
            want, _ = R.run_ref_dequant(name, blk.tobytes())
            # x = e_i: the dot is the i-th dequantised weight
            got = np.array([ctx.gemv_f32(typ, blk, eye[i], 1, 256)[0] for i in range(256)], np.float32)
            assert np.array_equal(got, want.astype(np.float32)), name


def test_time_dot_rows_matches_plain_calls(ctx):
    rng = np.random.default_rng(8)
    rows, cols = 300, 896
    w = G.synth_q8_0(rng, rows * 28)
    x = rng.normal(size=cols).astype(np.float32)
    want = ctx.gemv_f32(H.Q8_0, w, x, rows, cols)
    ms, y = ctx.time_dot_rows(H.Q8_0, w, x, rows, cols, iters=3, flush_bytes=1 << 20)
    assert ms > 0 and np.array_equal(bits(y), bits(want))
    ids = np.array([7, 0, 299, 7, 150], np.int32)
    ms, y = ctx.time_dot_rows(H.Q8_0, w, x, rows, cols, ids=ids, iters=2)
    assert ms > 0 and np.array_equal(bits(y), bits(want[ids]))
