"""Kernel parity on the GPU: every result is compared bit for bit with the
oracle on the same inputs (integer sums, Q8_K bytes and fp32 outputs), at
the decode path's real shapes."""
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


def test_rms_scale_every_float(ctx):
    # The RMSNorm scale f32(1/sqrt(f64(v))) of tensor/ops.go:212-214 as the
    # kernels compute it (for normal positive v a reciprocal square root
    # estimate and one Newton step) equals the IEEE square root and division
    # for every one of the 2^32 bit patterns.
    bad, first = ctx.check_rms_scale(0, 1 << 32)
    assert bad == 0, f"{bad} mismatches, first at {first:#010x}"


@pytest.mark.parametrize("cols", [256, 512, 896, 4864, 16384])
def test_quantize_q8k_bitexact(ctx, cols):
    rng = np.random.default_rng(cols)
    x = (rng.normal(size=cols) * rng.uniform(0.01, 1e4)).astype(np.float32)
    got = ctx.quantize_q8k(x)
    want = O.quantize_row_q8k(x)
    assert np.array_equal(got, want)


def test_quantize_q8k_edge_cases(ctx):
    x = np.array([((i % 17) - 8) * 0.125 for i in range(512)], np.float32)  # reference fixture
    assert np.array_equal(ctx.quantize_q8k(x), O.quantize_row_q8k(x))
    z = np.zeros(768, np.float32)
    z[300] = -3.0
    z[600] = np.nan
    z[700] = -0.0
    assert np.array_equal(ctx.quantize_q8k(z), O.quantize_row_q8k(z))
    t = np.full(256, 1e-40, np.float32)  # subnormal block
    t[5] = -2e-39
    assert np.array_equal(ctx.quantize_q8k(t), O.quantize_row_q8k(t))


def special_blocks():
    """Blocks that reach every branch of the quantiser: an infinite amax
    (d = Inf, isc = 0, Inf*0 = NaN quants), a signalling NaN (skipped by the
    amax like a quiet one), an amax below 127/FLT_MAX (isc = Inf, so x*isc is
    +-Inf or NaN), an all -0 block (zero block), and exact halves (amax 127,
    isc 1: x = k + 0.5 rounds away from zero)."""
    rng = np.random.default_rng(77)
    blocks = []
    b = rng.normal(size=256).astype(np.float32)
    b[3] = np.inf
    blocks.append(b)
    b = rng.normal(size=256).astype(np.float32)
    b[9] = -np.inf
    b[10] = np.nan
    blocks.append(b)
    b = rng.normal(size=256).astype(np.float32)
    b.view(np.uint32)[17] = 0x7F800001  # signalling NaN
    b.view(np.uint32)[18] = 0xFFC00001  # negative quiet NaN
    blocks.append(b)
    b = (rng.normal(size=256) * 1e-38).astype(np.float32)  # amax ~ 3e-38 < 127/FLT_MAX
    b[0] = 0.0
    b[1] = -0.0
    blocks.append(b)
    blocks.append(np.full(256, -0.0, np.float32))
    b = np.clip((np.arange(256, dtype=np.float32) - 128.0) + 0.5, -126.5, 126.5)
    b[0] = 127.0
    blocks.append(b.astype(np.float32))
    b = np.full(256, np.nan, np.float32)  # NaNs only: amax 0, a zero block
    blocks.append(b)
    return np.concatenate(blocks)


def test_quantize_q8k_special_blocks(ctx):
    x = special_blocks()
    assert np.array_equal(ctx.quantize_q8k(x), O.quantize_row_q8k(x))
    # the same blocks in every position of a four-block workgroup
    for shift in (1, 2, 3):
        y = np.concatenate([np.zeros(256 * shift, np.float32), x])
        assert np.array_equal(ctx.quantize_q8k(y), O.quantize_row_q8k(y))


SHAPES_Q4K = [(896, 896), (128, 896), (4864, 896), (896, 4864), (7, 512)]


@pytest.mark.parametrize("rows,cols", SHAPES_Q4K)
def test_gemv_q4k_bitexact(ctx, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    nb = cols // 256
    w = G.synth_q4_k(rng, rows * nb)
    x = rng.normal(size=cols).astype(np.float32)
    q8k = O.quantize_row_q8k(x)
    y, isums = ctx.gemv(H.Q4_K, w, q8k, rows, cols, want_isums=True)
    want = O.gemv(w, G.Q4_K, rows, cols, q8k=q8k)
    assert np.array_equal(bits(y), bits(want))
    ws = w.reshape(rows, nb, 144)
    for r in range(0, rows, max(1, rows // 17)):
        for b in range(nb):
            s = np.zeros(8, np.int32)
            O.lib().orc_q4k_block_isums(O.ptr(np.ascontiguousarray(ws[r, b]), O.U8P),
                                        O.ptr(np.ascontiguousarray(q8k[b * 292:(b + 1) * 292]), O.U8P),
                                        O.ptr(s, O.I32P))
            assert np.array_equal(isums[r, b], s), (r, b)


@pytest.mark.parametrize("rows,cols", [(128, 896), (896, 4864), (33, 768)])
def test_gemv_q6k_bitexact(ctx, rows, cols):
    rng = np.random.default_rng(rows * 11 + cols)
    nb = cols // 256
    w = G.synth_q6_k(rng, rows * nb)
    x = rng.normal(size=cols).astype(np.float32)
    q8k = O.quantize_row_q8k(x)
    y, isums = ctx.gemv(H.Q6_K, w, q8k, rows, cols, want_isums=True)
    want = O.gemv(w, G.Q6_K, rows, cols, q8k=q8k)
    assert np.array_equal(bits(y), bits(want))
    ws = w.reshape(rows, nb, 210)
    for r in range(0, rows, max(1, rows // 13)):
        for b in range(nb):
            s = O.lib().orc_q6k_block_isum(O.ptr(np.ascontiguousarray(ws[r, b]), O.U8P),
                                           O.ptr(np.ascontiguousarray(q8k[b * 292:(b + 1) * 292]), O.U8P))
            assert isums[r, b] == s


def test_gemv_q6k_reference_golden(ctx):
    from tests.test_oracle import q6k_golden_weights, ref_fixture_x
    w0, w1 = q6k_golden_weights()
    w = np.concatenate([w0, w1])
    q8k = O.quantize_row_q8k(ref_fixture_x(512))
    y = ctx.gemv(H.Q6_K, w, q8k, 2, 512)
    assert abs(y[0] - (-8705.69238281)) <= 1e-2 and abs(y[1] - 3759.21655273) <= 1e-2
    assert np.array_equal(bits(y), bits(O.gemv(w, G.Q6_K, 2, 512, q8k=q8k)))


@pytest.mark.skipif(not R.ref_available("q4_k"), reason="oracle/_ref not built")
def test_gemv_q4k_unit_vectors_vs_reference_c_oracle(ctx):
    from tests.test_oracle import q4k_fixture_block
    blk = q4k_fixture_block()
    want, _ = R.run_ref_dequant("q4_k", blk.tobytes())
    got = np.empty(256, np.float32)
    for i in range(256):
        got[i] = ctx.gemv(H.Q4_K, blk, R.q8k_onehot(i), 1, 256)[0]
    assert np.array_equal(got, want.astype(np.float32))


@pytest.mark.parametrize("rows,cols", [(4096, 896), (151936, 896), (37, 64)])
def test_gemv_q8_0_bitexact(ctx, rows, cols):
    rng = np.random.default_rng(rows + cols)
    w = G.synth_q8_0(rng, rows * (cols // 32))
    x = rng.normal(size=cols).astype(np.float32)
    y = ctx.gemv(H.Q8_0, w, x, rows, cols)
    if rows > 20000:
        idx = rng.choice(rows, 3000, replace=False)
        rb = (cols // 32) * 34
        sub = np.concatenate([w[i * rb:(i + 1) * rb] for i in idx])
        want = O.gemv(sub, G.Q8_0, len(idx), cols, x=x)
        assert np.array_equal(bits(y[idx]), bits(want))
    else:
        assert np.array_equal(bits(y), bits(O.gemv(w, G.Q8_0, rows, cols, x=x)))


def test_gemv_q8_0_order_known_answers(ctx):
    from tests.test_oracle import q8_0_row
    big = float(2 ** 24)
    one = q8_0_row(np.ones(96))
    cases = []
    x = np.zeros(96, np.float32)
    x[[0, 8, 16, 24]] = [big, 1, 1, 1]
    cases.append((x, big + 2))
    x = np.zeros(96, np.float32)
    x[0] = big
    x[1:8] = 1
    cases.append((x, big))
    x = np.zeros(96, np.float32)
    x[0] = big
    x[32] = 1
    x[64] = 1
    cases.append((x, big))
    for x, want in cases:
        assert ctx.gemv(H.Q8_0, one, x, 1, 96)[0] == want


@pytest.mark.parametrize("rows,cols", [(896, 896), (128, 896), (4864, 896), (896, 4864), (9, 64)])
def test_gemv_q5_0_bitexact(ctx, rows, cols):
    # tensor/ops.go:25-74 on f32 x (the real-model format of 896-wide matrices)
    rng = np.random.default_rng(rows + cols)
    w = G.synth_q5_0(rng, rows * (cols // 32))
    x = rng.normal(size=cols).astype(np.float32)
    got = ctx.gemv(H.Q5_0, w, x, rows, cols)
    want = O.gemv(w, G.Q5_0, rows, cols, x=x)
    assert np.array_equal(bits(got), bits(want))


def test_gemv_q5_0_order_known_answers(ctx):
    from tests.test_oracle import q5_0_block
    ones = q5_0_block(0x3C00, 0xFFFFFFFF, [0x11] * 16)
    big = np.float32(2 ** 24)
    cases = [([0, 16, 1], [1, big, 1], big), ([0, 1, 17], [big, 3, -1], big + 4)]
    for idx, vals, want in cases:
        x = np.zeros(32, np.float32)
        x[idx] = vals
        assert ctx.gemv(H.Q5_0, ones, x, 1, 32)[0] == want
    qs = [0x11] * 16
    qs[0] = 0x3D
    blk = q5_0_block(0x3C00, 0xFFFFFFFE, qs)
    x = np.zeros(32, np.float32)
    x[0] = 1.0
    x[16] = np.float32(1 + 2 ** -23)
    assert ctx.gemv(H.Q5_0, blk, x, 1, 32)[0] == np.float32(2.0 ** -21)
