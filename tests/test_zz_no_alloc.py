"""c2h_quantize_q8k_noalloc (the entry point that allocates nothing) against
c2h_quantize_q8k, byte for byte, on two calls in a row (the second smaller),
plus the size limit.  Named so that pytest collects it last."""
import numpy as np
import pytest

from c2slm_amd import _lib as H

pytestmark = pytest.mark.gpu


def special_row(rng, cols):
    x = rng.standard_normal(cols).astype(np.float32)
    nb = cols // 256
    if nb >= 4:  # blocks with the quantiser's special cases
        x[256:512] = 0.0                                   # zero block
        x[512:768] = np.float32(-0.0)                      # all -0
        x[768 + 5] = np.inf                                # +Inf amax
        x[768 + 9] = np.nan
    return x


def test_noalloc_matches_quantize_q8k_twice():
    rng = np.random.default_rng(77)
    with H.Ctx(None) as ctx:
        for cols in (4864 + 100, 896):  # second call smaller: stale bytes must not leak
            x = special_row(rng, cols)
            want = ctx.quantize_q8k(x)
            got = ctx.quantize_q8k_noalloc(x)
            assert got.shape == want.shape == ((cols // 256) * 292,)
            assert np.array_equal(got, want), cols


def test_noalloc_limits():
    rng = np.random.default_rng(78)
    with H.Ctx(None) as ctx:
        x = rng.standard_normal(H.NOALLOC_MAX_COLS).astype(np.float32)
        assert np.array_equal(ctx.quantize_q8k_noalloc(x), ctx.quantize_q8k(x))
        assert ctx.quantize_q8k_noalloc(x[:255]).size == 0  # no whole block: nothing written
        with pytest.raises(H.C2hError) as e:
            ctx.quantize_q8k_noalloc(np.zeros(H.NOALLOC_MAX_COLS + 256, np.float32))
        assert e.value.code == -1
