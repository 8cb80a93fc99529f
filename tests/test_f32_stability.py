"""Float64 library calls of the reference, pinned at the float32 level.

The reference rounds float64 results of Go's math.Exp (softmax,
tensor/ops.go:330) and math.Pow/Cos/Sin (the RoPE table,
tensor/ops.go:237-257) to float32; the oracle and the device use glibc and
the HIP device library.  tests/golden/f32_stability.c finds every input
whose exact result lies within the error band of two float64 libraries of
an f32 rounding boundary; at every other input any such library (Go's
included) yields the same float32.  The list is committed in
tests/golden/f32_stability.json and recomputed here:
  exp   all 1,120,924,085 float32 inputs t <= 0 with exp(t) >= 2^-150: one
        exception, t = 0xc16912cd (-14.56709);
  RoPE  every (position < 36,864, frequency) entry at head_dim 64 and 128:
        no exception below position 2,387 (pow within 1 ulp) / 2,387 and 624
        (pow within 4 ulp, head_dim 64 / 128).
The oracle's own table (glibc) must equal the exact rounding at every
stable entry."""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests.golden import make_f32_stability as M


@pytest.fixture(scope="module")
def golden():
    with open(M.OUT) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def computed():
    return M.compute()


def test_exception_lists_recompute(golden, computed):
    assert computed == golden


def test_exp_exceptions_are_few(golden):
    assert golden["exp"]["inputs"] == 1120924085
    assert golden["exp"]["exceptions"] == ["0xc16912cd"]


@pytest.mark.parametrize("hd", [64, 128])
def test_oracle_rope_table_is_the_exact_rounding(golden, hd):
    case = next(r for r in golden["rope"] if r["head_dim"] == hd)
    P, theta = case["positions"], case["theta"]
    half = hd // 2
    cs = np.zeros(P * half, np.float32)
    sn = np.zeros(P * half, np.float32)
    O.lib().orc_rope_table(O.ptr(cs, O.F32P), O.ptr(sn, O.F32P), P, hd, np.float32(theta))
    i = np.arange(half, dtype=np.longdouble)
    F = np.where(i == 0, np.longdouble(1), 1 / np.power(np.longdouble(theta), 2 * i / hd))
    val = np.arange(P, dtype=np.longdouble)[:, None] * F[None, :]
    want_c = np.cos(val).astype(np.float32).reshape(-1)
    want_s = np.sin(val).astype(np.float32).reshape(-1)
    unstable = {(p * half + j, w) for p, j, w in case["list_k1"]}
    bad = [(k, "cos") for k in np.nonzero(cs != want_c)[0] if (k, "cos") not in unstable]
    bad += [(k, "sin") for k in np.nonzero(sn != want_s)[0] if (k, "sin") not in unstable]
    assert not bad, bad[:10]
