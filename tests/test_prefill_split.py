"""The integer identity batched prefill uses for Q6_K projections
(k_q6_pf_pack / k_pf_gemm_q6): the reference's super-block sum
isum = sum_j sc_j * (s_j - 32 * bsum_j) (c2_tensor_gemv2_q6_k_q8_k_gen.go
:168-203) equals 64 * sum(q8 * hi) + sum(q8 * lo), where B = (q6 - 32) * sc
element by element, hi = B >> 6 and lo = B & 63 both fit int8."""
import numpy as np


def split(q6, sc):
    b = (q6.astype(np.int64) - 32) * sc.astype(np.int64)
    return b >> 6, b & 63, b


def test_split_is_exact_and_fits_int8_for_every_quant_and_scale():
    q6, sc = np.meshgrid(np.arange(64), np.arange(-128, 128), indexing="ij")
    hi, lo, b = split(q6.ravel(), sc.ravel())
    assert np.array_equal(64 * hi + lo, b)
    assert hi.min() >= -128 and hi.max() <= 127
    assert lo.min() >= 0 and lo.max() <= 63
    # the extremes the header states
    assert hi.min() == -64 and hi.max() == 64
    assert b.min() == -4064 and b.max() == 4096


def reference_isum(q6, sc, q8, bsum):
    """c2_tensor_gemv2_q6_k_q8_k_gen.go's integer: per 16-element sub-block
    j, (sum(q6 * q8) - 32 * bsum_j) * sc_j, summed over the 16 sub-blocks."""
    total = 0
    for j in range(16):
        s = int(np.dot(q6[16 * j:16 * j + 16].astype(np.int64), q8[16 * j:16 * j + 16].astype(np.int64)))
        total += (s - 32 * int(bsum[j])) * int(sc[j])
    return total


def test_super_block_sum_through_the_split_equals_the_reference():
    rng = np.random.default_rng(7)
    for case in range(200):
        q6 = rng.integers(0, 64, 256)
        sc = rng.integers(-128, 128, 16)
        q8 = rng.integers(-127, 128, 256)
        if case == 0:  # the largest magnitudes
            q6[:] = 0
            sc[:] = -128
            q8[:] = 127
        bsum = q8.reshape(16, 16).sum(axis=1)
        hi, lo, _ = split(q6, np.repeat(sc, 16))
        got = 64 * int(np.dot(q8, hi)) + int(np.dot(q8, lo))
        want = reference_isum(q6, sc, q8, bsum)
        assert got == want
        # both int8 GEMM accumulators and the combination stay in int32
        assert abs(int(np.dot(q8, hi))) < 2 ** 31 // 64 and abs(got) < 2 ** 31
