"""Pins the integer oracle of the fast int8 path (two int8 digits per activation, exact i32
sums, one shared dequantisation) with numpy's int64 products, invariants of the digit split,
and its distance from the fused reference semantics."""
import math

import numpy as np
import pytest

from helpers import int8_weights, normal, pack_int8, rel_norm_err

INT8 = 3
NONE, RELU, SILU = range(3)


def test_digits_are_the_rounded_scaled_row(orc):
    rng = np.random.default_rng(0)
    rows = [normal(rng, 300), normal(rng, 300) * np.float32(1e-30), normal(rng, 300) * np.float32(3e30),
            np.float32(2.0) ** rng.integers(-149, 127, 300).astype(np.float32),
            np.full(300, 32639.0, np.float32), np.linspace(-1, 1, 300, dtype=np.float32)]
    a = np.stack(rows).astype(np.float32)
    m, k = a.shape
    hi, lo, ex = orc.quantize_rows(a, k, m, k)
    for r in range(m):
        e = int(ex[r])
        scaled = a[r].astype(np.float64) * 2.0**e  # exact: a power-of-two scaling in f64
        v = np.rint(scaled).astype(np.int64)  # round half to even
        assert np.array_equal(hi[r].astype(np.int64) * 256 + lo[r], v), r
        assert np.abs(v).max() <= 32639
        amax = np.abs(a[r].astype(np.float64)).max()
        assert amax * 2.0 ** (e + 1) > 32639  # the largest exponent that fits
        assert lo[r].min() >= -128 and lo[r].max() <= 127


def test_zero_and_nonfinite_rows(orc):
    a = np.zeros((3, 8), np.float32)
    a[1, 3] = np.nan
    a[2, 5] = -np.inf
    hi, lo, ex = orc.quantize_rows(a, 8, 3, 8)
    assert ex[0] == 0 and ex[1] == orc.EXP_NONFINITE and ex[2] == orc.EXP_NONFINITE
    assert np.all(hi == 0) and np.all(lo == 0)
    assert np.isnan(orc.dequant(5, 7, orc.EXP_NONFINITE, 0.01))
    # An exact zero sum is +0 whatever the scale's sign, as the reference's sums start at +0.
    assert orc.dequant(0, 0, 3, -0.5).view(np.uint32) == 0


def test_integer_products_match_numpy(orc):
    rng = np.random.default_rng(1)
    m, k, n = 9, 333, 21
    hi = rng.integers(-128, 128, (m, k)).astype(np.int8)
    lo = rng.integers(-128, 128, (m, k)).astype(np.int8)
    q = rng.integers(-128, 128, (n, k)).astype(np.int8)
    ah, al = orc.int_products(hi, lo, q)
    assert np.array_equal(ah, hi.astype(np.int64) @ q.astype(np.int64).T)
    assert np.array_equal(al, lo.astype(np.int64) @ q.astype(np.int64).T)


def test_dequantisation_is_one_rounding_of_the_exact_sum_then_exact_scaling(orc):
    rng = np.random.default_rng(2)
    for _ in range(2000):
        ah, al = (int(x) for x in rng.integers(-2**30, 2**30, 2))
        e = int(rng.integers(-100, 120))
        s = np.float32(rng.random() * 0.01 + 1e-4)
        got = orc.dequant(ah, al, e, s)
        exact = (ah * 256 + al)
        t = np.float32(exact)  # int -> f64 exact here (|x| < 2^53), then one RNE to f32
        assert np.float64(t) == float(np.float32(float(exact)))
        with np.errstate(over="ignore"):
            want = np.float32(np.float32(t * s) * np.float32(2.0) ** -e) if abs(e) < 126 else None
        if want is not None and np.isfinite(want) and abs(want) > 1e-37:
            assert got == want


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 7, 5), (13, 100, 50), (64, 128, 96), (9, 1024, 200)])
def test_fast_path_is_within_1e_4_of_the_reference_and_near_the_triple_loop(orc, m, k, n):
    rng = np.random.default_rng(m * 1000 + k)
    a = normal(rng, (m, k))
    q, s = int8_weights(rng, n, k)
    values, scales = pack_int8(q, s)
    bias = normal(rng, n)
    c0 = normal(rng, (m, n))
    for act, accumulate, with_bias in [(NONE, False, False), (RELU, False, True), (SILU, True, True)]:
        b = bias if with_bias else None
        fast, ref = c0.copy().reshape(-1), c0.copy().reshape(-1)
        assert orc.matmul_fast(a.reshape(-1), k, m, values, scales, n, k, fast, n, b, act, 0.5, accumulate) == 0
        assert orc.matmul(True, a.reshape(-1), k, m, values, scales, INT8, n, k, ref, n, b, act, 0.5,
                          accumulate) == 0
        err = rel_norm_err(fast.reshape(m, n), ref.reshape(m, n))
        assert err <= 1e-4, (act, err)


def test_fast_sums_are_the_integer_sums(orc):
    # With Act::None, scale 1, no bias: c == dequant(numpy int64 products of the digits).
    rng = np.random.default_rng(3)
    m, k, n = 17, 200, 40
    a = normal(rng, (m, k))
    q, s = int8_weights(rng, n, k)
    values, scales = pack_int8(q, s)
    c = np.zeros(m * n, np.float32)
    orc.matmul_fast(a.reshape(-1), k, m, values, scales, n, k, c, n)
    hi, lo, ex = orc.quantize_rows(a.reshape(-1), k, m, k)
    ah = hi.astype(np.int64) @ q.astype(np.int64).T
    al = lo.astype(np.int64) @ q.astype(np.int64).T
    want = np.array([[orc.dequant(ah[r, o], al[r, o], ex[r], s[o]) for o in range(n)] for r in range(m)],
                    np.float32)
    assert np.array_equal(c.reshape(m, n).view(np.uint32), want.view(np.uint32))


def test_rows_are_independent_of_the_batch(orc):
    # A row's result does not depend on the other rows, so one-row and many-row calls agree.
    rng = np.random.default_rng(4)
    m, k, n = 12, 96, 33
    a = normal(rng, (m, k))
    q, s = int8_weights(rng, n, k)
    values, scales = pack_int8(q, s)
    full = np.zeros(m * n, np.float32)
    orc.matmul_fast(a.reshape(-1), k, m, values, scales, n, k, full, n, None, SILU)
    for r in range(m):
        one = np.zeros(n, np.float32)
        orc.matmul_fast(a[r].copy(), k, 1, values, scales, n, k, one, n, None, SILU)
        assert np.array_equal(one.view(np.uint32), full.reshape(m, n)[r].view(np.uint32))


def test_a_wrong_digit_weight_is_caught(orc):
    # A plausible slip (combining the digits as hi * 128 + lo) breaks the numpy identity above.
    ah, al = 1000, 37
    assert orc.dequant(ah, al, 0, 1.0) == np.float32(ah * 256 + al)
    assert orc.dequant(ah, al, 0, 1.0) != np.float32(ah * 128 + al)


def q8_fast_by_parts(orc, a, m, k, q, d, n):
    """The fast Q8_0 sums from independent parts: numpy int64 block products of the oracle's digits,
    then the f32 fma chain over blocks evaluated in exact rational arithmetic."""
    from exact import fma32

    hi, lo, ex = orc.quantize_rows(a, k, m, k)
    out = np.zeros((m, n), np.float32)
    blocks = k // 32
    for r in range(m):
        for o in range(n):
            f = np.float32(0.0)
            for b in range(blocks):
                sl = slice(32 * b, 32 * b + 32)
                t = int(hi[r, sl].astype(np.int64) @ q[o, sl].astype(np.int64)) * 256 + \
                    int(lo[r, sl].astype(np.int64) @ q[o, sl].astype(np.int64))
                f = fma32(d[o, b], np.float32(t), f)
            out[r, o] = np.float32(math.ldexp(float(f), -int(ex[r])))
    return out


def test_q8_0_fast_path_is_its_block_sums(orc):
    from helpers import pack_q8_0, q8_0_weights

    rng = np.random.default_rng(21)
    for m, k, n in ((1, 32, 3), (3, 96, 17), (4, 160, 9)):
        a = normal(rng, m * k)
        q, d = q8_0_weights(rng, n, k, full_range=True)
        values, scales = pack_q8_0(q, d)
        got = np.zeros(m * n, np.float32)
        assert orc.matmul_fast_q8(a, k, m, values, scales, n, k, got, n) == 0
        want = q8_fast_by_parts(orc, a.reshape(m, k), m, k, q, d, n)
        assert np.array_equal(got.reshape(m, n).view(np.uint32), want.view(np.uint32)), (m, k, n)


def test_q8_0_fast_path_is_within_1e_4_of_the_reference(orc):
    from helpers import pack_q8_0, q8_0_weights

    Q8_0 = 4
    rng = np.random.default_rng(22)
    for m, k, n in ((7, 1024, 64), (2, 2048, 33), (16, 96, 40)):
        a = normal(rng, m * k)
        q, d = q8_0_weights(rng, n, k)
        values, scales = pack_q8_0(q, d)
        fast = np.zeros(m * n, np.float32)
        ref = np.zeros(m * n, np.float32)
        assert orc.matmul_fast_q8(a, k, m, values, scales, n, k, fast, n) == 0
        assert orc.matmul(True, a, k, m, values, scales, Q8_0, n, k, ref, n) == 0
        assert rel_norm_err(fast.reshape(m, n), ref.reshape(m, n)) <= 1e-4


def test_a_misplaced_block_scale_is_caught(orc):
    """Planted in the check, not the product: swapping two blocks' scales of one output changes
    the result, so the block-scale indexing is exercised."""
    from helpers import pack_q8_0, q8_0_weights

    rng = np.random.default_rng(23)
    m, k, n = 2, 128, 5
    a = normal(rng, m * k)
    q, d = q8_0_weights(rng, n, k)
    d[:, 1] = d[:, 0] * np.float32(4.0)
    values, scales = pack_q8_0(q, d)
    good = np.zeros(m * n, np.float32)
    orc.matmul_fast_q8(a, k, m, values, scales, n, k, good, n)
    d2 = d.copy()
    d2[:, [0, 1]] = d2[:, [1, 0]]
    values2, scales2 = pack_q8_0(q, d2)
    bad = np.zeros(m * n, np.float32)
    orc.matmul_fast_q8(a, k, m, values2, scales2, n, k, bad, n)
    assert not np.array_equal(good, bad)
    assert np.array_equal(good.reshape(m, n).view(np.uint32),
                          q8_fast_by_parts(orc, a.reshape(m, k), m, k, q, d, n).view(np.uint32))


def test_guard_flag_threshold_is_exact(orc):
    # e = 0 for a row whose largest value is 32639; each 0.25 has v = 0 and d = 64 (d^2 = 4096), so
    # the row is flagged once 256 * 4096 * count > 32639^2 = 1065304321, that is from 1016 quarters.
    for count, flagged in ((1015, 0), (1016, 1)):
        row = np.full(1 + count, 0.25, np.float32)
        row[0] = 32639.0
        assert orc.row_exponent(row) == 0
        assert orc.guard_flags(row, row.size, 1, row.size)[0] == flagged, count
    # integers below 32640 keep every bit (d = 0): never flagged, however spiky
    row = np.zeros(4096, np.float32)
    row[3] = 32639.0
    row[100:110] = 1.0
    assert orc.guard_flags(row, row.size, 1, row.size)[0] == 0
    # rows with a NaN or an infinity are not flagged
    row = np.full(64, 0.3, np.float32)
    row[1] = np.inf
    assert orc.guard_flags(row, 64, 1, 64)[0] == 0


def test_guard_flags_the_rows_whose_error_could_pass_the_gate(orc):
    """The flag against the fast path's measured error: every unflagged row of spikes up to
    sqrt(k) x is within 6e-4 of the fused reference (the gate is 1e-3); N(0, 1) rows are not
    flagged; the guarded oracle gives flagged rows the fused reference's bits and the others the
    integer oracle's."""
    rng = np.random.default_rng(21)
    for k in (1024, 4096, 16384):
        n, m = 256, 32
        q, s = int8_weights(rng, n, k)
        values, scales = pack_int8(q, s)
        a = rng.standard_normal((m, k)).astype(np.float32)
        spikes = [0, 0, 3, 10, 30, 100, 300, 1000] * 4
        for r, sp in enumerate(spikes):
            if sp:
                a[r, rng.integers(k)] = sp * (r + 1)
        flags = orc.guard_flags(a.reshape(-1), k, m, k).astype(bool)
        assert not flags[0] and not flags[1]
        fast = np.zeros(m * n, np.float32)
        guarded = np.zeros(m * n, np.float32)
        ref = np.zeros(m * n, np.float32)
        orc.matmul_fast(a.reshape(-1), k, m, values, scales, n, k, fast, n)
        orc.matmul_fast(a.reshape(-1), k, m, values, scales, n, k, guarded, n, guard=True)
        orc.matmul(True, a.reshape(-1), k, m, values, scales, 3, n, k, ref, n)
        fast, guarded, ref = fast.reshape(m, n), guarded.reshape(m, n), ref.reshape(m, n)
        err = np.abs(fast - ref).max(axis=1) / np.abs(ref).max(axis=1)
        assert flags.any() and err[~flags].max() <= 6e-4, (k, err[~flags].max())
        assert np.array_equal(guarded[flags].view(np.uint32), ref[flags].view(np.uint32))
        assert np.array_equal(guarded[~flags].view(np.uint32), fast[~flags].view(np.uint32))
