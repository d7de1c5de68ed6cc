"""Pins the oracle's restatement of telmo's matrix product (src/kernels/mod.rs, scalar.rs,
avx512.rs) with the closed forms the reference's own tests use: exact input-order sums, an f64
triple loop, narrow weights equal to their widened values, widen equal to decode, and the
exp/sigmoid accuracy bounds."""
import math

import numpy as np
import pytest

from exact import fma32

F32, F16, BF16, INT8, Q8_0 = range(5)
NONE, RELU, SILU = range(3)


def reference_f64(a, m, k, w, n, bias, act, scale, accumulate, c0):
    """src/kernels/mod.rs:808-838: the plain triple loop in f64."""
    s = a.reshape(m, k).astype(np.float64) @ w.reshape(n, k).astype(np.float64).T
    if bias is not None:
        s = s + bias.astype(np.float64)[None, :]
    if act == RELU:
        s = np.maximum(s, 0.0)
    elif act == SILU:
        s = s / (1.0 + np.exp(-s))
    s = s * scale
    if accumulate:
        s = s + c0.reshape(m, n).astype(np.float64)
    return s.astype(np.float32)


@pytest.mark.parametrize("fused", [True, False])
def test_tiles_sum_their_products_in_input_order(orc, fused):
    # src/kernels/mod.rs:885-931 (k, lda, k_stride) cases; fused sums checked with exact fmaf,
    # unfused with numpy's IEEE f32 product then sum.
    for k, lda, ks in [(1, 1, 16), (7, 9, 16), (256, 300, 40)]:
        for rows in ([1, 2, 5, 8] if k < 256 else [1, 8]):
            a = orc.random(rows * lda, 40)
            b = orc.random(k * ks + 16, 41)
            start = orc.random(rows * 16, 42)
            for load in (False, True):
                out = start.copy()
                orc.tile(fused, k, a, lda, rows, b, ks, out, load)
                cols = range(16) if k < 256 else [0, 7, 15]
                for r in range(rows if k < 256 else 1):
                    for j in cols:
                        s = np.float32(start[r * 16 + j]) if load else np.float32(0.0)
                        for i in range(k):
                            x, y = a[r * lda + i], b[i * ks + j]
                            s = fma32(x, y, s) if fused else np.float32(s + np.float32(x * y))
                        assert out[r * 16 + j].view(np.uint32) == s.view(np.uint32), (k, rows, load, r, j)


def test_a_dropped_fma_is_caught():
    # The exact-FMA check above distinguishes fused from unfused sums on this data.
    a, b, c = np.float32(1 + 2.0**-12), np.float32(1 + 2.0**-12), np.float32(-(1 + 2.0**-11))
    assert fma32(a, b, c) != np.float32(np.float32(a * b) + c)


def test_the_epilogue_agrees_across_instruction_sets_and_stays_in_its_columns(orc):
    # src/kernels/mod.rs:933-960
    acc = orc.random(16, 50) * np.float32(8.0)
    bias = orc.random(16, 51)
    c0 = orc.random(20, 52)
    for cols in range(1, 17):
        for act in (NONE, RELU, SILU):
            for with_bias, accumulate in [(False, False), (True, False), (True, True)]:
                b = bias if with_bias else None
                want, got = c0.copy(), c0.copy()
                orc.store(False, acc, want, cols, b, act, 0.5, accumulate)
                orc.store(True, acc, got, cols, b, act, 0.5, accumulate)
                assert np.array_equal(got[cols:], c0[cols:])
                assert np.all(np.abs(got - want) <= 1e-6 + 1e-6 * np.abs(want))


SHAPES = [(1, 1, 1), (1, 7, 5), (5, 13, 17), (6, 64, 16), (7, 33, 31), (13, 100, 50), (64, 128, 96)]
EPIS = [(NONE, False, False), (RELU, False, True), (SILU, True, True), (NONE, True, False)]


@pytest.mark.parametrize("fused", [True, False])
def test_matmul_matches_the_reference_for_every_shape_and_epilogue(orc, fused):
    # src/kernels/mod.rs:962-1005 with f32 weights from rows.
    for m, k, n in SHAPES:
        a = orc.random(m * k, 1)
        w = orc.random(n * k, 2)
        bias = orc.random(n, 3)
        c0 = orc.random(m * n, 4)
        values, scales = orc.encode(w, n, k, F32)
        for act, accumulate, with_bias in EPIS:
            b = bias if with_bias else None
            want = reference_f64(a, m, k, w, n, b, act, 0.5, accumulate, c0)
            got = c0.copy()
            assert orc.matmul(fused, a, k, m, values, None, F32, n, k, got, n, b, act, 0.5, accumulate) == 0
            tol = 1e-5 * math.sqrt(k) * (1.0 + np.abs(want.reshape(-1)))
            assert np.all(np.abs(got - want.reshape(-1)) <= tol), (m, k, n, act)


def test_a_transposed_weight_fails_the_triple_loop(orc):
    # Guards the check above: reading w as [k, n] instead of [n, k] is caught.
    m, k, n = 5, 13, 17
    a, w = orc.random(m * k, 1), orc.random(n * k, 2)
    values, _ = orc.encode(w, n, k, F32)
    got = np.zeros(m * n, np.float32)
    orc.matmul(True, a, k, m, values, None, F32, n, k, got, n)
    wrong = reference_f64(a, m, k, w.reshape(n, k).T.copy().reshape(-1)[: n * k].reshape(n, k).reshape(-1), n,
                          None, NONE, 1.0, False, None)
    assert not np.allclose(got, wrong.reshape(-1), atol=1e-3)


def test_matmul_rejects_what_the_reference_asserts(orc):
    # src/kernels/mod.rs:669-677: early return for m = 0 or n = 0, then lda, ldc and lengths.
    a = orc.random(12, 1)
    values, _ = orc.encode(orc.random(16, 2), 4, 4, F32)
    c = np.zeros(12, np.float32)
    assert orc.matmul(True, a, 4, 0, values, None, F32, 4, 4, c, 4) == 0
    assert orc.matmul(True, a, 3, 3, values, None, F32, 4, 4, c, 4) == -2  # lda < k
    assert orc.matmul(True, a, 4, 3, values, None, F32, 4, 4, c, 3) == -2  # ldc < n
    assert orc.matmul(True, a, 4, 4, values, None, F32, 4, 4, c, 4) == -2  # a too short
    assert orc.matmul(True, a, 4, 3, values, None, F32, 4, 4, c, 4, bias=np.zeros(3, np.float32)) == -2


def test_k_zero_stores_the_epilogue_of_zero(orc):
    # src/kernels/mod.rs:669-671 returns only for m = 0 or n = 0, so k = 0 stores epi(0).
    m, n = 3, 5
    bias = orc.random(n, 3)
    c = np.full(m * n, 7.0, np.float32)
    values = np.zeros(0, np.uint8)
    assert orc.matmul(True, np.zeros(1, np.float32), 0, m, values, None, F32, n, 0, c, n, bias, RELU, 2.0) == 0
    assert np.array_equal(c.reshape(m, n), np.tile(np.maximum(bias, 0) * 2, (m, 1)))


@pytest.mark.parametrize("fused", [True, False])
def test_narrow_weights_give_the_sums_of_their_widened_values(orc, fused):
    # src/kernels/mod.rs:1071-1128
    for m, k, n in [(1, 64, 20), (7, 288, 33), (13, 544, 16), (6, 32, 5), (3, 544, 40)]:
        a = orc.random(m * k, 21)
        i = np.arange(n * k)
        w = (orc.random(n * k, 22) * (1 + i // k).astype(np.float32) * np.float32(0.1)).astype(np.float32)
        bias = orc.random(n, 23)
        for p in (F16, BF16, INT8, Q8_0):
            values, scales = orc.encode(w, n, k, p)
            wide_v, _ = orc.encode(orc.decode(values, scales, n, k, p), n, k, F32)
            c1, c2 = np.zeros(m * n, np.float32), np.zeros(m * n, np.float32)
            orc.matmul(fused, a, k, m, values, scales, p, n, k, c1, n, bias, SILU, 0.5)
            orc.matmul(fused, a, k, m, wide_v, None, F32, n, k, c2, n, bias, SILU, 0.5)
            assert np.array_equal(c1.view(np.uint32), c2.view(np.uint32)), (p, m, k, n)
            want = reference_f64(a, m, k, w, n, bias, SILU, 0.5, False, None).reshape(-1)
            unit = {F16: 1e-3, BF16: 8e-3}.get(p, 1e-2)
            wmax = np.abs(w.reshape(n, k)).max(axis=1)
            tol = unit * math.sqrt(k) * np.tile(wmax, m)
            assert np.all(np.abs(c1 - want) <= tol), p


def _assert_widens_exactly(orc, p, k, values, scales):
    want = orc.decode(values, scales, 16, k, p)
    got = orc.widen(p, k, values, scales)
    assert np.array_equal(got.T.view(np.uint32), want.view(np.uint32)), p


def test_widening_gives_the_decoded_values_bit_for_bit(orc):
    # src/kernels/mod.rs:1130-1183
    halves = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.uint8)
    ints = np.concatenate([np.arange(256, dtype=np.uint8),
                           (orc.random(256 * 15, 30) * np.float32(128.0)).astype(np.int8).view(np.uint8)])
    r = orc.random(8 * 16, 31)
    scales = np.array([(int(v.view(np.uint32)) & 0x807FFFFF) | (((i * 37) % 255) << 23)
                       for i, v in enumerate(r)], np.uint32).view(np.float32)
    for p in (F16, BF16):
        _assert_widens_exactly(orc, p, len(halves) // 32, halves, np.zeros(0, np.float32))
    _assert_widens_exactly(orc, INT8, 256, ints, scales[:16])
    _assert_widens_exactly(orc, Q8_0, 256, ints, scales)
    # Every int8 value times one scale is the single rounded product.
    q = np.arange(256, dtype=np.uint8).view(np.int8)
    s = np.float32(0.0071)
    got = orc.widen(INT8, 16, q.view(np.uint8), np.full(16, s, np.float32))
    assert np.array_equal(got.reshape(-1), (q.astype(np.float32) * s).astype(np.float32))


def test_exp_is_within_two_ulp_and_sigmoid_within_5e_7(orc):
    # src/kernels/avx512.rs:279-281 states about 2 ulp; src/kernels/mod.rs:1261-1277 bounds
    # the sigmoid by 1e-9 + 5e-7 * value.
    for x in np.linspace(-87.0, 88.0, 4001, dtype=np.float32):
        got = float(orc.exp_simd(x))
        want = math.exp(float(x))
        assert abs(got - want) <= 2.5 * np.spacing(np.float32(want)), x
    for i in range(-1000, 1001):
        x = np.float32(i) * np.float32(0.0875)
        want = 1.0 / (1.0 + math.exp(-float(x)))
        sig = np.float32(1.0) / (np.float32(1.0) + orc.exp_simd(np.float32(0.0) - x))
        assert abs(float(sig) - want) <= 1e-9 + 5e-7 * want, x
    # SiLU is x * sigmoid(x) as x / (1 + e^-x).
    for x in [-20.0, -1.0, 0.0, 0.5, 3.0, 30.0]:
        assert abs(float(orc.silu_simd(x)) - x / (1 + math.exp(-x))) <= 1e-6 * (1 + abs(x))
