"""The oracle's row kernels of the Conformer glue: LayerNorm (AVX-512 order) and GLU.

The reference pins its SIMD row kernels only against its scalar ones. Here the oracle's LayerNorm
is checked against the scalar formula in f64 (src/kernels/scalar.rs:126-134), against a closed
form (an alternating row gives exactly +-1/sqrt(1 + eps)), and on constant rows (exactly beta).
The exact bits of the sixteen-partial summation order stay unpinned: only the reference's code
could fix them.
"""
import numpy as np


def scalar_layer_norm(x, gamma, beta, eps):
    x64 = x.astype(np.float64)
    mean = x64.sum() / x.size
    var = ((x64 - mean) ** 2).sum() / x.size
    rstd = 1.0 / np.sqrt(var + eps)
    return (((x64 - mean) * rstd).astype(np.float32) * gamma + beta).astype(np.float32)


def test_layer_norm_matches_the_scalar_formula(orc):
    rng = np.random.default_rng(3)
    for n in (1, 5, 16, 17, 100, 1024, 1000):
        for loc, spread in ((0.0, 1.0), (3.0, 0.01), (-50.0, 20.0)):
            x = (loc + spread * rng.standard_normal(n)).astype(np.float32)
            gamma = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
            beta = (0.1 * rng.standard_normal(n)).astype(np.float32)
            got = orc.layer_norm(x, gamma, beta, 1e-5)
            want = scalar_layer_norm(x, gamma, beta, 1e-5)
            tol = 2e-5 * (1.0 + np.abs(loc) / spread) if n > 1 else 1e-6
            assert np.max(np.abs(got - want)) <= tol, (n, loc, spread, np.max(np.abs(got - want)))


def test_layer_norm_closed_form(orc):
    for n in (32, 64, 1024):
        for eps in (1e-5, 0.25, 3.0):
            x = np.where(np.arange(n) % 2 == 0, np.float32(1.0), np.float32(3.0)).astype(np.float32)
            got = orc.layer_norm(x, np.ones(n, np.float32), np.zeros(n, np.float32), eps)
            r = np.float32(1.0) / np.sqrt(np.float32(1.0) + np.float32(eps), dtype=np.float32)
            want = np.where(np.arange(n) % 2 == 0, -r, r).astype(np.float32)
            assert np.array_equal(got, want), (n, eps)


def test_layer_norm_of_a_constant_row_is_beta(orc):
    rng = np.random.default_rng(4)
    for c in (0.0, 1.5, -7.25, 1024.0):
        n = 48
        beta = rng.standard_normal(n).astype(np.float32)
        got = orc.layer_norm(np.full(n, c, np.float32), rng.standard_normal(n).astype(np.float32), beta, 1e-5)
        assert np.array_equal(got, beta)


def test_a_dropped_eps_is_caught(orc):
    # the closed-form row with a large eps tells eps apart from none
    n, eps = 64, 3.0
    x = np.where(np.arange(n) % 2 == 0, np.float32(1.0), np.float32(3.0)).astype(np.float32)
    got = orc.layer_norm(x, np.ones(n, np.float32), np.zeros(n, np.float32), eps)
    assert abs(abs(float(got[0])) - 0.5) < 1e-6  # 1 / sqrt(1 + 3)


def test_glu_is_a_times_sigmoid_b(orc):
    rng = np.random.default_rng(5)
    a = (4 * rng.standard_normal(4000)).astype(np.float32)
    b = (6 * rng.standard_normal(4000)).astype(np.float32)
    got = orc.glu(a, b).astype(np.float64)
    want = a.astype(np.float64) / (1.0 + np.exp(-b.astype(np.float64)))
    assert np.all(np.abs(got - want) <= 1e-6 * (1.0 + np.abs(want)))


def scalar_softmax(x):
    """The reference's scalar softmax (src/kernels/scalar.rs:136-147): f32 exp of x - max, an f64
    sum, inv = f32(1 / sum), x * inv."""
    x = x.astype(np.float32)
    e = np.exp((x - x.max()).astype(np.float32)).astype(np.float32)
    inv = np.float32(1.0 / e.astype(np.float64).sum())
    return (e * inv).astype(np.float32)


def test_softmax_matches_the_scalar_kernel_as_the_reference_tests_it(orc):
    # src/kernels/mod.rs:1186-1215: random(n, 9) * 30 for these n, within 1e-6 + 1e-5 |p| of the
    # scalar kernel and summing to 1 within 1e-5.
    for n in (1, 3, 4, 8, 15, 17, 1030, 16384):
        x = (orc.random(n, 9) * np.float32(30.0)).astype(np.float32)
        got = orc.softmax(x)
        want = scalar_softmax(x)
        assert abs(float(got.astype(np.float32).sum(dtype=np.float32)) - 1.0) < 1e-5, n
        assert np.all(np.abs(got - want) <= 1e-6 + 1e-5 * np.abs(want)), n


def test_softmax_of_a_constant_row_is_one_over_n(orc):
    # every e is exp(0) = 1 exactly, every partial sum and the total are exact integers
    for n in (1, 16, 48, 1000, 16384):
        for c in (0.0, -3.5, 1e4):
            got = orc.softmax(np.full(n, c, np.float32))
            assert np.all(got == np.float32(1.0) / np.float32(n)), (n, c)


def test_softmax_keeps_the_exp_clamp(orc):
    # x - max below -87.33654 is clamped, so far-off entries get exp(-87.33654), not 0, and the
    # sum stays exactly 1
    for n in (2, 17, 64):
        x = np.full(n, -1000.0, np.float32)
        x[n // 2] = 0.0
        got = orc.softmax(x)
        tiny = np.float32(orc.exp_simd(np.float32(-87.33654)))
        assert tiny > 0
        assert got[n // 2] == np.float32(1.0)
        assert np.all(np.delete(got, n // 2) == tiny), n


def test_softmax_sums_in_sixteen_partials(orc):
    # one large e in partial 0 and small ones spread over the other partials: a single running sum
    # loses the small ones, sixteen partials keep them, so the two orders give different outputs
    n = 16 * 64
    x = np.full(n, -17.0, np.float32)  # e = exp(-17) ~ 4e-8, under half an ulp of 1
    x[0] = 0.0
    got = orc.softmax(x)
    e = np.array([orc.exp_simd(np.float32(v)) for v in (x - x.max())], np.float32)
    running = np.float32(0.0)
    for v in e:
        running = np.float32(running + v)
    assert got[0] != np.float32(np.float32(1.0) / running) * e[0]
    assert np.float32(1.0) / running == np.float32(1.0)  # the running sum lost every small term
    assert got[0] < np.float32(1.0)
