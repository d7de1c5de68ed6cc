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
