"""Input builders shared by the tests (seeded; the shapes and distributions of the benchmark
configurations: N(0,1) activations, int8 weights uniform in [-127, 127], scales U(0.001, 0.01))."""
import numpy as np


def normal(rng, shape):
    return rng.standard_normal(shape).astype(np.float32)


def int8_weights(rng, n, k):
    q = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
    s = (0.001 + 0.009 * rng.random(n)).astype(np.float32)
    return q, s


def pack_int8(q, s):
    """Panel layout of int8 rows q [n, k] with scales s [n] (src/quant.rs:200-269)."""
    n, k = q.shape
    panels = -(-n // 16)
    pad = np.zeros((panels * 16, k), np.int8)
    pad[:n] = q
    values = pad.reshape(panels, 16, k).transpose(0, 2, 1).reshape(-1).view(np.uint8).copy()
    scales = np.zeros(panels * 16, np.float32)
    scales[:n] = s
    return values, scales


def rel_norm_err(got, want):
    """Row-normwise infinity error: max_ij |got - want| / max_j |want_i|."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    den = np.maximum(np.abs(want).max(axis=1, keepdims=True), 1e-30)
    return float((np.abs(got - want) / den).max())


def q8_0_weights(rng, n, k, full_range=False):
    """Q8_0 weights: int8 q [n, k] and f16-exact block scales d [n, k / 32] (GGUF's Q8_0)."""
    lo = -128 if full_range else -127
    q = rng.integers(lo, 128, size=(n, k)).astype(np.int8)
    d = (0.001 + 0.009 * rng.random((n, k // 32))).astype(np.float16).astype(np.float32)
    return q, d


def pack_q8_0(q, d):
    """Panel layout of Q8_0 rows: values as int8, scales [(p * blocks + b) * 16 + j] (src/quant.rs:8-13)."""
    n, k = q.shape
    values, _ = pack_int8(q, np.ones(n, np.float32))
    panels, blocks = -(-n // 16), k // 32
    scales = np.zeros((panels, blocks, 16), np.float32)
    for o in range(n):
        scales[o // 16, :, o % 16] = d[o]
    return values, scales.reshape(-1)
