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


INT8_P, Q8_0_P = 3, 4


def tdt_network(rng, h, vocab, durations, layers=2, precision=INT8_P, max_symbols=10, blank_bias=0.0,
                lstm_scale=0.0004):
    """A random TDT prediction network and joint (src/parakeet.rs:1412-1577) in the panel layout:
    int8 (or Q8_0) joint (vocab + durations) x h, LSTM layers 4h x 2h, projection h x h, f32 biases
    and embedding. LSTM scales stay small so its gates are not saturated and its recurrence does not
    amplify small differences from step to step (with scales 5x larger, 1e-6 of noise in the state
    grows to 1e-2 over 25 tokens); blank_bias is added to the blank's (the last token's) joint bias."""
    def mat(n, k, lo, hi):
        if precision == Q8_0_P:  # block scales in the int8 scales' range, f16-exact
            q = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
            d = (lo + (hi - lo) * rng.random((n, k // 32))).astype(np.float16).astype(np.float32)
            return pack_q8_0(q, d)
        q = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
        sc = (lo + (hi - lo) * rng.random(n)).astype(np.float32)
        return pack_int8(q, sc)

    outputs = vocab + len(durations)
    joint_b = (0.5 * rng.standard_normal(outputs)).astype(np.float32)
    joint_b[vocab - 1] += blank_bias
    return {
        "p": precision, "h": h, "vocab": vocab, "durations": list(durations), "max_symbols": max_symbols,
        "joint": mat(outputs, h, 0.001, 0.01), "joint_b": joint_b,
        "emb": (0.5 * rng.standard_normal((vocab, h))).astype(np.float32),
        "lstm": [mat(4 * h, 2 * h, lstm_scale, 2 * lstm_scale) for _ in range(layers)],
        "lstm_b": [(0.1 * rng.standard_normal(4 * h)).astype(np.float32) for _ in range(layers)],
        "proj": mat(h, h, 0.001, 0.003), "proj_b": (0.1 * rng.standard_normal(h)).astype(np.float32),
    }
