"""The oracle's depthwise convolution (src/kernels/scalar.rs:164-187) and the conv module's loop
around it (src/parakeet.rs:1107-1122, src/granite.rs:900-915).

Pinned by:
- the reference's own test (src/kernels/mod.rs:1279-1300): every frame of an 11 x 24 input,
  kernel 9, against an f64 direct sum within 1e-5;
- exact integer correlations: small integer inputs and weights keep every product and sum exact
  in f32, so each output equals numpy's correlate of the zero-padded channel (a flipped kernel, a
  wrong centre or a wrong padding fails);
- numpy's float32 arithmetic (one rounding per operation) on random values, which pins the
  rounded product then rounded sum in tap order (a fused multiply-add or a reordered sum differs);
- the strided, offset rows against the stride-1 rows, and SiLU against the SIMD sigmoid.
"""
import numpy as np
import pytest


def f64_direct(x, w, bias, t):
    frames, channels = x.shape
    kernel = w.shape[0]
    s = bias.astype(np.float64).copy()
    for j in range(kernel):
        src = t + j - kernel // 2
        if 0 <= src < frames:
            s += w[j].astype(np.float64) * x[src].astype(np.float64)
    return s


def test_the_reference_case_matches_a_direct_sum(orc):
    frames, channels, kernel = 11, 24, 9
    x = orc.random(frames * channels, 12).reshape(frames, channels)
    w = orc.random(kernel * channels, 13).reshape(kernel, channels)
    bias = orc.random(channels, 14)
    for t in range(frames):
        got = orc.dwconv1d_frame(x, t, w, bias)
        assert np.max(np.abs(got.astype(np.float64) - f64_direct(x, w, bias, t))) < 1e-5, t


@pytest.mark.parametrize("frames,channels,kernel", [(1, 3, 9), (5, 7, 9), (40, 16, 31), (12, 5, 4), (9, 2, 1)])
def test_integer_inputs_equal_numpy_correlate(orc, frames, channels, kernel):
    rng = np.random.default_rng(frames * 100 + kernel)
    x = rng.integers(-8, 9, size=(frames, channels)).astype(np.float32)
    w = rng.integers(-8, 9, size=(kernel, channels)).astype(np.float32)
    bias = rng.integers(-50, 51, size=channels).astype(np.float32)
    got = orc.dwconv1d(x, w, bias)
    half = kernel // 2
    for c in range(channels):
        # full[i] = sum_j x[i + j - (kernel - 1)] * w[j]; frame t sits at i = t + kernel - 1 - half
        full = np.correlate(x[:, c].astype(np.int64), w[:, c].astype(np.int64), "full")
        want = full[kernel - 1 - half:kernel - 1 - half + frames] + bias[c].astype(np.int64)
        assert np.array_equal(got[:, c].astype(np.int64), want), c


def test_rounding_is_a_product_then_a_sum_in_tap_order(orc):
    rng = np.random.default_rng(5)
    frames, channels, kernel = 30, 64, 9
    x = rng.standard_normal((frames, channels)).astype(np.float32)
    w = rng.standard_normal((kernel, channels)).astype(np.float32)
    bias = rng.standard_normal(channels).astype(np.float32)
    got = orc.dwconv1d(x, w, bias)
    want = np.empty_like(got)
    fused = np.empty_like(got)
    for t in range(frames):
        acc = bias.copy()
        acc_f = bias.copy()
        for j in range(kernel):
            src = t + j - kernel // 2
            if 0 <= src < frames:
                acc = acc + w[j] * x[src]  # float32: the product rounds, then the sum
                acc_f = (acc_f.astype(np.float64) + w[j].astype(np.float64) * x[src]).astype(np.float32)
        want[t] = acc
        fused[t] = acc_f
    assert np.array_equal(got, want)
    assert not np.array_equal(got, fused)  # the data tell a fused multiply-add apart


def test_strided_rows_pick_frames_of_the_stride_one_output(orc):
    rng = np.random.default_rng(9)
    frames, channels, kernel = 23, 10, 7
    x = rng.standard_normal((frames, channels)).astype(np.float32)
    w = rng.standard_normal((kernel, channels)).astype(np.float32)
    bias = rng.standard_normal(channels).astype(np.float32)
    full = orc.dwconv1d(x, w, bias, rows=frames + 6)
    for t0, stride, rows in ((0, 2, 12), (3, 2, 8), (1, 3, 9), (5, 1, 20)):
        got = orc.dwconv1d(x, w, bias, rows=rows, t0=t0, stride=stride)
        assert np.array_equal(got, full[t0:t0 + stride * rows:stride]), (t0, stride)
    # frames beyond the input see only the padding: bias, then the taps that still reach back
    past = orc.dwconv1d(x, w, bias, rows=1, t0=frames + kernel // 2)
    assert np.array_equal(past[0], bias)


def test_silu_follows_the_sums(orc):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((17, 33)).astype(np.float32)
    w = rng.standard_normal((9, 33)).astype(np.float32)
    bias = rng.standard_normal(33).astype(np.float32)
    plain = orc.dwconv1d(x, w, bias)
    act = orc.dwconv1d(x, w, bias, silu=True)
    want = np.vectorize(orc.silu_simd, otypes=[np.float32])(plain)
    assert np.array_equal(act, want)
    sig = plain.astype(np.float64) / (1.0 + np.exp(-plain.astype(np.float64)))
    assert np.max(np.abs(act - sig) / (1.0 + np.abs(sig))) < 1e-6


def test_empty_kernel_and_empty_input_give_the_bias(orc):
    bias = np.arange(6, dtype=np.float32)
    x = np.ones((4, 6), np.float32)
    assert np.array_equal(orc.dwconv1d(x, np.zeros((0, 6), np.float32), bias), np.tile(bias, (4, 1)))
    assert np.array_equal(orc.dwconv1d(np.zeros((0, 6), np.float32), np.ones((3, 6), np.float32), bias, rows=2),
                          np.tile(bias, (2, 1)))
