"""The CPU baseline (a C++ port of telmo's SIMD + thread-pool path) agrees bit for bit with the
fused oracle before it is timed, and its pool keeps the reference's contract
(src/threads.rs:217-265, src/kernels/mod.rs:1039-1069)."""
import ctypes

import numpy as np
import pytest

from helpers import tdt_network

F32, F16, BF16, INT8, Q8_0 = range(5)
NONE, RELU, SILU = range(3)


@pytest.fixture(scope="module")
def cb(orc):
    L = ctypes.CDLL(orc.CPUBASE)
    L.cb_pool_new.restype = ctypes.c_void_p
    L.cb_pool_new.argtypes = [ctypes.c_size_t]
    L.cb_pool_free.argtypes = [ctypes.c_void_p]
    L.cb_pool_test.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_long]
    L.cb_matmul.argtypes = ([ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t,
                             ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t,
                             ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_void_p,
                             ctypes.c_size_t, ctypes.c_int, ctypes.c_float, ctypes.c_int])
    return L


def cb_matmul(L, pool, isa, a, lda, m, values, scales, p, n, k, c, ldc, bias, act, scale, acc):
    ptr = lambda x: None if x is None else x.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    return L.cb_matmul(pool, isa, ptr(a), a.size, lda, m, ptr(values), ptr(scales), p, n, k, ptr(c), c.size, ldc,
                       ptr(bias), 0 if bias is None else bias.size, act, scale, int(acc))


def isas(L):
    best = L.cb_isa()
    return [i for i in (2, 1) if i <= best]


def test_every_task_runs_once_and_failures_come_back(cb):
    for threads in (1, 2, 3, 8):
        pool = cb.cb_pool_new(threads)
        for tasks in (0, 1, 7, 100):
            counts = np.zeros(max(tasks, 1), np.uint32)
            assert cb.cb_pool_test(pool, tasks, counts.ctypes.data, -1) == 0
            assert np.all(counts[:tasks] == 1)
        counts = np.zeros(2000, np.uint32)
        for _ in range(20):
            assert cb.cb_pool_test(pool, 100, counts.ctypes.data, -1) == 0
        assert np.all(counts[:100] == 20)
        counts = np.zeros(10, np.uint32)
        assert cb.cb_pool_test(pool, 10, counts.ctypes.data, 3) == -1
        assert np.all(counts == 1)  # every other task still ran
        assert cb.cb_pool_test(pool, 10, counts.ctypes.data, -1) == 0  # the pool still works
        cb.cb_pool_free(pool)


@pytest.mark.parametrize("p", [F32, F16, BF16, INT8, Q8_0])
def test_the_simd_port_is_bit_identical_to_the_fused_oracle(orc, cb, p):
    if not isas(cb):
        pytest.skip("no AVX2/AVX-512 on this host")
    pool = cb.cb_pool_new(3)
    for m, k, n in [(1, 64, 20), (7, 288, 33), (13, 544, 16), (6, 32, 5), (3, 544, 40), (8, 64, 50), (9, 96, 40),
                    (64, 128, 96)]:
        if p == Q8_0 and k % 32:
            continue
        a = orc.random(m * k, 21)
        w = orc.random(n * k, 22)
        bias, c0 = orc.random(n, 23), orc.random(m * n, 24)
        values, scales = orc.encode(w, n, k, p)
        sc = scales if len(scales) else None
        for act, acc, with_bias in [(NONE, False, False), (RELU, False, True), (SILU, True, True)]:
            b = bias if with_bias else None
            want = c0.copy()
            orc.matmul(True, a, k, m, values, sc, p, n, k, want, n, b, act, 0.5, acc)
            for isa in isas(cb):
                got = c0.copy()
                assert cb_matmul(cb, pool, isa, a, k, m, values, sc, p, n, k, got, n, b, act, 0.5, acc) == 0
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (isa, p, m, k, n, act)
    cb.cb_pool_free(pool)


def test_results_are_bit_identical_across_thread_counts(orc, cb):
    if not isas(cb):
        pytest.skip("no AVX2/AVX-512 on this host")
    m, k, n = 50, 300, 200
    a = orc.random(m * k, 7)
    values, _ = orc.encode(orc.random(n * k, 8), n, k, F32)
    for isa in isas(cb):
        first = None
        for threads in (1, 2, 3, 6, 8):
            pool = cb.cb_pool_new(threads)
            c = np.zeros(m * n, np.float32)
            assert cb_matmul(cb, pool, isa, a, k, m, values, None, F32, n, k, c, n, None, SILU, 1.0, False) == 0
            cb.cb_pool_free(pool)
            if first is None:
                first = c
            assert np.array_equal(first.view(np.uint32), c.view(np.uint32)), (isa, threads)


def test_the_port_refuses_what_the_reference_asserts(orc, cb):
    pool = cb.cb_pool_new(2)
    a = orc.random(12, 1)
    values, _ = orc.encode(orc.random(16, 2), 4, 4, F32)
    c = np.zeros(12, np.float32)
    assert cb_matmul(cb, pool, 0, a, 3, 3, values, None, F32, 4, 4, c, 4, None, NONE, 1.0, False) == -2
    assert cb_matmul(cb, pool, 0, a, 4, 0, values, None, F32, 4, 4, c, 4, None, NONE, 1.0, False) == 0
    cb.cb_pool_free(pool)


def _tdt_cases():
    """Zero-joint networks (logits exactly the joint bias) whose token lists the oracle's tests pin
    by hand, and one start part-way through a frame."""
    from test_oracle_tdt import joint_bias, zero_joint

    base = tdt_network(np.random.default_rng(7), 32, 20, [0, 1, 2, 3, 4], layers=2, max_symbols=3)
    nan = joint_bias(20, 5, 9, 1)
    nan[0] = np.nan
    tie = joint_bias(20, 5, 9, 2)
    tie[6], tie[24] = tie[9], tie[22]
    return [(zero_joint(base, joint_bias(20, 5, 19, 3)), 23, 0, 0),
            (zero_joint(base, joint_bias(20, 5, 7, 0)), 6, 0, 0),
            (zero_joint(base, joint_bias(20, 5, 11, 2)), 9, 0, 0),
            (zero_joint(base, joint_bias(20, 5, 4, 0)), 3, 1, 2),
            (zero_joint(base, tie), 4, 0, 0),
            (zero_joint(base, nan), 2, 0, 0),
            (base, 5, 5, 1)]


def _decode_both(orc, net, frames, frame, on_frame, pool):
    enc = np.random.default_rng(frames).standard_normal((frames, net["h"])).astype(np.float32)
    width = len(net["lstm"]) * 2 * net["h"]
    s1, p1 = np.zeros(width, np.float32), np.zeros(net["h"], np.float32)
    s2, p2 = s1.copy(), p1.copy()
    want = orc.tdt_decode(net, enc, s1, p1, frame, on_frame)
    got = orc.cpu_tdt_decode(net, enc, s2, p2, pool, frame, on_frame)
    return want, got, (s1, p1), (s2, p2)


def test_the_tdt_decode_port_keeps_decode_inners_control_flow(orc, cb):
    if not isas(cb):
        pytest.skip("no AVX2/AVX-512 on this host")
    pool = cb.cb_pool_new(3)
    for net, frames, frame, on_frame in _tdt_cases():
        want, got, _, _ = _decode_both(orc, net, frames, frame, on_frame, pool)
        assert got == want
    cb.cb_pool_free(pool)


@pytest.mark.parametrize("precision", ["int8", "q8_0"])
def test_the_tdt_decode_port_agrees_with_the_oracle_on_random_networks(orc, cb, precision):
    """Fused f32 sums (the port) against the fast path's integer sums (the oracle): the same tokens,
    states and predictions within the fast path's error."""
    if not isas(cb):
        pytest.skip("no AVX2/AVX-512 on this host")
    pool = cb.cb_pool_new(4)
    rng = np.random.default_rng(11)
    net = tdt_network(rng, 64, 100, [0, 1, 2, 3, 4], precision=INT8 if precision == "int8" else Q8_0,
                      blank_bias=3.0)
    want, got, (s1, p1), (s2, p2) = _decode_both(orc, net, 60, 0, 0, pool)
    assert len(want[0]) > 5 and got == want
    assert np.max(np.abs(s1 - s2)) < 1e-3 and np.max(np.abs(p1 - p2)) < 1e-3
    cb.cb_pool_free(pool)
