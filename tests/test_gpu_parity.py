"""Parity of the HIP path with the oracle, through the C ABI, on an MI355X.

* Exact mode: bit-identical to the reference's fused arithmetic (src/kernels/avx512.rs tile and
  store, mod.rs gemm_panels) for every precision, shape and epilogue.
* Fast mode, int8 weights: bit-identical to the integer oracle (two int8 digits, exact i32 sums,
  one dequantisation), and within 1e-4 row-normwise of the reference's fused f32 sums (gate 1e-3).
* The GEMVs (m <= 16) and the GEMM give the same bits for the same row.
* The committed golden fixtures (tests/golden) hold in both modes.
"""
import numpy as np
import pytest

from helpers import int8_weights, normal, pack_int8, rel_norm_err

pytestmark = pytest.mark.gpu

F32, F16, BF16, INT8, Q8_0 = range(5)
NONE, RELU, SILU = range(3)
EPIS = [(NONE, False, False), (RELU, False, True), (SILU, True, True), (NONE, True, False)]


def say(*args):
    print("[case]", *args, flush=True)


def epi_of(telmo_amd, bias, act, accumulate, scale=0.5):
    return telmo_amd.Epilogue(bias=bias, act=telmo_amd.Act(act), scale=scale, accumulate=accumulate)


def run_gpu(tk, a, lda, m, values, scales, p, n, k, c0, ldc, bias, act, acc, scale=0.5):
    import telmo_amd

    w = telmo_amd.PackedWeights.from_parts(tk, n, k, telmo_amd.Precision(p), values,
                                           scales if scales is not None and len(scales) else None)
    c = c0.copy()
    tk.matmul(a, lda, m, w, c, ldc, epi_of(telmo_amd, bias, act, acc, scale))
    w.close()
    return c


EXACT_SHAPES = [(1, 1, 1), (1, 7, 5), (5, 13, 17), (6, 64, 16), (7, 33, 31), (13, 100, 50), (64, 128, 96),
                (3, 544, 40), (9, 64, 8198)]


@pytest.mark.parametrize("p", [F32, F16, BF16, INT8, Q8_0])
def test_exact_mode_is_bit_identical_to_the_fused_reference(tk, orc, p):
    tk.set_mode(tk.EXACT)
    try:
        for m, k, n in EXACT_SHAPES:
            if p == Q8_0 and k % 32:
                continue
            say("exact", p, m, k, n)
            a = orc.random(m * k, 1)
            w = orc.random(n * k, 2)
            bias, c0 = orc.random(n, 3), orc.random(m * n, 4)
            values, scales = orc.encode(w, n, k, p)
            for act, acc, with_bias in EPIS:
                b = bias if with_bias else None
                want = c0.copy()
                assert orc.matmul(True, a, k, m, values, scales, p, n, k, want, n, b, act, 0.5, acc) == 0
                got = run_gpu(tk, a, k, m, values, scales, p, n, k, c0, n, b, act, acc)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (p, m, k, n, act)
    finally:
        tk.set_mode(tk.FAST)


# (700, 2048, 1000) and (1300, 2048, 700) take the k-split kernel with 48- and 64-row tiles;
# (100, 1000, 4100) the direct kernel on a wide product with fewer 64 x 64 tiles than CUs.
FAST_SHAPES = [(1, 1, 1), (3, 7, 5), (8, 64, 16), (9, 64, 16), (13, 100, 50), (64, 128, 96), (130, 1000, 255),
               (200, 640, 8198), (257, 2048, 130), (1, 4096, 1024), (8, 1280, 2560), (16, 2048, 100),
               (4, 2112, 300), (16, 2049, 77), (2, 64, 140000), (11, 700, 20000), (700, 2048, 1000),
               (1300, 2048, 700), (100, 1000, 4100)]


@pytest.mark.parametrize("m,k,n", FAST_SHAPES)
def test_fast_int8_is_bit_identical_to_its_integer_oracle(tk, orc, m, k, n):
    rng = np.random.default_rng(m * 7919 + k * 31 + n)
    a = normal(rng, m * k)
    q, s = int8_weights(rng, n, k)
    values, scales = pack_int8(q, s)
    bias, c0 = normal(rng, n), normal(rng, m * n)
    for act, acc, with_bias in EPIS:
        say("fast", m, k, n, act, acc, with_bias)
        b = bias if with_bias else None
        want = c0.copy()
        assert orc.matmul_fast(a, k, m, values, scales, n, k, want, n, b, act, 0.5, acc) == 0
        got = run_gpu(tk, a, k, m, values, scales, INT8, n, k, c0, n, b, act, acc)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, k, n, act)
        ref = c0.copy()
        orc.matmul(True, a, k, m, values, scales, INT8, n, k, ref, n, b, act, 0.5, acc)
        err = rel_norm_err(got.reshape(m, n), ref.reshape(m, n))
        print(f"[err] m={m} k={k} n={n} act={act}: {err:.2e}")
        assert err <= 1e-3


def _random_dispatch_shapes():
    """Four seeded random shapes in each region of the int8 dispatch: the GEMV (m <= 16), the direct
    kernel, the k-split kernel (at least 32 k-blocks, few tiles), the 64 x 64 LDS kernel (at least
    2048 outputs), the 128 x 128 LDS kernel on narrow products (at least 256 of its tiles) and on
    wide ones (at least 1024 tiles). Sizes are ragged on purpose."""
    rng = np.random.default_rng(2024)
    regions = [((1, 16), (1, 3000), (1, 5000)), ((17, 700), (1, 1800), (1, 1000)),
               ((17, 500), (2048, 4200), (16, 1000)), ((17, 900), (1, 1500), (2048, 4000)),
               ((4096, 6000), (1, 700), (900, 2032)), ((2000, 3000), (1, 200), (8192, 12000))]
    out = []
    for (m0, m1), (k0, k1), (n0, n1) in regions:
        for _ in range(4):
            out.append((int(rng.integers(m0, m1 + 1)), int(rng.integers(k0, k1 + 1)), int(rng.integers(n0, n1 + 1)),
                        int(rng.integers(0, len(EPIS)))))
    return out


@pytest.mark.parametrize("m,k,n,e", _random_dispatch_shapes())
def test_random_shapes_in_every_dispatch_region_match_the_integer_oracle(tk, orc, m, k, n, e):
    """Whichever kernel the dispatch picks for a shape, the outputs are the integer oracle's bits."""
    rng = np.random.default_rng(m * 131 + k * 17 + n)
    a = normal(rng, m * k)
    q, s = int8_weights(rng, n, k)
    values, scales = pack_int8(q, s)
    bias, c0 = normal(rng, n), normal(rng, m * n)
    act, acc, with_bias = EPIS[e]
    b = bias if with_bias else None
    say("dispatch", m, k, n, act, acc, with_bias)
    want = c0.copy()
    assert orc.matmul_fast(a, k, m, values, scales, n, k, want, n, b, act, 0.5, acc) == 0
    got = run_gpu(tk, a, k, m, values, scales, INT8, n, k, c0, n, b, act, acc)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, k, n, act)


def test_gemv_rows_equal_gemm_rows(tk):
    import telmo_amd

    rng = np.random.default_rng(11)
    m, k, n = 64, 640, 8198
    a = normal(rng, (m, k))
    q, s = int8_weights(rng, n, k)
    values, scales = pack_int8(q, s)
    w = telmo_amd.PackedWeights.from_parts(tk, n, k, telmo_amd.Precision.INT8, values, scales)
    bias = normal(rng, n)
    epi = telmo_amd.Epilogue(bias=bias)
    say("gemv-vs-gemm", m, k, n)
    full = np.zeros(m * n, np.float32)
    tk.linear(a.reshape(-1), m, w, full, epi)
    full = full.reshape(m, n)
    for rows in range(1, 17):
        for r0 in (0, 17, m - rows):
            part = np.zeros(rows * n, np.float32)
            tk.linear(np.ascontiguousarray(a[r0:r0 + rows]).reshape(-1), rows, w, part, epi)
            assert np.array_equal(part.reshape(rows, n).view(np.uint32), full[r0:r0 + rows].view(np.uint32)), \
                (rows, r0)
    w.close()


@pytest.mark.parametrize("m", [3, 40])
def test_strides_leave_the_gaps_alone(tk, orc, m):
    rng = np.random.default_rng(12)
    k, n, lda, ldc = 100, 37, 130, 50
    a = normal(rng, m * lda)
    q, s = int8_weights(rng, n, k)
    values, scales = pack_int8(q, s)
    c0 = np.full(m * ldc, 7.25, np.float32)
    for mode in (0, 1):
        tk.set_mode(mode)
        say("strides", m, mode)
        want = c0.copy()
        if mode == 0:
            orc.matmul_fast(a, lda, m, values, scales, n, k, want, ldc, None, RELU, 2.0, True)
        else:
            orc.matmul(True, a, lda, m, values, scales, INT8, n, k, want, ldc, None, RELU, 2.0, True)
        got = run_gpu(tk, a, lda, m, values, scales, INT8, n, k, c0, ldc, None, RELU, True, 2.0)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        assert np.all(got.reshape(m, ldc)[:, n:] == 7.25)
    tk.set_mode(0)


def test_empty_and_zero_k(tk):
    import telmo_amd

    say("empty")
    w = telmo_amd.PackedWeights.from_parts(tk, 5, 0, telmo_amd.Precision.INT8, np.zeros(0, np.uint8),
                                           np.zeros(16, np.float32))
    bias = np.arange(5, dtype=np.float32) - 2
    c = np.full(15, 9.0, np.float32)
    tk.linear(np.zeros(1, np.float32), 3, w, c, telmo_amd.Epilogue(bias=bias, act=telmo_amd.Act.RELU, scale=2.0))
    assert np.array_equal(c.reshape(3, 5), np.tile(np.maximum(bias, 0) * 2, (3, 1)))
    c = np.full(15, 9.0, np.float32)
    tk.linear(np.zeros(1, np.float32), 0, w, c)  # m = 0: nothing happens
    assert np.all(c == 9.0)
    w.close()


def test_refusals_follow_the_reference(tk):
    import telmo_amd

    rng = np.random.default_rng(13)
    q, s = int8_weights(rng, 20, 64)
    values, scales = pack_int8(q, s)
    w = telmo_amd.PackedWeights.from_parts(tk, 20, 64, telmo_amd.Precision.INT8, values, scales)
    a = np.zeros(3 * 64, np.float32)
    c = np.zeros(3 * 20, np.float32)
    say("refusals")
    for args, code in [((a, 63, 3, w, c, 20), -2), ((a, 64, 3, w, c, 19), -2), ((a, 64, 4, w, c, 20), -2),
                       ((a, 64, 3, w, c[:59], 20), -2)]:
        with pytest.raises(telmo_amd.TelmoError) as e:
            tk.matmul(*args)
        assert e.value.code == code
    with pytest.raises(telmo_amd.TelmoError) as e:
        tk.linear(a, 3, w, c, telmo_amd.Epilogue(bias=np.zeros(19, np.float32)))
    assert e.value.code == -2
    with pytest.raises(telmo_amd.TelmoError) as e:
        telmo_amd.PackedWeights.from_parts(tk, 20, 64, telmo_amd.Precision.INT8, values[:-1], scales)
    assert e.value.code == -7
    w.close()


@pytest.mark.parametrize("m", [2, 30])
def test_rows_with_nan_or_inf_give_nan_rows(tk, m):
    import telmo_amd

    rng = np.random.default_rng(14)
    k, n = 128, 48
    a = normal(rng, (m, k))
    a[0, 5] = np.nan
    a[1, 7] = np.inf
    q, s = int8_weights(rng, n, k)
    values, scales = pack_int8(q, s)
    w = telmo_amd.PackedWeights.from_parts(tk, n, k, telmo_amd.Precision.INT8, values, scales)
    c = np.zeros(m * n, np.float32)
    say("nonfinite", m)
    tk.linear(a.reshape(-1), m, w, c)
    c = c.reshape(m, n)
    assert np.all(np.isnan(c[:2])) and np.all(np.isfinite(c[2:]))
    w.close()


def test_device_entry_points_match_host_ones(tk):
    import torch

    import telmo_amd

    rng = np.random.default_rng(15)
    for m, k, n in [(4, 640, 2560), (300, 1024, 1000)]:
        a = normal(rng, (m, k))
        q, s = int8_weights(rng, n, k)
        values, scales = pack_int8(q, s)
        bias = normal(rng, n)
        w = telmo_amd.PackedWeights.from_parts(tk, n, k, telmo_amd.Precision.INT8, values, scales)
        host = normal(rng, m * n)
        dev = torch.from_numpy(host.copy()).cuda()
        epi = telmo_amd.Epilogue(bias=bias, act=telmo_amd.Act.SILU, accumulate=True, scale=0.5)
        say("device", m, k, n)
        tk.linear(a.reshape(-1), m, w, host, epi)
        tk.linear_device(torch.from_numpy(a).cuda(), m, w, dev,
                         telmo_amd.Epilogue(bias=torch.from_numpy(bias).cuda(), act=telmo_amd.Act.SILU,
                                            accumulate=True, scale=0.5))
        tk.synchronize()
        assert np.array_equal(dev.cpu().numpy().view(np.uint32), host.view(np.uint32))
        w.close()


def test_glu_matches_the_reference_steps(tk, orc):
    import torch

    rng = np.random.default_rng(16)
    m, half = 7, 300
    x = normal(rng, (m, 2 * half)) * np.float32(6.0)
    out = torch.zeros((m, half), dtype=torch.float32, device="cuda")
    say("glu")
    tk.glu_device(torch.from_numpy(x).cuda(), 2 * half, m, half, out, half)
    tk.synchronize()
    got = out.cpu().numpy()
    want = np.array([[x[r, j] / (np.float32(1.0) + orc.exp_simd(np.float32(0.0) - x[r, half + j]))
                      for j in range(half)] for r in range(m)], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_config_1_at_full_size(tk, orc):
    # 750 x 1024 activations ~N(0,1), 4096 x 1024 int8 weights, scales U(0.001, 0.01), seed 0.
    rng = np.random.default_rng(0)
    m, k, n = 750, 1024, 4096
    a = normal(rng, (m, k)).reshape(-1)
    q, s = int8_weights(rng, n, k)
    values, scales = pack_int8(q, s)
    say("config1", m, k, n)
    got = run_gpu(tk, a, k, m, values, scales, INT8, n, k, np.zeros(m * n, np.float32), n, None, NONE, False, 1.0)
    want = np.zeros(m * n, np.float32)
    orc.matmul_fast(a, k, m, values, scales, n, k, want, n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ref = np.zeros(m * n, np.float32)
    orc.matmul(True, a, k, m, values, scales, INT8, n, k, ref, n)
    err = rel_norm_err(got.reshape(m, n), ref.reshape(m, n))
    print(f"[config1] row-normwise error vs the fused reference: {err:.3e}")
    assert err <= 1e-3


def test_golden_fixtures(tk):
    """The committed fixtures (tests/golden): exact mode gives the fused reference's bits for every
    precision; fast mode gives the integer oracle's bits for int8 and Q8_0."""
    from golden_cases import ACT, PREC, cases, load

    for meta in cases():
        g = load(meta)
        m, k, n, lda, ldc = meta["m"], meta["k"], meta["n"], meta["lda"], meta["ldc"]
        bias = g["bias"] if meta["bias"] else None
        p, act = PREC[meta["precision"]], ACT[meta["act"]]
        say("golden", meta["name"])
        tk.set_mode(tk.EXACT)
        try:
            got = run_gpu(tk, g["a"], lda, m, g["values"], g["scales"], p, n, k, g["c0"], ldc, bias, act,
                          meta["accumulate"], meta["scale"])
        finally:
            tk.set_mode(tk.FAST)
        assert np.array_equal(got.view(np.uint32), g["c_fused"].view(np.uint32)), meta["name"]
        if meta["precision"] in ("int8", "q8_0"):
            got = run_gpu(tk, g["a"], lda, m, g["values"], g["scales"], p, n, k, g["c0"], ldc, bias, act,
                          meta["accumulate"], meta["scale"])
            assert np.array_equal(got.view(np.uint32), g["c_fast"].view(np.uint32)), meta["name"]


def test_layer_norm_matches_the_reference_order(tk, orc):
    """LayerNorm rows on the GPU are bit-identical to the oracle's AVX-512 restatement, in place too."""
    import torch

    rng = np.random.default_rng(17)
    # 16-byte and unaligned rows, 1 to 16 rows per block, rows past the LDS-staged kernel, and batches
    # on both sides of the four-wavefront kernel's row limit
    for m, n, ldx in ((37, 1024, 1024), (5, 1000, 1003), (19, 17, 17), (3, 1, 4), (40, 4096, 4100),
                      (33, 2048, 2048), (2, 16368, 16368), (3, 16369, 16369), (21, 100, 104), (6, 1020, 1024),
                      (2050, 1024, 1024)):
        x = (2.0 + 3.0 * rng.standard_normal((m, ldx))).astype(np.float32)
        gamma = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        beta = (0.1 * rng.standard_normal(n)).astype(np.float32)
        say("layer_norm", m, n, ldx)
        want = np.array([orc.layer_norm(x[r, :n], gamma, beta, 1e-5) for r in range(m)], np.float32)
        xd = torch.from_numpy(x).cuda()
        gd, bd = torch.from_numpy(gamma).cuda(), torch.from_numpy(beta).cuda()
        out = torch.full((m, n + 2), 9.5, dtype=torch.float32, device="cuda")
        tk.layer_norm_device(xd, ldx, m, n, gd, bd, 1e-5, out, n + 2)
        tk.layer_norm_device(xd, ldx, m, n, gd, bd, 1e-5, xd, ldx)  # in place
        tk.synchronize()
        got = out.cpu().numpy()
        assert np.array_equal(got[:, :n].view(np.uint32), want.view(np.uint32)), (m, n)
        assert np.all(got[:, n:] == 9.5)
        got_in_place = xd.cpu().numpy()
        assert np.array_equal(got_in_place[:, :n].view(np.uint32), want.view(np.uint32)), (m, n)


DWCONV_CASES = [  # frames, channels, kernel, ldx, ldo, t0, stride, rows, silu
    (750, 1024, 9, 1024, 1024, 0, 1, 750, True),
    (3, 37, 9, 40, 41, 0, 1, 3, False),
    (20, 300, 4, 300, 303, 0, 1, 20, True),
    (50, 257, 7, 257, 260, 3, 2, 24, True),
    (100, 512, 15, 515, 512, 1, 2, 50, False),
    (9, 5, 1, 5, 5, 0, 1, 11, True),
    (4, 6, 0, 6, 6, 0, 1, 4, False),
    (12000, 1024, 9, 1024, 1024, 0, 1, 12000, True),
    (60, 300, 25, 300, 300, 0, 1, 60, True),  # up to 32 taps, stride 1
    (45, 100, 16, 100, 100, 0, 1, 45, False),  # up to 16 taps, stride 1
    (33, 70, 12, 70, 70, 1, 2, 16, True),  # up to 16 taps, stride 2
    (80, 129, 31, 129, 129, 2, 2, 39, False),  # up to 32 taps, stride 2
    (70, 200, 20, 200, 200, 3, 4, 17, True),  # stride 4: the direct kernel
    (90, 64, 5, 64, 64, 1, 3, 30, True),  # stride 3: the direct kernel
    (50, 64, 33, 64, 64, 0, 1, 50, True),  # 33 taps: the direct kernel
    (0, 40, 9, 40, 40, 0, 1, 3, True),  # no input frames: SiLU(bias)
]


@pytest.mark.parametrize("case", DWCONV_CASES)
def test_depthwise_conv_matches_the_reference_steps(tk, orc, case):
    """The depthwise convolution (+ SiLU) is bit-identical to the oracle's dwconv1d_frame loop, and
    leaves the gaps of out and the rows past it alone."""
    import torch

    from telmo_amd import Act

    frames, channels, kernel, ldx, ldo, t0, stride, rows, silu = case
    rng = np.random.default_rng(frames + channels + kernel)
    x = (2.0 * rng.standard_normal((frames, ldx))).astype(np.float32)
    w = (0.3 * rng.standard_normal((kernel, channels))).astype(np.float32)
    bias = rng.standard_normal(channels).astype(np.float32)
    say("dwconv1d", case)
    want = orc.dwconv1d(x[:, :channels], w, bias, rows=rows, t0=t0, stride=stride, silu=silu)
    xd = torch.from_numpy(x).cuda() if frames else None
    wd = torch.from_numpy(w).cuda() if kernel else torch.zeros(1, device="cuda")
    bd = torch.from_numpy(bias).cuda()
    out = torch.full((rows + 1, ldo), 9.5, dtype=torch.float32, device="cuda")
    tk.dwconv1d_device(xd, ldx, frames, channels, wd, kernel, bd, out, ldo, rows=rows, t0=t0, stride=stride,
                       act=Act.SILU if silu else Act.NONE)
    tk.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(got[:rows, :channels].view(np.uint32), want.view(np.uint32)), case
    assert np.all(got[:rows, channels:] == 9.5) and np.all(got[rows:] == 9.5)


@pytest.mark.parametrize("batch,frames,rows,t0,stride", [(4, 40, 40, 0, 1), (32, 375, 375, 0, 1), (3, 17, 9, 1, 2)])
def test_depthwise_conv_batches_sequences_apart(tk, orc, batch, frames, rows, t0, stride):
    """A batch of sequences laid one after another is convolved each on its own: no tap reaches into
    a neighbouring sequence."""
    import torch

    from telmo_amd import Act

    channels, kernel = 300, 9
    rng = np.random.default_rng(batch * frames)
    x = rng.standard_normal((batch * frames, channels)).astype(np.float32)
    w = (0.3 * rng.standard_normal((kernel, channels))).astype(np.float32)
    bias = rng.standard_normal(channels).astype(np.float32)
    say("dwconv1d batch", batch, frames, rows, t0, stride)
    want = np.concatenate([orc.dwconv1d(x[b * frames:(b + 1) * frames], w, bias, rows=rows, t0=t0, stride=stride,
                                        silu=True) for b in range(batch)])
    out = torch.full((batch * rows, channels), 9.5, dtype=torch.float32, device="cuda")
    tk.dwconv1d_device(torch.from_numpy(x).cuda(), channels, frames, channels, torch.from_numpy(w).cuda(), kernel,
                       torch.from_numpy(bias).cuda(), out, channels, rows=rows, t0=t0, stride=stride, act=Act.SILU,
                       batch=batch)
    tk.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_depthwise_conv_refusals(tk):
    import torch

    import telmo_amd
    from telmo_amd import Act

    x = torch.zeros((8, 16), device="cuda")
    w = torch.zeros((3, 16), device="cuda")
    b = torch.zeros(16, device="cuda")
    with pytest.raises(telmo_amd.TelmoError):
        tk.dwconv1d_device(x, 16, 8, 16, w, 3, b, torch.zeros((8, 16), device="cuda"), 16, act=Act.RELU)
    with pytest.raises(telmo_amd.TelmoError):
        tk.dwconv1d_device(x, 16, 8, 16, w, 3, b, x[4:], 16, rows=4)  # out overlaps x
    with pytest.raises(telmo_amd.TelmoError):
        tk.dwconv1d_device(x, 8, 8, 16, w, 3, b, torch.zeros((8, 16), device="cuda"), 16)  # ldx < channels


Q8_SHAPES = [(1, 32, 3), (1, 640, 200), (4, 96, 33), (8, 1280, 2560), (16, 1920, 100), (5, 2048, 70), (17, 96, 50),
             (64, 128, 96), (130, 992, 255), (257, 2048, 130), (750, 1024, 512)]


@pytest.mark.parametrize("m,k,n", Q8_SHAPES)
def test_fast_q8_0_is_bit_identical_to_its_integer_oracle(tk, orc, m, k, n):
    """Q8_0 weights in fast mode: per-block exact sums scaled in block order, on the GEMV (m <= 16)
    and the GEMM; bit-identical to the oracle, within the gate of the fused reference."""
    from helpers import pack_q8_0, q8_0_weights

    rng = np.random.default_rng(m * 7 + k * 3 + n)
    a = normal(rng, m * k)
    q, d = q8_0_weights(rng, n, k, full_range=True)
    values, scales = pack_q8_0(q, d)
    bias, c0 = normal(rng, n), normal(rng, m * n)
    for act, acc, with_bias in EPIS:
        b = bias if with_bias else None
        say("fast-q8", m, k, n, act, acc)
        want = c0.copy()
        assert orc.matmul_fast_q8(a, k, m, values, scales, n, k, want, n, b, act, 0.5, acc) == 0
        got = run_gpu(tk, a, k, m, values, scales, Q8_0, n, k, c0, n, b, act, acc)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, k, n, act)
    ref = np.zeros(m * n, np.float32)
    assert orc.matmul(True, a, k, m, values, scales, Q8_0, n, k, ref, n) == 0
    got = run_gpu(tk, a, k, m, values, scales, Q8_0, n, k, np.zeros(m * n, np.float32), n, None, NONE, False, 1.0)
    err = rel_norm_err(got.reshape(m, n), ref.reshape(m, n))
    print(f"[err] q8 m={m} k={k} n={n}: {err:.2e}")
    assert err <= 1e-3


def _random_q8_shapes():
    """Seeded random Q8_0 shapes (k a multiple of 32): the GEMV (m <= 16), the GEMM with 64 x 64
    tiles and the GEMM on products with at least 1024 128 x 128 tiles."""
    rng = np.random.default_rng(2025)
    regions = [((1, 16), (1, 90), (1, 5000)), ((17, 900), (1, 80), (1, 3000)), ((2000, 2600), (1, 6), (8192, 10000))]
    out = []
    for (m0, m1), (b0, b1), (n0, n1) in regions:
        for _ in range(3):
            out.append((int(rng.integers(m0, m1 + 1)), 32 * int(rng.integers(b0, b1 + 1)), int(rng.integers(n0, n1 + 1)),
                        int(rng.integers(0, len(EPIS)))))
    return out


@pytest.mark.parametrize("m,k,n,e", _random_q8_shapes())
def test_random_q8_0_shapes_match_the_integer_oracle(tk, orc, m, k, n, e):
    from helpers import pack_q8_0, q8_0_weights

    rng = np.random.default_rng(m * 131 + k * 17 + n + 1)
    a = normal(rng, m * k)
    q, d = q8_0_weights(rng, n, k, full_range=True)
    values, scales = pack_q8_0(q, d)
    bias, c0 = normal(rng, n), normal(rng, m * n)
    act, acc, with_bias = EPIS[e]
    b = bias if with_bias else None
    say("dispatch-q8", m, k, n, act, acc, with_bias)
    want = c0.copy()
    assert orc.matmul_fast_q8(a, k, m, values, scales, n, k, want, n, b, act, 0.5, acc) == 0
    got = run_gpu(tk, a, k, m, values, scales, Q8_0, n, k, c0, n, b, act, acc)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, k, n, act)


@pytest.mark.parametrize("m,k,n,e", [(200, 4096, 1000, 0), (300, 2080, 1500, 1), (700, 480, 1800, 2),
                                     (1000, 224, 4000, 3)])
def test_q8_0_products_on_each_tile_size(tk, orc, m, k, n, e):
    """The Q8_0 product's three tile sizes (32 x 32 below one 64 x 64 tile per CU, 32 x 64 below
    three, 64 x 64 from there): long and odd block counts (k = 4096, 2080, 480, 224: 128, 65, 15
    and 7 blocks; an odd count's last k-block holds one), partial row blocks and panels;
    bit-identical to the oracle."""
    from helpers import pack_q8_0, q8_0_weights

    rng = np.random.default_rng(m + k * 5 + n * 11)
    a = normal(rng, m * k)
    q, d = q8_0_weights(rng, n, k, full_range=True)
    values, scales = pack_q8_0(q, d)
    bias, c0 = normal(rng, n), normal(rng, m * n)
    act, acc, with_bias = EPIS[e % len(EPIS)]
    b = bias if with_bias else None
    say("q8-tiles", m, k, n, act, acc, with_bias)
    want = c0.copy()
    assert orc.matmul_fast_q8(a, k, m, values, scales, n, k, want, n, b, act, 0.5, acc) == 0
    got = run_gpu(tk, a, k, m, values, scales, Q8_0, n, k, c0, n, b, act, acc)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, k, n, act)


def test_fast_q8_0_unaligned_rows_take_the_gemm(tk, orc):
    from helpers import pack_q8_0, q8_0_weights

    rng = np.random.default_rng(31)
    m, k, n, lda = 3, 160, 40, 161
    a = normal(rng, m * lda)
    q, d = q8_0_weights(rng, n, k)
    values, scales = pack_q8_0(q, d)
    say("fast-q8-unaligned")
    want = np.zeros(m * n, np.float32)
    assert orc.matmul_fast_q8(a, lda, m, values, scales, n, k, want, n) == 0
    got = run_gpu(tk, a, lda, m, values, scales, Q8_0, n, k, np.zeros(m * n, np.float32), n, None, NONE, False, 1.0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_pack_matrices_upload_like_their_parts(tk, tmp_path):
    """Pack::matrix then upload (tg_pack_upload_matrix) gives the same products, bit for bit, as the
    same panel bytes handed to tg_weights_upload; shape mismatches are refused as the reference does."""
    import telmo_amd
    from packs import sample_pack

    data = sample_pack(lambda w, n, k, p: telmo_amd.encode(w, n, k, telmo_amd.Precision(p)))
    path = tmp_path / "sample.pack"
    path.write_bytes(data)
    pack = telmo_amd.Pack.open(str(path))
    rng = np.random.default_rng(41)
    a = normal(rng, 9 * 64)
    for name in ("w8", "wq", "wh"):
        say("pack", name)
        values, scales = pack.matrix_parts(name)
        prec = [e for e in pack.entries() if e.name == name][0].precision
        w_pack = pack.matrix(tk, name, 40, 64)
        w_parts = telmo_amd.PackedWeights.from_parts(tk, 40, 64, prec, values, scales)
        for mode in (tk.FAST, tk.EXACT):
            tk.set_mode(mode)
            c1 = np.zeros(9 * 40, np.float32)
            c2 = np.zeros(9 * 40, np.float32)
            tk.linear(a, 9, w_pack, c1)
            tk.linear(a, 9, w_parts, c2)
            assert np.array_equal(c1.view(np.uint32), c2.view(np.uint32)), (name, mode)
        tk.set_mode(tk.FAST)
        w_pack.close()
        w_parts.close()
    with pytest.raises(telmo_amd.TelmoError, match="Entry w8 is 40 x 64, and the model needs 64 x 40."):
        pack.matrix(tk, "w8", 64, 40)
    with pytest.raises(telmo_amd.TelmoError, match="Entry bias isn't a matrix."):
        pack.matrix(tk, "bias", 2, 3)
    with pytest.raises(telmo_amd.TelmoError, match="Entry nope is missing."):
        pack.matrix(tk, "nope", 2, 3)


@pytest.mark.parametrize("m,k,n", [(1100, 200, 16380), (1030, 64, 16384), (2000, 320, 4100), (4100, 200, 1000),
                                   (4100, 1000, 1000), (3000, 1024, 1000), (1500, 2048, 1000), (1440, 4096, 1000)])
def test_large_products_take_the_lds_staged_gemm_bit_exactly(tk, orc, m, k, n):
    """Products of 2048 outputs or more with >= 384 128 x 128 tiles (2000 x 4100: 16 x 33), and
    narrow products (< 2048 outputs) with >= 256 of them, run the 128 x 128 LDS-staged GEMM; narrower
    grids with more than 256 tiles of 64 x 64 the 64 x 64 one (3000 x 1000: 47 x 16; 1500 x 1000 with
    k = 2048, which the k-split kernel took before: 24 x 16; with k = 4096 and 1440 rows the k-split
    kernel's 48-row tiles instead, 480 workgroups in two rounds); partial edge tiles in
    both directions, every epilogue, bit-identical to the integer oracle. k = 1000 (16 k-blocks)
    goes round the three-stage ring five times and ends on a partial round."""
    rng = np.random.default_rng(m + k + n)
    a = normal(rng, m * k)
    q, s = int8_weights(rng, n, k)
    values, scales = pack_int8(q, s)
    bias, c0 = normal(rng, n), normal(rng, m * n)
    for act, acc, with_bias in EPIS[:3]:
        b = bias if with_bias else None
        say("large", m, k, n, act, acc)
        want = c0.copy()
        orc.matmul_fast(a, k, m, values, scales, n, k, want, n, b, act, 0.5, acc)
        got = run_gpu(tk, a, k, m, values, scales, INT8, n, k, c0, n, b, act, acc)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, k, n, act)


@pytest.mark.parametrize("m,k,n,ldc,bias_off", [(4100, 64, 4100, 4103, 0), (4100, 64, 4096, 4096, 1),
                                                 (2100, 128, 2050, 2051, 0), (2100, 128, 2048, 2048, 3)])
def test_large_products_with_unaligned_rows_or_bias(tk, orc, m, k, n, ldc, bias_off):
    """The LDS-staged GEMM's outputs go 16 bytes at a time only when c's rows and the bias are
    16-byte aligned; an odd ldc or a bias starting one or three floats into its buffer takes the
    output-at-a-time path on every tile. 128 x 128 tiles (4100 x 4100) and 64 x 64 tiles
    (2100 x 2050); bias, accumulation and the columns past n left alone, bit-identical to the
    integer oracle."""
    import torch

    import telmo_amd

    rng = np.random.default_rng(m + n + ldc + bias_off)
    a = normal(rng, (m, k))
    q, s = int8_weights(rng, n, k)
    values, scales = pack_int8(q, s)
    bias_buf = normal(rng, n + bias_off)
    bias = bias_buf[bias_off:]
    c0 = normal(rng, m * ldc)
    want = c0.copy()
    orc.matmul_fast(a.reshape(-1), k, m, values, scales, n, k, want, ldc, bias, SILU, 0.5, True)
    w = telmo_amd.PackedWeights.from_parts(tk, n, k, telmo_amd.Precision.INT8, values, scales)
    cd = torch.from_numpy(c0.copy()).cuda()
    bd = torch.from_numpy(bias_buf).cuda()[bias_off:]
    say("unaligned", m, k, n, ldc, bias_off)
    tk.matmul_device(torch.from_numpy(a).cuda(), k, m, w, cd, ldc,
                     telmo_amd.Epilogue(bias=bd, act=telmo_amd.Act.SILU, scale=0.5, accumulate=True))
    tk.synchronize()
    assert np.array_equal(cd.cpu().numpy().view(np.uint32), want.view(np.uint32)), (m, k, n, ldc, bias_off)
    w.close()


@pytest.mark.parametrize("m,k,n,ldb", [(7, 128, 255, 255), (40, 128, 255, 256), (1, 33, 16, 20), (130, 300, 40, 64)])
def test_rowmajor_right_hand_side_is_the_fused_reference(tk, orc, m, k, n, ldb):
    """BView::row_major (f32 activations as the right-hand side) gives the fused reference's bits: the
    same values packed into panels through the oracle's fused matmul. The shapes include the
    attention products' (m <= 128) x 128 -> 255."""
    import torch

    import telmo_amd

    rng = np.random.default_rng(m + k + n)
    a = normal(rng, (m, k))
    npad = -(-n // 16) * 16
    b = normal(rng, (k - 1) * ldb + npad)  # exactly what the reference's view needs
    bias = normal(rng, n)
    dense = np.stack([b[i * ldb:i * ldb + n] for i in range(k)])  # [k, n]
    values, _ = orc.encode(np.ascontiguousarray(dense.T), n, k, F32)  # the same values as 16-column panels
    for act, acc in ((NONE, False), (SILU, True)):
        c0 = normal(rng, (m, n))
        want = c0.copy()
        orc.matmul(True, a.reshape(-1), k, m, values, None, F32, n, k, want.reshape(-1), n, bias, act, 0.5, acc)
        say("rowmajor", m, k, n, ldb, act)
        cd = torch.from_numpy(c0.copy()).cuda()
        tk.matmul_rowmajor_device(torch.from_numpy(a).cuda(), k, m, torch.from_numpy(b).cuda(), k, n, ldb, cd, n,
                                  telmo_amd.Epilogue(bias=torch.from_numpy(bias).cuda(), act=telmo_amd.Act(act), scale=0.5,
                                                     accumulate=acc))
        tk.synchronize()
        assert np.array_equal(cd.cpu().numpy().view(np.uint32), want.view(np.uint32)), (m, k, n, act)
    with pytest.raises(telmo_amd.TelmoError):  # one float short of the last panel
        tk.matmul_rowmajor_device(torch.from_numpy(a).cuda(), k, m, torch.from_numpy(b[:-1]).cuda(), k, n, ldb, cd, n)


@pytest.mark.parametrize("m,k,n", [(750, 1024, 4096), (16, 640, 8198)])
def test_unit_scales_agree_with_the_library_f32_gemm(tk, orc, m, k, n):
    """With all scales 1 and no activation the product is an ordinary f32 GEMM against integer-valued
    weights: both modes are checked against hipBLASLt's f32 GEMM (TF32 / XF32 off) on the same GPU, a
    run-only cross-check with a library routine. Exact mode: two f32 sums of k products in different
    orders, so within twice the recursive-summation bound, 2 k 2^-24 sum |a_i w_i|, per output; fast
    mode: within the 1e-4 row-normwise bound."""
    import torch

    import telmo_amd

    rng = np.random.default_rng(m + n)
    q = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
    values, scales = pack_int8(q, np.ones(n, np.float32))
    w = telmo_amd.PackedWeights.from_parts(tk, n, k, telmo_amd.Precision.INT8, values, scales)
    a = normal(rng, (m, k))
    torch.backends.cuda.matmul.allow_tf32 = False
    ad = torch.from_numpy(a).cuda()
    lib = (ad @ torch.from_numpy(q.astype(np.float32)).cuda().t()).cpu().numpy()
    say("library cross-check", m, k, n)
    for mode, bound in ((telmo_amd.Kernels.EXACT, None), (telmo_amd.Kernels.FAST, 1e-4)):
        tk.set_mode(mode)
        c = torch.zeros((m, n), dtype=torch.float32, device="cuda")
        tk.linear_device(ad, m, w, c)
        tk.synchronize()
        got = c.cpu().numpy()
        if bound is None:
            mag = np.abs(a).astype(np.float64) @ np.abs(q.astype(np.float64)).T
            assert np.all(np.abs(got.astype(np.float64) - lib) <= 2 * k * 2.0**-24 * mag)
        else:
            assert rel_norm_err(got, lib) <= bound
    tk.set_mode(telmo_amd.Kernels.FAST)
    w.close()



def test_row_fixtures(tk):
    """The committed LayerNorm, GLU and depthwise-convolution fixtures, bit for bit."""
    import torch

    from golden_cases import load, rows

    from telmo_amd import Act

    for meta in rows():
        g = load(meta)
        say("row fixture", meta["name"])
        if meta["kind"] == "layer_norm":
            m, n = meta["m"], meta["n"]
            out = torch.zeros((m, n), device="cuda")
            tk.layer_norm_device(torch.from_numpy(g["x"]).cuda(), n, m, n, torch.from_numpy(g["gamma"]).cuda(),
                                 torch.from_numpy(g["beta"]).cuda(), meta["eps"], out, n)
        elif meta["kind"] == "glu":
            m, h = meta["m"], meta["half"]
            out = torch.zeros((m, h), device="cuda")
            tk.glu_device(torch.from_numpy(g["x"]).cuda(), 2 * h, m, h, out, h)
        elif meta["kind"] == "dwconv":
            c = meta["channels"]
            out = torch.zeros((meta["rows"], c), device="cuda")
            tk.dwconv1d_device(torch.from_numpy(g["x"]).cuda(), c, meta["frames"], c, torch.from_numpy(g["w"]).cuda(),
                               meta["kernel"], torch.from_numpy(g["bias"]).cuda(), out, c, rows=meta["rows"],
                               t0=meta["t0"], stride=meta["stride"], act=Act.SILU if meta["silu"] else Act.NONE)
        else:
            continue
        tk.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), g["out"].view(np.uint32)), meta["name"]


# (m, k, n, ldo): the M=750 layer's pw1 (32 x 64 GLU tiles), 128 x 128 GLU tiles, 64 x 64 ones (a
# half of 1056 outputs, which the 128 x 128 tiles do not take), ragged rows and inputs, strided and
# unaligned outputs, and products the fused kernel does not take (n % 64 != 0, GEMV rows), which go
# through the context's buffer.
GLU_SHAPES = [(750, 1024, 2048, 1024), (1100, 200, 16384, 8192), (4100, 64, 2048, 1030), (1500, 96, 2112, 1060),
              (37, 200, 256, 130), (130, 64, 128, 64), (300, 100, 96, 48), (5, 64, 128, 64)]


@pytest.mark.parametrize("m,k,n,ldo", GLU_SHAPES)
def test_linear_glu_is_linear_then_glu(tk, orc, m, k, n, ldo):
    """tg_linear_glu_device writes exactly what tg_linear_device followed by tg_glu_device writes
    (src/parakeet.rs:1087-1104), for every epilogue it accepts; and the GLU of the oracle's product
    for one of them."""
    import torch

    import telmo_amd

    rng = np.random.default_rng(m + k + n)
    a = normal(rng, (m, k))
    q, s = int8_weights(rng, n, k)
    values, scales = pack_int8(q, s)
    w = telmo_amd.PackedWeights.from_parts(tk, n, k, telmo_amd.Precision.INT8, values, scales)
    ad = torch.from_numpy(a).cuda()
    bias = torch.from_numpy(normal(rng, n)).cuda()
    half = n // 2
    for act, with_bias, scale in ((NONE, False, 1.0), (NONE, True, 1.0), (SILU, True, 0.5)):
        say("linear_glu", m, k, n, ldo, act, with_bias)
        epi = telmo_amd.Epilogue(bias=bias if with_bias else None, act=telmo_amd.Act(act), scale=scale)
        g = torch.empty((m, n), dtype=torch.float32, device="cuda")
        want = torch.full((m, ldo), 7.5, dtype=torch.float32, device="cuda")
        got = torch.full((m, ldo), 7.5, dtype=torch.float32, device="cuda")
        tk.linear_device(ad, m, w, g, epi)
        tk.glu_device(g, n, m, half, want, ldo)
        tk.linear_glu_device(ad, m, w, got, ldo, epi)
        tk.synchronize()
        assert np.array_equal(got.cpu().numpy().view(np.uint32), want.cpu().numpy().view(np.uint32)), (m, k, n)
    if m * k * n > 10 ** 9:  # the oracle is plain C; the big case is covered by the comparison above
        w.close()
        return
    # the oracle: the integer product, then the reference's glu
    c = np.zeros(m * n, np.float32)
    assert orc.matmul_fast(a.reshape(-1), k, m, values, scales, n, k, c, n, None, NONE, 1.0, False) == 0
    c = c.reshape(m, n)
    want = np.stack([orc.glu(c[r, :half], c[r, half:]) for r in range(m)])
    got = torch.empty((m, ldo), dtype=torch.float32, device="cuda")
    tk.linear_glu_device(ad, m, w, got, ldo)
    tk.synchronize()
    assert np.array_equal(got.cpu().numpy()[:, :half].view(np.uint32), want.view(np.uint32))
    w.close()


def test_linear_glu_refuses_what_it_cannot_do(tk):
    import torch

    import telmo_amd

    rng = np.random.default_rng(5)
    q, s = int8_weights(rng, 130, 64)
    w = telmo_amd.PackedWeights.from_parts(tk, 130, 64, telmo_amd.Precision.INT8, *pack_int8(q, s))
    a = torch.zeros((40, 64), dtype=torch.float32, device="cuda")
    out = torch.zeros((40, 65), dtype=torch.float32, device="cuda")
    with pytest.raises(telmo_amd.TelmoError, match="not accumulated"):
        tk.linear_glu_device(a, 40, w, out, epi=telmo_amd.Epilogue(accumulate=True))
    with pytest.raises(telmo_amd.TelmoError, match="out is too short"):
        tk.linear_glu_device(a, 40, w, out, 65, out_len=39 * 65 + 64)
    with pytest.raises(telmo_amd.TelmoError, match="ldo must be"):
        tk.linear_glu_device(a, 40, w, out, 64)
    w.close()
    q, s = int8_weights(rng, 129, 64)
    w = telmo_amd.PackedWeights.from_parts(tk, 129, 64, telmo_amd.Precision.INT8, *pack_int8(q, s))
    with pytest.raises(telmo_amd.TelmoError, match="even"):
        tk.linear_glu_device(a, 40, w, out, 65)
    w.close()


def test_strides_whose_span_wraps_size_t_are_refused_before_any_launch(tk):
    """(m - 1) * lda + k is computed without wrapping: with lda = 2^63 and m = 3 it does not fit in
    size_t, so no buffer is long enough and every entry point refuses the call on the host."""
    import torch

    import telmo_amd

    rng = np.random.default_rng(5)
    m, k, n = 3, 64, 32
    q, s = int8_weights(rng, n, k)
    values, scales = pack_int8(q, s)
    w = telmo_amd.PackedWeights.from_parts(tk, n, k, telmo_amd.Precision.INT8, values, scales)
    a = torch.zeros(m * k, device="cuda")
    c = torch.zeros(m * n, device="cuda")
    huge = 1 << 63
    say("span-wrap", m, k, n)
    with pytest.raises(telmo_amd.TelmoError, match="a is too short"):
        tk.matmul_device(a, huge, m, w, c, n)
    with pytest.raises(telmo_amd.TelmoError, match="c is too short"):
        tk.matmul_device(a, k, m, w, c, huge)
    qa = torch.zeros(tk.quant_bytes(m, k), dtype=torch.uint8, device="cuda")
    ex = torch.zeros(m, dtype=torch.int32, device="cuda")
    with pytest.raises(telmo_amd.TelmoError, match="a is too short"):
        tk.quantize_rows_device(a, huge, m, k, qa, ex)
    with pytest.raises(telmo_amd.TelmoError, match="c is too short"):
        tk.matmul_quantized_device(qa, ex, m, w, c, huge)
    with pytest.raises(telmo_amd.TelmoError, match="out is too short"):
        tk.linear_glu_device(a, m, w, c, ldo=huge)
    tk.synchronize()
    assert not c.any()
    w.close()


def test_weight_sizes_whose_byte_count_would_wrap_are_refused(tk):
    """n x k beyond 2^48 weights (or n, k beyond 2^31) is refused before the length check, so a panel
    byte count that wraps size_t cannot match a short buffer."""
    import telmo_amd

    say("weights-wrap")
    values = np.zeros(64, np.uint8)
    scales = np.zeros(16, np.float32)
    for n, k in ((1 << 40, 1 << 20), (16, 1 << 31), (1 << 31, 64)):
        with pytest.raises(telmo_amd.TelmoError, match="n and k must be"):
            telmo_amd.PackedWeights.from_parts(tk, n, k, telmo_amd.Precision.INT8, values, scales)
