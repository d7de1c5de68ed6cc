"""Parity at the benchmark configurations' full sizes, through the entry points the benchmark and
the device layer use, on an MI355X.

* One Conformer layer's projection set at T = 750 frames (d = 1024, ff = 4096): each of
  the eight products with its epilogue: FF up (SiLU), FF down (x0.5, accumulate) on the k-split
  kernel, QKV, attention out on the strided V third of the QKV rows (lda = 3072, accumulate), pw1
  with its GLU fused, pw2 (accumulate), and the second FFN.
* The 24-layer encoder stack at M = 12000 and 7500 rows: the same products at those
  rows, on the 128 x 128 LDS-staged kernel.

Every output element is compared: bit for bit with the integer oracle (the fast path's two-digit
sums), and within 1e-3 row-normwise of the fused f32 reference (the reference's AVX-512 sums).
Inputs come from telmo's test generator (src/kernels/mod.rs:795-805): N(0, 1) activations, int8
weights in [-127, 127] and scales in [0.001, 0.01]."""
import numpy as np
import pytest

import bench
from helpers import rel_norm_err

pytestmark = pytest.mark.gpu

INT8 = 3
NONE, SILU = 0, 2
D, FF, CONV = 1024, 4096, 2048
TOL = 1e-3


def say(*args):
    print("[case]", *args, flush=True)


def weights(tk, n, k, seed):
    import telmo_amd

    values, scales = bench.panel_layout(bench.synth_int8(n, k, seed), bench.synth_scales(n, seed + 1))
    return values, scales, telmo_amd.PackedWeights.from_parts(tk, n, k, telmo_amd.Precision.INT8, values, scales)


def check_product(tk, orc, m, k, n, act, scale, accumulate, seed, lda=None):
    """One product c = epi(a . w) through Kernels.matmul_device on GPU tensors, against both oracles on
    every row. With lda > k the rows are the last k columns of [m, lda] rows (the V third of QKV)."""
    import torch

    import telmo_amd

    lda = k if lda is None else lda
    a = bench.synth_normal((m, lda), seed)
    values, scales, w = weights(tk, n, k, seed + 10)
    c0 = bench.synth_normal((m, n), seed + 20) if accumulate else np.zeros((m, n), np.float32)
    off = lda - k
    say("product", m, k, n, act, scale, accumulate, lda)
    ad = torch.from_numpy(a).cuda()
    cd = torch.from_numpy(c0).cuda()
    epi = telmo_amd.Epilogue(act=telmo_amd.Act(act), scale=scale, accumulate=accumulate)
    if lda == k:
        tk.linear_device(ad, m, w, cd, epi)
    else:
        tk.matmul_device(ad[:, off:], lda, m, w, cd, n, epi, a_len=ad.numel() - off)
    tk.synchronize()
    got = cd.cpu().numpy()
    w.close()
    flat = a.reshape(-1)[off:]
    want = c0.copy().reshape(-1)
    assert orc.matmul_fast(flat, lda, m, values, scales, n, k, want, n, None, act, scale, accumulate) == 0
    assert np.array_equal(got.reshape(-1).view(np.uint32), want.view(np.uint32)), (m, k, n)
    ref = c0.copy().reshape(-1)
    assert orc.matmul(True, flat, lda, m, values, scales, INT8, n, k, ref, n, None, act, scale, accumulate) == 0
    err = rel_norm_err(got, ref.reshape(m, n))
    print(f"[err] {m}x{k}->{n}: {err:.3e}", flush=True)
    assert err <= TOL


def check_glu(tk, orc, m, k, n, seed):
    """pw1 with its GLU (Kernels.linear_glu_device) against the oracles' product then GLU."""
    import torch

    a = bench.synth_normal((m, k), seed)
    values, scales, w = weights(tk, n, k, seed + 10)
    half = n // 2
    say("pw1+glu", m, k, n)
    out = torch.full((m, half), 7.0, device="cuda")
    tk.linear_glu_device(torch.from_numpy(a).cuda(), m, w, out)
    tk.synchronize()
    got = out.cpu().numpy()
    w.close()
    g = np.zeros(m * n, np.float32)
    assert orc.matmul_fast(a.reshape(-1), k, m, values, scales, n, k, g, n) == 0
    g = g.reshape(m, n)
    want = np.stack([orc.glu(g[r, :half], g[r, half:]) for r in range(m)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ref = np.zeros(m * n, np.float32)
    assert orc.matmul(True, a.reshape(-1), k, m, values, scales, INT8, n, k, ref, n) == 0
    ref = ref.reshape(m, n)
    ref_glu = np.stack([orc.glu(ref[r, :half], ref[r, half:]) for r in range(m)]).astype(np.float64)
    ra, rb = ref[:, :half].astype(np.float64), ref[:, half:].astype(np.float64)
    sig = 1.0 / (1.0 + np.exp(-rb))
    # The product's own gate (1e-3 of each half's row maximum) carried through the GLU to first
    # order: d(a s(b)) = s(b) da + a s(b) (1 - s(b)) db. The GLU amplifies the b half's error by up
    # to |a| / 4, so the output's row-normwise error alone is no measure of the product's.
    ma = np.abs(ra).max(axis=1, keepdims=True)
    mb = np.abs(rb).max(axis=1, keepdims=True)
    bound = TOL * (ma * sig + np.abs(ra) * sig * (1.0 - sig) * mb) + 1e-6 * np.abs(ref_glu).max(axis=1, keepdims=True)
    excess = (np.abs(got - ref_glu) / bound).max()
    print(f"[err] {m}x{k}->{n} + GLU: {rel_norm_err(got, ref_glu):.3e} row-normwise, "
          f"{excess:.3f} of the propagated 1e-3 bound", flush=True)
    assert excess <= 1.0


# name, k, n, act, scale, accumulate, lda: the layer's products in Parakeet::layer's order
# (src/parakeet.rs:1011-1172)
PRODUCTS = [
    ("ff1_up", D, FF, SILU, 1.0, False, None),
    ("ff1_down", FF, D, NONE, 0.5, True, None),
    ("qkv", D, 3 * D, NONE, 1.0, False, None),
    ("att_out", D, D, NONE, 1.0, True, 3 * D),
    ("pw2", D, D, NONE, 1.0, True, None),
    ("ff2_up", D, FF, SILU, 1.0, False, None),
    ("ff2_down", FF, D, NONE, 0.5, True, None),
]


@pytest.mark.parametrize("name,k,n,act,scale,acc,lda", PRODUCTS, ids=[p[0] for p in PRODUCTS])
def test_layer_products_at_750_frames(tk, orc, name, k, n, act, scale, acc, lda):
    check_product(tk, orc, 750, k, n, act, scale, acc, seed=100 + PRODUCTS.index(
        (name, k, n, act, scale, acc, lda)) * 50, lda=lda)


def test_layer_pw1_glu_at_750_frames(tk, orc):
    check_glu(tk, orc, 750, D, CONV, seed=900)


BIG = [
    (12000, "ff_up", D, FF, SILU, 1.0, False, None),
    (12000, "ff_down", FF, D, NONE, 0.5, True, None),
    (12000, "qkv", D, 3 * D, NONE, 1.0, False, None),
    (12000, "att_out", D, D, NONE, 1.0, True, 3 * D),
    (12000, "pw2", D, D, NONE, 1.0, True, None),
    (7500, "ff_up", D, FF, SILU, 1.0, False, None),
    (7500, "ff_down", FF, D, NONE, 0.5, True, None),
]


@pytest.mark.parametrize("m,name,k,n,act,scale,acc,lda", BIG, ids=[f"{b[0]}-{b[1]}" for b in BIG])
def test_encoder_stack_products(tk, orc, m, name, k, n, act, scale, acc, lda):
    check_product(tk, orc, m, k, n, act, scale, acc, seed=2000 + BIG.index((m, name, k, n, act, scale, acc, lda)) * 50,
                  lda=lda)


@pytest.mark.parametrize("m", [12000, 7500])
def test_encoder_stack_pw1_glu(tk, orc, m):
    check_glu(tk, orc, m, D, CONV, seed=3000 + m)


# Call sites outside the benchmark's workloads whose shapes no other test reaches: Granite's out_mid (the CTC
# posteriors back to the hidden width, k = vocab = 16384, src/granite.rs:1060-1067) in chunks of 2,
# 16 and 256 rows with its bias, and Parakeet's subsampling pw1 (k = 256 channels, m = 64 T rows for
# T encoder frames, ReLU and bias, src/parakeet.rs:950-960).
def test_granite_out_mid_shape(tk, orc):
    import torch

    import telmo_amd

    k, n = 16384, 1024
    values, scales, w = weights(tk, n, k, 4000)
    bias = bench.synth_normal((n,), 4002)
    for m in (2, 16, 256):
        say("granite mid", m, k, n)
        a = np.abs(bench.synth_normal((m, k), 4003 + m)) * np.float32(1e-4)  # softmax rows: small, positive
        c = torch.zeros((m, n), device="cuda")
        tk.linear_device(torch.from_numpy(a).cuda(), m, w, c, telmo_amd.Epilogue(bias=torch.from_numpy(bias).cuda()))
        tk.synchronize()
        got = c.cpu().numpy()
        want = np.zeros(m * n, np.float32)
        orc.matmul_fast(a.reshape(-1), k, m, values, scales, n, k, want, n, bias)
        assert np.array_equal(got.reshape(-1).view(np.uint32), want.view(np.uint32)), m
        ref = np.zeros(m * n, np.float32)
        orc.matmul(True, a.reshape(-1), k, m, values, scales, INT8, n, k, ref, n, bias)
        assert rel_norm_err(got, ref.reshape(m, n)) <= TOL
    w.close()


def test_parakeet_subsampling_pw1_shape(tk, orc):
    import torch

    import telmo_amd

    m, k, n = 64 * 750, 256, 256
    values, scales, w = weights(tk, n, k, 5000)
    bias = bench.synth_normal((n,), 5002)
    a = bench.synth_normal((m, k), 5003)
    say("parakeet sub.pw1", m, k, n)
    c = torch.zeros((m, n), device="cuda")
    tk.linear_device(torch.from_numpy(a).cuda(), m, w, c,
                     telmo_amd.Epilogue(bias=torch.from_numpy(bias).cuda(), act=telmo_amd.Act.RELU))
    tk.synchronize()
    got = c.cpu().numpy()
    w.close()
    want = np.zeros(m * n, np.float32)
    orc.matmul_fast(a.reshape(-1), k, m, values, scales, n, k, want, n, bias, 1)
    assert np.array_equal(got.reshape(-1).view(np.uint32), want.view(np.uint32))
    ref = np.zeros(m * n, np.float32)
    orc.matmul(True, a.reshape(-1), k, m, values, scales, INT8, n, k, ref, n, bias, 1)
    assert rel_norm_err(got, ref.reshape(m, n)) <= TOL


# The fast path's error bound. Each row's inputs are rounded to 15 bits of their largest magnitude,
# so the error of an output grows with kappa = max|a| sqrt(k) / ||a||_2 of its row: about 3.4 for
# N(0, 1) rows, up to sqrt(k) for a row that is one spike. Measured on random int8 weights, the
# row-normwise error stays below FAST_ERR_PER_KAPPA * kappa (1.4e-5 to 3.3e-5 over k = 1024 to
# 16384 and spikes of 10 to 1000 sigma), so without a guard the 1e-3 gate holds up to kappa of
# about 28. The product entry points' accuracy guard (on by default) flags the rows whose two digits
# drop more than 2^-12 of the row and gives them the fused reference's sums: every row then meets
# the gate.
FAST_ERR_PER_KAPPA = 3.5e-5


@pytest.mark.parametrize("k,spike,epi", [(4096, 300.0, 0), (16384, 30.0, 0), (16384, 300.0, 0), (1024, 1000.0, 0),
                                         (4096, 300.0, 1), (16384, 300.0, 1), (4096, 25.0, 0), (16384, 12.0, 1)])
def test_rows_with_a_spike_meet_the_gate_under_the_guard(tk, orc, k, spike, epi):
    """Heavy-tailed rows (one input of `spike` sigma per row, the rest N(0, 1)), kappa up to sqrt(k):
    with the guard every row is within 1e-3 of the fused reference, the flagged ones bit-equal to it,
    and the whole product equals the guarded integer oracle; with the guard off the product equals
    the integer oracle and each row stays within FAST_ERR_PER_KAPPA * kappa; the exact mode gives the
    fused reference's bits. epi 1: bias, SiLU, scale 0.5 and accumulation onto nonzero rows."""
    import torch

    import telmo_amd

    m, n = 96, 1024
    rng = np.random.default_rng(k + int(spike))
    a = bench.synth_normal((m, k), 6000 + k)
    a[np.arange(m), rng.integers(0, k, m)] = np.float32(spike) * np.sign(rng.standard_normal(m)).astype(np.float32)
    values, scales, w = weights(tk, n, k, 6100)
    c0 = bench.synth_normal((m, n), 6200) if epi else np.zeros((m, n), np.float32)
    bias = bench.synth_normal((n,), 6300) if epi else None
    act, scale, acc = (2, 0.5, True) if epi else (0, 1.0, False)
    e = telmo_amd.Epilogue(bias=None if bias is None else torch.from_numpy(bias).cuda(), act=telmo_amd.Act(act),
                           scale=scale, accumulate=acc)
    say("spike", m, k, n, spike, epi)
    ad = torch.from_numpy(a).cuda()

    def run():
        c = torch.from_numpy(c0.copy()).cuda()
        tk.linear_device(ad, m, w, c, e)
        tk.synchronize()
        return c.cpu().numpy()

    def oracle(guard):
        out = c0.copy().reshape(-1)
        assert orc.matmul_fast(a.reshape(-1), k, m, values, scales, n, k, out, n, bias, act, scale, acc,
                               guard=guard) == 0
        return out.reshape(m, n)

    ref = c0.copy().reshape(-1)
    orc.matmul(True, a.reshape(-1), k, m, values, scales, INT8, n, k, ref, n, bias, act, scale, acc)
    ref = ref.reshape(m, n)
    flags = orc.guard_flags(a.reshape(-1), k, m, k).astype(bool)
    kappa = np.abs(a).max(axis=1) * np.sqrt(k) / np.linalg.norm(a.astype(np.float64), axis=1)

    assert tk.guard()
    got = run()
    assert np.array_equal(got.view(np.uint32), oracle(True).view(np.uint32))
    assert np.array_equal(got[flags].view(np.uint32), ref[flags].view(np.uint32))
    per_row = np.abs(got - ref).max(axis=1) / np.abs(ref).max(axis=1)
    print(f"[err] k={k} spike={spike} epi={epi}: {flags.sum()} of {m} rows flagged (kappa "
          f"{kappa[flags].min() if flags.any() else 0:.1f}+), max err {per_row.max():.2e}, unflagged kappa up to "
          f"{kappa[~flags].max() if (~flags).any() else 0:.1f}", flush=True)
    assert per_row.max() <= 1e-3

    tk.set_guard(False)
    try:
        got = run()
    finally:
        tk.set_guard(True)
    assert np.array_equal(got.view(np.uint32), oracle(False).view(np.uint32))
    if not epi:
        per_row = np.abs(got - ref).max(axis=1) / np.abs(ref).max(axis=1)
        assert np.all(per_row <= FAST_ERR_PER_KAPPA * kappa)

    tk.set_mode(tk.EXACT)
    try:
        got = run()
    finally:
        tk.set_mode(tk.FAST)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    w.close()


def test_guard_on_the_host_and_no_allocation_entry_points(tk, orc):
    """The host-pointer tg_linear and tg_matmul_device_noalloc apply the same guard: the guarded
    oracle's bits, with accumulation. Rows of the decode GEMV (here 8 aligned rows of 640) are not
    guarded: the unguarded oracle's bits."""
    import torch

    import telmo_amd

    m, k, n = 64, 4096, 512
    a = bench.synth_normal((m, k), 6400)
    a[::3, 7] = np.float32(500.0)
    values, scales, w = weights(tk, n, k, 6500)
    c0 = bench.synth_normal((m, n), 6600)
    want = c0.copy().reshape(-1)
    orc.matmul_fast(a.reshape(-1), k, m, values, scales, n, k, want, n, None, 0, 1.0, True, guard=True)
    flags = orc.guard_flags(a.reshape(-1), k, m, k)
    assert 0 < flags.sum() < m
    say("guard host", m, k, n)
    got = c0.copy()
    tk.linear(a, m, w, got, telmo_amd.Epilogue(accumulate=True))
    assert np.array_equal(got.reshape(-1).view(np.uint32), want.view(np.uint32))
    say("guard noalloc", m, k, n)
    cd = torch.from_numpy(c0.copy()).cuda()
    tk.matmul_device_noalloc(torch.from_numpy(a).cuda(), k, m, w, cd, n, telmo_amd.Epilogue(accumulate=True))
    tk.synchronize()
    assert np.array_equal(cd.cpu().numpy().reshape(-1).view(np.uint32), want.view(np.uint32))
    w.close()

    m, k, n = 8, 640, 256
    a = bench.synth_normal((m, k), 6700)
    a[:, 5] = np.float32(3000.0)
    values, scales, w = weights(tk, n, k, 6800)
    assert orc.guard_flags(a.reshape(-1), k, m, k).all()
    say("guard gemv", m, k, n)
    cd = torch.zeros((m, n), device="cuda")
    tk.linear_device(torch.from_numpy(a).cuda(), m, w, cd)
    tk.synchronize()
    want = np.zeros(m * n, np.float32)
    orc.matmul_fast(a.reshape(-1), k, m, values, scales, n, k, want, n)
    assert np.array_equal(cd.cpu().numpy().reshape(-1).view(np.uint32), want.view(np.uint32))
    w.close()


def test_granite_rel_table_goes_through_matmul(tk, orc):
    """Granite's relative-position table is a PackedWeights [2 context - 1, head_dim]
    (src/granite.rs:199, 474), multiplied by the block's query rows, which sit 3 d apart in the QKV
    rows (matmul_serial with lda = 3 d, src/granite.rs:1003-1014): (m <= 128) x 128 -> 255 through
    Kernels.matmul, the integer oracle's bits."""
    import torch

    import telmo_amd

    d, hd, n = 1024, 128, 255
    values, scales, w = weights(tk, n, hd, 7000)
    for m in (1, 37, 128):
        q = bench.synth_normal((m, 3 * d), 7002 + m)
        say("granite rel", m, hd, n)
        c = torch.zeros((m, n), device="cuda")
        epi = telmo_amd.Epilogue(scale=0.088)
        qd = torch.from_numpy(q).cuda()
        tk.matmul_device(qd, 3 * d, m, w, c, n, epi, a_len=(m - 1) * 3 * d + hd)
        tk.synchronize()
        want = np.zeros(m * n, np.float32)
        orc.matmul_fast(q.reshape(-1)[:(m - 1) * 3 * d + hd], 3 * d, m, values, scales, n, hd, want, n, None, NONE,
                        0.088)
        assert np.array_equal(c.cpu().numpy().reshape(-1).view(np.uint32), want.view(np.uint32)), m
    w.close()


def test_row_kernels_refuse_buffers_shorter_than_their_rows(tk):
    """The row kernels check the lengths of their buffers against the rows they touch, as the
    reference asserts its slices (src/kernels/avx512.rs:348, 412; scalar.rs:174-182), before any
    launch; the wrappers keep those lengths inside each tensor's storage."""
    import torch

    import telmo_amd
    from telmo_amd import _lib

    L = _lib.lib()
    x = torch.zeros((4, 32), device="cuda")
    g = torch.ones(32, device="cuda")
    out = torch.zeros((4, 32), device="cuda")
    p = lambda t: t.data_ptr()  # noqa: E731
    # LayerNorm: gamma one value short, then out one row short
    assert L.tg_layer_norm_device(tk._ctx, p(x), 128, 32, 4, 32, p(g), 31, p(g), 32, 1e-5, p(out), 128, 32) == -2
    assert L.tg_layer_norm_device(tk._ctx, p(x), 128, 32, 4, 32, p(g), 32, p(g), 32, 1e-5, p(out), 127, 32) == -2
    assert L.tg_layer_norm_device(tk._ctx, p(x), 127, 32, 4, 32, p(g), 32, p(g), 32, 1e-5, p(out), 128, 32) == -2
    # GLU: x holds 4 rows of 2 x 16, out 4 rows of 16
    assert L.tg_glu_device(tk._ctx, p(x), 127, 32, 4, 16, p(out), 128, 32) == -2
    assert L.tg_glu_device(tk._ctx, p(x), 128, 32, 4, 16, p(out), 3 * 32 + 15, 32) == -2
    assert L.tg_glu_device(tk._ctx, p(x), 128, 32, 4, 16, p(out), 3 * 32 + 16, 32) == 0
    # depthwise convolution: bias, taps, input and output each one short
    w = torch.zeros((3, 32), device="cuda")
    args = lambda xl, wl, bl, ol: (tk._ctx, p(x), xl, 32, 4, 1, 32, p(w), wl, 3, p(g), bl, 0, 1, 4, 0, p(out), ol, 32)  # noqa: E731
    assert L.tg_dwconv1d_device(*args(128, 96, 31, 128)) == -2
    assert L.tg_dwconv1d_device(*args(128, 95, 32, 128)) == -2
    assert L.tg_dwconv1d_device(*args(127, 96, 32, 128)) == -2
    assert L.tg_dwconv1d_device(*args(128, 96, 32, 127)) == -2
    assert L.tg_dwconv1d_device(*args(128, 96, 32, 128)) == 0
    tk.synchronize()
    # the wrappers: an expanded view counts more elements than its storage holds
    with pytest.raises(ValueError):
        tk.layer_norm_device(torch.zeros(1, device="cuda").expand(4 * 32), 32, 4, 32, g, g, 1e-5, out, 32)
    with pytest.raises(telmo_amd.TelmoError):  # out[1:] holds three of the four rows
        tk.glu_device(x, 32, 4, 16, out[1:], 32)
    with pytest.raises(telmo_amd.TelmoError):
        tk.layer_norm_device(x, 32, 4, 32, g[:31], g, 1e-5, out, 32)
