"""The fused row paths of the device layer against their unfused equivalents, through the C ABI, on an
MI355X: each must write exactly the bytes of the calls it replaces.

* tg_layer_norm_quant_device = tg_layer_norm_device then tg_quantize_rows_device (digits, exponents,
  and the f32 LayerNorm when asked for, in place too);
* tg_matmul_quantized_to_quant_device = tg_matmul_quantized_device into f32 rows then
  tg_quantize_rows_device, for every launch of a sequence and every replay of a captured graph (its
  workspace of f32 rows and row maxima is rewritten by every launch);
* tg_layer_norm_pair_quant_device = tg_layer_norm_device in place then tg_layer_norm_quant_device of
  its outputs (a stack's layer boundary);
* tg_dwconv1d_quant_device = tg_dwconv1d_device then tg_quantize_rows_device, the f32 rows also
  bit-identical to the oracle's dwconv1d_frame loop.
"""
import numpy as np
import pytest

import bench
from helpers import pack_int8, int8_weights, normal

pytestmark = pytest.mark.gpu


def say(*args):
    print("[case]", *args, flush=True)


def same_floats(got, want):
    """Bit-equal outside NaNs, NaN in the same places: which NaN an operation on two NaNs returns (and
    so its sign bit) depends on the instruction the compiler picks, not on the arithmetic."""
    import torch

    nan = torch.isnan(want)
    return torch.equal(torch.isnan(got), nan) and torch.equal(got[~nan].view(torch.int32), want[~nan].view(torch.int32))


def quantised(tk, x, ldx, m, k):
    """qa and exps of rows of x through the row quantiser, qa zero-filled first."""
    import torch

    qa = torch.zeros(tk.quant_bytes(m, k), dtype=torch.uint8, device="cuda")
    ex = torch.zeros(m, dtype=torch.int32, device="cuda")
    tk.quantize_rows_device(x, ldx, m, k, qa, ex, a_len=(m - 1) * ldx + k)
    return qa, ex


LN_CASES = [(750, 1024, 1024), (12000, 1024, 1024), (37, 1000, 1003), (5, 64, 64), (19, 100, 103), (3, 4096, 4096),
            (16, 17, 17), (33, 2048, 2048), (1, 1, 4), (21, 100, 104), (40, 1020, 1020),
            (2100, 1000, 1000)]


@pytest.mark.parametrize("m,n,ldx", LN_CASES)
def test_layer_norm_quant_is_layer_norm_then_quantise(tk, m, n, ldx):
    import torch

    rng = np.random.default_rng(m + n)
    x = (1.5 + 3.0 * rng.standard_normal((m, ldx))).astype(np.float32)
    if m > 3:
        x[2, min(5, n - 1)] = np.nan  # a non-finite row
    gamma = (1.0 + 0.2 * rng.standard_normal(n)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(n)).astype(np.float32)
    say("ln_quant", m, n, ldx)
    xd, gd, bd = (torch.from_numpy(v).cuda() for v in (x, gamma, beta))
    ln = torch.full((m, n), 3.0, device="cuda")
    tk.layer_norm_device(xd, ldx, m, n, gd, bd, 1e-5, ln, n)
    want_qa, want_ex = quantised(tk, ln, n, m, n)
    qa = torch.zeros_like(want_qa)
    ex = torch.zeros_like(want_ex)
    out = torch.full((m, n), 3.0, device="cuda")
    tk.layer_norm_quant_device(xd, ldx, m, n, gd, bd, 1e-5, qa, ex, out=out)
    tk.synchronize()
    assert same_floats(out, ln)
    assert torch.equal(qa, want_qa)
    assert torch.equal(ex, want_ex)
    qa2 = torch.full_like(want_qa, 0)
    tk.layer_norm_quant_device(xd, ldx, m, n, gd, bd, 1e-5, qa2, ex)  # no f32 output
    if ldx == n:  # in place: x becomes its LayerNorm
        tk.layer_norm_quant_device(xd, ldx, m, n, gd, bd, 1e-5, qa, ex, out=xd)
        tk.synchronize()
        assert same_floats(xd, ln)
    tk.synchronize()
    assert torch.equal(qa2, want_qa)


# The one-launch kernel (< 2048 rows of <= 1024 values, a multiple of 4, aligned) with n = 1024 and
# below, and the two launches elsewhere: 2048 rows and more, n = 4096, n not a multiple of 4, a row
# stride that breaks the 16-byte alignment.
PAIR_CASES = [(750, 1024, 1024), (40, 1020, 1020), (5, 64, 64), (1, 4, 4), (33, 2048, 2048), (2100, 1000, 1000),
              (12000, 1024, 1024), (19, 100, 103), (16, 17, 17), (3, 4096, 4096), (37, 1000, 1024)]


@pytest.mark.parametrize("m,n,ldx", PAIR_CASES)
def test_layer_norm_pair_is_the_two_calls(tk, m, n, ldx):
    import torch

    rng = np.random.default_rng(m + 3 * n + ldx)
    x = (0.5 + 2.0 * rng.standard_normal((m, ldx))).astype(np.float32)
    if m > 3:
        x[2, min(5, n - 1)] = np.inf  # a non-finite row
    g1, g2 = ((1.0 + 0.2 * rng.standard_normal(n)).astype(np.float32) for _ in range(2))
    b1, b2 = ((0.1 * rng.standard_normal(n)).astype(np.float32) for _ in range(2))
    say("ln pair", m, n, ldx)
    dev = lambda a: torch.from_numpy(a).cuda()  # noqa: E731
    g1d, b1d, g2d, b2d = dev(g1), dev(b1), dev(g2), dev(b2)
    want_x = dev(x.copy())
    tk.layer_norm_device(want_x, ldx, m, n, g1d, b1d, 1e-5, want_x, ldx)
    want_qa = torch.zeros(tk.quant_bytes(m, n), dtype=torch.uint8, device="cuda")
    want_ex = torch.zeros(m, dtype=torch.int32, device="cuda")
    tk.layer_norm_quant_device(want_x, ldx, m, n, g2d, b2d, 1e-5, want_qa, want_ex)
    got_x = dev(x.copy())
    got_qa, got_ex = torch.zeros_like(want_qa), torch.zeros_like(want_ex)
    tk.layer_norm_pair_quant_device(got_x, ldx, m, n, g1d, b1d, 1e-5, g2d, b2d, 1e-5, got_qa, got_ex)
    tk.synchronize()
    assert same_floats(got_x, want_x)  # the columns past n left alone as well
    assert torch.equal(got_ex, want_ex)
    assert torch.equal(got_qa, want_qa)


# m, k, n, act, with_bias, scale. An activation or a scale other than 1 is applied by the product's
# epilogue below 2048 rows and by the quantiser, as it loads the product's biased sums, from there
# (SiLU, ReLU with a scale, a negative scale alone); with neither, the quantiser takes the row maxima
# from the product.
QOUT_CASES = [
    (750, 1024, 4096, 2, False, 1.0), (12000, 1024, 4096, 2, False, 1.0), (7500, 1024, 4096, 2, False, 0.75),
    (750, 1024, 4096, 0, True, 1.0), (12000, 1024, 4096, 0, False, 1.0),
    (37, 200, 130, 0, True, 0.75), (37, 200, 130, 0, True, 1.0), (130, 64, 200, 1, True, 0.75),
    (1, 100, 64, 2, False, -2.0), (300, 1000, 1000, 1, True, 1.0), (5000, 256, 100, 0, False, 1.0),
    (2100, 640, 4100, 2, True, 0.75), (64, 4096, 1024, 0, False, 1.0), (5, 64, 17000, 2, True, 1.0),
    (3000, 128, 640, 1, True, 0.5), (2500, 64, 300, 0, True, -1.5)]


@pytest.mark.parametrize("m,k,n,act,with_bias,scale", QOUT_CASES)
def test_quantised_output_product_is_product_then_quantise(tk, m, k, n, act, with_bias, scale):
    import torch

    import telmo_amd

    rng = np.random.default_rng(m * 3 + k + n)
    a = normal(rng, (m, k))
    if m > 10:
        a[7, 3] = np.inf  # a row whose outputs are all NaN
    q, s = int8_weights(rng, n, k)
    values, scales = pack_int8(q, s)
    w = telmo_amd.PackedWeights.from_parts(tk, n, k, telmo_amd.Precision.INT8, values, scales)
    bias = torch.from_numpy(normal(rng, n)).cuda() if with_bias else None
    epi = telmo_amd.Epilogue(bias=bias, act=telmo_amd.Act(act), scale=scale)
    say("qout", m, k, n, act, with_bias, scale)
    ad = torch.from_numpy(a).cuda()
    qa, ex = quantised(tk, ad, k, m, k)
    c = torch.zeros((m, n), device="cuda")
    tk.matmul_quantized_device(qa, ex, m, w, c, n, epi)
    want_qa, want_ex = quantised(tk, c, n, m, n)
    for rep in range(3):  # every launch rewrites the workspace it reads
        got_qa = torch.zeros_like(want_qa)
        got_ex = torch.zeros_like(want_ex)
        tk.matmul_quantized_to_quant_device(qa, ex, m, w, got_qa, got_ex, epi)
        tk.synchronize()
        assert torch.equal(got_ex, want_ex), rep
        assert torch.equal(got_qa, want_qa), rep
    w.close()


@pytest.mark.parametrize("m,k,n,act,with_bias,scale", [(750, 1024, 4096, 2, True, 1.0), (2500, 1024, 640, 2, True, 0.5),
                                                      (37, 96, 130, 0, False, 1.0), (750, 1024, 2048, 0, False, 1.0),
                                                      (37, 160, 192, 1, True, 0.5)])
def test_q8_0_quantised_output_and_glu_are_the_two_calls(tk, m, k, n, act, with_bias, scale):
    """Q8_0 weights through the quantised-output product and the quantised GLU product: the product's
    rows then the quantiser, and the product's rows then the GLU kernel, bit for bit (the GLU in the
    product's epilogue on 64 x 64 and 32 x 64 tiles when n is a multiple of 64, else through a buffer;
    k = 160 leaves the last k-block one block)."""
    import torch

    import telmo_amd
    from helpers import pack_q8_0, q8_0_weights

    rng = np.random.default_rng(m + k + n + 5)
    a = normal(rng, (m, k))
    values, scales = pack_q8_0(*q8_0_weights(rng, n, k))
    w = telmo_amd.PackedWeights.from_parts(tk, n, k, telmo_amd.Precision.Q8_0, values, scales)
    bias = torch.from_numpy(normal(rng, n)).cuda() if with_bias else None
    epi = telmo_amd.Epilogue(bias=bias, act=telmo_amd.Act(act), scale=scale)
    say("q8 qout / glu", m, k, n, act)
    qa, ex = quantised(tk, torch.from_numpy(a).cuda(), k, m, k)
    c = torch.zeros((m, n), device="cuda")
    tk.matmul_quantized_device(qa, ex, m, w, c, n, epi)
    want_qa, want_ex = quantised(tk, c, n, m, n)
    got_qa, got_ex = torch.zeros_like(want_qa), torch.zeros_like(want_ex)
    tk.matmul_quantized_to_quant_device(qa, ex, m, w, got_qa, got_ex, epi)
    want_glu = torch.zeros((m, n // 2), device="cuda")
    tk.glu_device(c, n, m, n // 2, want_glu, n // 2)
    got_glu = torch.zeros((m, n // 2), device="cuda")
    tk.matmul_quantized_glu_device(qa, ex, m, w, got_glu, epi=epi)
    tk.synchronize()
    assert torch.equal(got_ex, want_ex) and torch.equal(got_qa, want_qa)
    assert torch.equal(got_glu.view(torch.int32), want_glu.view(torch.int32))
    w.close()


def test_quantised_output_product_replays_in_a_graph(tk):
    """Captured in a HIP graph and replayed, with eager work and synchronisations between the replays,
    the product gives the eager bytes every time."""
    import torch

    import telmo_amd

    m, k, n = 750, 1024, 4096
    rng = np.random.default_rng(9)
    q, s = int8_weights(rng, n, k)
    values, scales = pack_int8(q, s)
    stream = torch.cuda.Stream()
    kern = telmo_amd.Kernels(0, stream=stream.cuda_stream)
    w = telmo_amd.PackedWeights.from_parts(kern, n, k, telmo_amd.Precision.INT8, values, scales)
    epi = telmo_amd.Epilogue(act=telmo_amd.Act.SILU)
    with torch.cuda.stream(stream):
        a = torch.from_numpy(normal(rng, (m, k))).cuda()
        qa = torch.zeros(kern.quant_bytes(m, k), dtype=torch.uint8, device="cuda")
        ex = torch.zeros(m, dtype=torch.int32, device="cuda")
        kern.quantize_rows_device(a, k, m, k, qa, ex)
        want_qa = torch.zeros(kern.quant_bytes(m, n), dtype=torch.uint8, device="cuda")
        want_ex = torch.zeros(m, dtype=torch.int32, device="cuda")
        kern.matmul_quantized_to_quant_device(qa, ex, m, w, want_qa, want_ex, epi)
        got_qa, got_ex = torch.zeros_like(want_qa), torch.zeros_like(want_ex)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            kern.matmul_quantized_to_quant_device(qa, ex, m, w, got_qa, got_ex, epi)
        for rep in range(4):
            got_qa.zero_()
            got_ex.zero_()
            graph.replay()
            kern.matmul_quantized_to_quant_device(qa, ex, m, w, want_qa, want_ex, epi)  # eager work between
            stream.synchronize()
            say("graph replay", rep)
            assert torch.equal(got_qa, want_qa) and torch.equal(got_ex, want_ex), rep
    kern.synchronize()
    w.close()
    kern.close()


def test_quantised_output_refusals(tk):
    import torch

    import telmo_amd

    m, k, n = 40, 64, 128
    rng = np.random.default_rng(3)
    q, s = int8_weights(rng, n, k)
    w = telmo_amd.PackedWeights.from_parts(tk, n, k, telmo_amd.Precision.INT8, *pack_int8(q, s))
    qa = torch.zeros(tk.quant_bytes(m, k), dtype=torch.uint8, device="cuda")
    ex = torch.zeros(m, dtype=torch.int32, device="cuda")
    qo = torch.zeros(tk.quant_bytes(m, n), dtype=torch.uint8, device="cuda")
    eo = torch.zeros(m, dtype=torch.int32, device="cuda")
    with pytest.raises(telmo_amd.TelmoError):
        tk.matmul_quantized_to_quant_device(qa, ex, m, w, qo, eo, telmo_amd.Epilogue(accumulate=True))
    with pytest.raises(telmo_amd.TelmoError):
        tk.matmul_quantized_to_quant_device(qa, ex, m, w, qo[:-1], eo)
    tk.set_mode(tk.EXACT)
    try:
        with pytest.raises(telmo_amd.TelmoError):
            tk.matmul_quantized_to_quant_device(qa, ex, m, w, qo, eo)
    finally:
        tk.set_mode(tk.FAST)
    with pytest.raises(telmo_amd.TelmoError):
        tk.layer_norm_quant_device(torch.zeros((m, k), device="cuda"), k, m, k, torch.ones(k, device="cuda"),
                                   torch.zeros(k, device="cuda"), 1e-5, qa[:-1], ex)
    w.close()


# batch, frames, channels, kernel, silu, with_out, ldx. Row blocks of 16 that straddle sequences
# (375, 20, 7 frames), sequences shorter than a block, channels past 1024 (two slices) and not a
# multiple of 64, 9 / 16 / 31 taps, a NaN and an infinity in the input.
# batch, frames, channels, kernel, silu, with_out, ldx. From 1024 rows, calls with channels a
# multiple of 4 up to 1024, kernel <= 9 and 16-byte aligned rows take the whole-block kernel, four
# rows per thread below 6144 rows and eight from there: the second group (sequences straddling
# blocks, 5 taps with an f32 output and a padded stride, a single tap, sequences of two frames
# under nine taps, an even kernel on 64 channels) and the third (12000 rows; sequences of nine
# frames, shorter than a block, with an f32 output). The rest take the row-slice kernel: four-row
# workgroups below 8192 rows, the last case 16-row ones.
DWQ_CASES = [(1, 750, 1024, 9, True, False, 1024), (5, 20, 64, 9, True, True, 64),

             (4, 375, 1024, 9, True, False, 1024), (30, 45, 1000, 5, False, True, 1004),
             (100, 13, 256, 1, True, False, 256), (520, 2, 512, 9, True, True, 516), (40, 30, 64, 4, True, False, 68),

             (32, 375, 1024, 9, True, False, 1024), (700, 9, 128, 9, True, True, 132),

             (9, 7, 100, 16, False, True, 104), (3, 40, 1000, 31, True, True, 1000),
             (2, 33, 2048, 9, True, True, 2048), (4, 16, 1500, 5, False, False, 1504), (1, 1, 3, 3, True, True, 3),
             (2, 50, 130, 1, True, False, 130), (40, 210, 1500, 9, True, False, 1500)]


@pytest.mark.parametrize("case", DWQ_CASES)
def test_dwconv_quant_is_dwconv_then_quantise(tk, orc, case):
    import torch

    from telmo_amd import Act

    batch, frames, channels, kernel, silu, with_out, ldx = case
    total = batch * frames
    rng = np.random.default_rng(total + channels + kernel)
    x = (2.0 * rng.standard_normal((total, ldx))).astype(np.float32)
    if total > 40 and channels > 20:
        x[30, 11] = np.nan
        x[total - 2, channels - 1] = np.inf
    w = (0.3 * rng.standard_normal((kernel, channels))).astype(np.float32)
    bias = rng.standard_normal(channels).astype(np.float32)
    say("dwconv_quant", case)
    act = Act.SILU if silu else Act.NONE
    xd, wd, bd = (torch.from_numpy(v).cuda() for v in (x, w, bias))
    conv = torch.full((total, channels), 9.5, device="cuda")
    tk.dwconv1d_device(xd, ldx, frames, channels, wd, kernel, bd, conv, channels, act=act, batch=batch,
                       x_len=(total - 1) * ldx + channels)
    want_qa, want_ex = quantised(tk, conv, channels, total, channels)
    qa = torch.zeros_like(want_qa)
    ex = torch.zeros_like(want_ex)
    out = torch.full((total, channels), 9.5, device="cuda") if with_out else None
    assert tk.dwconv1d_quant_device(xd, ldx, frames, channels, wd, kernel, bd, qa, ex, act=act, batch=batch,
                                    out=out, ldo=channels, x_len=(total - 1) * ldx + channels)
    tk.synchronize()
    assert torch.equal(ex, want_ex)
    assert torch.equal(qa, want_qa)
    if with_out:
        assert same_floats(out, conv)
    want = np.concatenate([orc.dwconv1d(x[b * frames:(b + 1) * frames, :channels], w, bias, silu=silu)
                           for b in range(batch)])
    got = conv.cpu().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_dwconv_quant_refusals_and_fallback(tk):
    import torch

    import telmo_amd

    xx = torch.zeros((16, 16), device="cuda")
    x = xx[:8]
    w = torch.zeros((3, 16), device="cuda")
    b = torch.zeros(16, device="cuda")
    qa = torch.zeros(tk.quant_bytes(8, 16), dtype=torch.uint8, device="cuda")
    ex = torch.zeros(8, dtype=torch.int32, device="cuda")
    with pytest.raises(telmo_amd.TelmoError):  # qa too short for 16 rows
        tk.dwconv1d_quant_device(xx, 16, 8, 16, w, 3, b, qa, ex, batch=2)
    with pytest.raises(telmo_amd.TelmoError):  # out overlaps x
        tk.dwconv1d_quant_device(x, 16, 8, 16, w, 3, b, qa, ex, out=xx[4:12], ldo=16)
    with pytest.raises(telmo_amd.TelmoError):  # ldx < channels
        tk.dwconv1d_quant_device(x, 8, 8, 16, w, 3, b, qa, ex)
    w33 = torch.zeros((33, 16), device="cuda")
    assert not tk.dwconv1d_quant_device(x, 16, 8, 16, w33, 33, b, qa, ex)  # 33 taps: the caller's two calls
