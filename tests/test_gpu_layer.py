"""The device Conformer layer (telmo_amd.conformer, Parakeet::layer of src/parakeet.rs:1011-1172) against
the same sequence composed from the oracle's functions (tests/layer_oracle.py), on an MI355X.

* Bit for bit against the composition with the integer oracle: every fused step writes what its
  unfused calls write, so the whole layer must give the integer oracle's bits.
* Within 1e-3 row-normwise of the composition with the reference's fused f32 products.
* At T = 750 (d = 1024, ff = 4096), two layers stacked (also through run_stack), and the batch of 32
  utterances of 375 frames (12000 rows), whose utterances are independent: the first two and
  the last are checked.
"""
import numpy as np
import pytest

import bench
import layer_oracle
from helpers import rel_norm_err

pytestmark = pytest.mark.gpu

D, FF, K = 1024, 4096, 9


def say(*args):
    print("[case]", *args, flush=True)


def device_layer(tk, mats, norms, dw_w, dw_b, precision=3):
    import torch

    import telmo_amd
    from telmo_amd.conformer import LayerWeights

    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    W = {name: telmo_amd.PackedWeights.from_parts(tk, n, k, telmo_amd.Precision(precision), v, s)
         for name, (v, s, n, k) in mats.items()}
    return LayerWeights(W, {name: (dev(g), dev(b)) for name, (g, b) in norms.items()}, dev(dw_w), dev(dw_b))


def run_device(tk, layers, x, utterances, quantised_hidden=False, stack=False):
    """The layers in turn; stack: through run_stack, each boundary one call."""
    import torch

    from telmo_amd.conformer import ConformerLayer

    t = x.shape[0]
    layer = ConformerLayer(tk, D, FF, K, t, quantised_hidden=quantised_hidden)
    xd = torch.from_numpy(x.copy()).cuda()
    if stack:
        layer.run_stack(xd, t, layers, utterances=utterances)
    else:
        for w in layers:
            layer.forward(xd, t, w, utterances=utterances)
    tk.synchronize()
    return xd.cpu().numpy()


def close(layers):
    for w in layers:
        for m in w.mats.values():
            m.close()


@pytest.mark.parametrize("quantised_hidden", [False, True])
def test_layer_at_750_frames(tk, orc, quantised_hidden):
    mats, norms, dw_w, dw_b = bench.layer_params(100)
    x = bench.synth_normal((750, D), 7)
    say("layer", 750, quantised_hidden)
    w = device_layer(tk, mats, norms, dw_w, dw_b)
    got = run_device(tk, [w], x, 1, quantised_hidden)
    close([w])
    want = layer_oracle.oracle_layer(orc, x, mats, norms, dw_w, dw_b, fast=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ref = layer_oracle.oracle_layer(orc, x, mats, norms, dw_w, dw_b, fast=False)
    err = rel_norm_err(got, ref)
    print(f"[err] one layer at T=750 against the f32 reference layer: {err:.3e}", flush=True)
    assert err <= 1e-3


@pytest.mark.parametrize("stack", [False, True])
def test_two_stacked_layers(tk, orc, stack):
    """Two layers, as two calls of forward or through run_stack (the boundary's two LayerNorms in one
    call, the second layer starting from the quantised rows it leaves)."""
    p1 = bench.layer_params(400)
    p2 = bench.layer_params(700)
    x = bench.synth_normal((750, D), 8)
    say("two layers", 750, stack)
    ws = [device_layer(tk, *p1), device_layer(tk, *p2)]
    got = run_device(tk, ws, x, 1, stack=stack)
    close(ws)
    want = layer_oracle.oracle_layer(orc, layer_oracle.oracle_layer(orc, x, *p1, fast=True), *p2, fast=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ref = layer_oracle.oracle_layer(orc, layer_oracle.oracle_layer(orc, x, *p1, fast=False), *p2, fast=False)
    err = rel_norm_err(got, ref)
    print(f"[err] two layers at T=750 against the f32 reference: {err:.3e}", flush=True)
    assert err <= 1e-3


def test_three_stacked_layers_on_ragged_rows(tk, orc):
    """37 frames (a partial 16-row block) through three layers: run_stack, whose two boundaries are
    one launch each, writes the bits of three plain calls of forward, and the integer oracle's."""
    params = [bench.layer_params(1500 + 100 * i) for i in range(3)]
    x = bench.synth_normal((37, D), 11)
    say("three layers", 37)
    ws = [device_layer(tk, *p) for p in params]
    stacked = run_device(tk, ws, x, 1, stack=True)
    plain = run_device(tk, ws, x, 1)
    close(ws)
    assert np.array_equal(stacked.view(np.uint32), plain.view(np.uint32))
    want = x
    for p in params:
        want = layer_oracle.oracle_layer(orc, want, *p, fast=True)
    assert np.array_equal(stacked.view(np.uint32), want.view(np.uint32))


def test_batch_of_32_utterances(tk, orc):
    """M = 12000 rows: 32 utterances of 375 frames, each convolved on its own."""
    mats, norms, dw_w, dw_b = bench.layer_params(1000)
    frames, utt = 375, 32
    x = bench.synth_normal((frames * utt, D), 9)
    say("layer batch", frames * utt)
    w = device_layer(tk, mats, norms, dw_w, dw_b)
    got = run_device(tk, [w], x, utt, quantised_hidden=True)
    close([w])
    for u in (0, 1, utt - 1):
        rows = slice(u * frames, (u + 1) * frames)
        want = layer_oracle.oracle_layer(orc, x[rows], mats, norms, dw_w, dw_b, fast=True)
        assert np.array_equal(got[rows].view(np.uint32), want.view(np.uint32)), u
        ref = layer_oracle.oracle_layer(orc, x[rows], mats, norms, dw_w, dw_b, fast=False)
        err = rel_norm_err(got[rows], ref)
        print(f"[err] utterance {u} of the 32 x 375-frame batch against the f32 reference: {err:.3e}", flush=True)
        assert err <= 1e-3


def test_one_600_s_utterance(tk, orc):
    """M = 7500 rows of one utterance (one 600 s utterance: the 16-row-block convolution with eight rows
    per thread, the four-row LayerNorm at 7500 rows). Only the depthwise convolution mixes rows (four
    on either side), so windows of the output are checked against the oracle run on the window's
    rows and four more on each side: the first, a middle and the last 256 rows."""
    mats, norms, dw_w, dw_b = bench.layer_params(1200)
    t, half = 7500, K // 2
    x = bench.synth_normal((t, D), 10)
    say("layer one utterance", t)
    w = device_layer(tk, mats, norms, dw_w, dw_b)
    got = run_device(tk, [w], x, 1, quantised_hidden=True)
    close([w])
    for r0, r1 in ((0, 256), (3700, 3956), (t - 256, t)):
        lo, hi = max(0, r0 - half), min(t, r1 + half)
        want = layer_oracle.oracle_layer(orc, x[lo:hi], mats, norms, dw_w, dw_b, fast=True)[r0 - lo:r1 - lo]
        assert np.array_equal(got[r0:r1].view(np.uint32), want.view(np.uint32)), (r0, r1)
        ref = layer_oracle.oracle_layer(orc, x[lo:hi], mats, norms, dw_w, dw_b, fast=False)[r0 - lo:r1 - lo]
        err = rel_norm_err(got[r0:r1], ref)
        print(f"[err] rows {r0}-{r1} of one 7500-frame utterance against the f32 reference: {err:.3e}", flush=True)
        assert err <= 1e-3


@pytest.mark.parametrize("quantised_hidden", [True, False])
def test_q8_0_layer_at_750_frames(tk, orc, quantised_hidden):
    """The layer with Q8_0 matrices (Parakeet's recommended precision), the Q8_0 GEMM everywhere and
    the quantised GLU product, the feed-forward's hidden rows through the quantised-output product
    or through f32 rows and the row quantiser, against the oracle composition with the Q8_0 integer
    oracle."""
    mats, norms, dw_w, dw_b = bench.layer_params(1400, precision=4)
    x = bench.synth_normal((750, D), 15)
    say("layer q8_0", 750, "quantised hidden" if quantised_hidden else "f32 hidden")
    w = device_layer(tk, mats, norms, dw_w, dw_b, precision=4)
    got = run_device(tk, [w], x, 1, quantised_hidden=quantised_hidden)
    close([w])
    want = layer_oracle.oracle_layer(orc, x, mats, norms, dw_w, dw_b, fast=True, precision=4)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ref = layer_oracle.oracle_layer(orc, x, mats, norms, dw_w, dw_b, fast=False, precision=4)
    err = rel_norm_err(got, ref)
    print(f"[err] the Q8_0 layer at T=750 against the f32 reference: {err:.3e}", flush=True)
    assert err <= 1e-3


def test_layer_refuses_other_precisions(tk):
    """The device layer's products are the staged entry points, which take int8 and Q8_0 matrices:
    a layer holding another precision is refused before any launch."""
    import torch

    import telmo_amd
    from telmo_amd.conformer import ConformerLayer

    mats, norms, dw_w, dw_b = bench.layer_params(1700)
    w = device_layer(tk, mats, norms, dw_w, dw_b)
    _, _, n, k = mats["ff1_in"]
    f16 = telmo_amd.PackedWeights.from_parts(tk, n, k, telmo_amd.Precision.F16,
                                             np.zeros(-(-n // 16) * 16 * k * 2, np.uint8))
    w.mats["ff1_in"].close()
    w.mats["ff1_in"] = f16
    layer = ConformerLayer(tk, D, FF, K, 64)
    x = torch.zeros((64, D), device="cuda")
    with pytest.raises(ValueError, match="int8 or Q8_0"):
        layer.forward(x, 64, w)
    close([w])


def test_position_projection(tk, orc):
    """The attention's position projection (Parakeet::layer's pos_proj of the relative positions,
    conformer.py's pos branch): p_out = pos . W through tg_linear_device, with the accuracy guard."""
    import torch

    import telmo_amd
    from telmo_amd.conformer import ConformerLayer

    mats, norms, dw_w, dw_b = bench.layer_params(1600)
    t = 300
    q, sc = bench.synth_int8(D, D, 1650), bench.synth_scales(D, 1651)
    pv, ps = bench.panel_layout(q, sc)
    mats = dict(mats, pos=(pv, ps, D, D))
    x = bench.synth_normal((t, D), 16)
    pos = bench.synth_normal((2 * t - 1, D), 17)
    say("layer pos", t)
    w = device_layer(tk, mats, norms, dw_w, dw_b)
    layer = ConformerLayer(tk, D, FF, K, t)
    xd = torch.from_numpy(x.copy()).cuda()
    p_out = torch.zeros((2 * t - 1, D), device="cuda")
    layer.forward(xd, t, w, pos=torch.from_numpy(pos).cuda(), p_out=p_out)
    tk.synchronize()
    close([w])
    want = np.zeros((2 * t - 1) * D, np.float32)
    assert orc.matmul_fast(pos.reshape(-1), D, 2 * t - 1, pv, ps, D, D, want, D, guard=True) == 0
    assert np.array_equal(p_out.cpu().numpy().reshape(-1).view(np.uint32), want.view(np.uint32))
    # the layer's own output is unchanged by the projection
    mats.pop("pos")
    want_x = layer_oracle.oracle_layer(orc, x, mats, norms, dw_w, dw_b, fast=True)
    assert np.array_equal(xd.cpu().numpy().view(np.uint32), want_x.view(np.uint32))
    assert telmo_amd.Precision.INT8 == 3
