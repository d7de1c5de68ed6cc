"""The device Conformer layer (telmo_amd.conformer, Parakeet::layer of src/parakeet.rs:1011-1172) against
the same sequence composed from the oracle's functions (tests/layer_oracle.py), on an MI355X.

* Bit for bit against the composition with the integer oracle: every fused step writes what its
  unfused calls write, so the whole layer must give the integer oracle's bits.
* Within 1e-3 row-normwise of the composition with the reference's fused f32 products.
* At T = 750 (config 2's shapes), two layers stacked, and the batch of 32 utterances of 375 frames
  (config 3's rows), whose utterances are independent: the first two and the last are checked.
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


def device_layer(tk, mats, norms, dw_w, dw_b):
    import torch

    import telmo_amd
    from telmo_amd.conformer import LayerWeights

    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    W = {name: telmo_amd.PackedWeights.from_parts(tk, n, k, telmo_amd.Precision.INT8, v, s)
         for name, (v, s, n, k) in mats.items()}
    return LayerWeights(W, {name: (dev(g), dev(b)) for name, (g, b) in norms.items()}, dev(dw_w), dev(dw_b))


def run_device(tk, layers, x, utterances, quantised_hidden=False):
    import torch

    from telmo_amd.conformer import ConformerLayer

    t = x.shape[0]
    layer = ConformerLayer(tk, D, FF, K, t, quantised_hidden=quantised_hidden)
    xd = torch.from_numpy(x.copy()).cuda()
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


def test_two_stacked_layers(tk, orc):
    p1 = bench.layer_params(400)
    p2 = bench.layer_params(700)
    x = bench.synth_normal((750, D), 8)
    say("two layers", 750)
    ws = [device_layer(tk, *p1), device_layer(tk, *p2)]
    got = run_device(tk, ws, x, 1)
    close(ws)
    want = layer_oracle.oracle_layer(orc, layer_oracle.oracle_layer(orc, x, *p1, fast=True), *p2, fast=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ref = layer_oracle.oracle_layer(orc, layer_oracle.oracle_layer(orc, x, *p1, fast=False), *p2, fast=False)
    err = rel_norm_err(got, ref)
    print(f"[err] two layers at T=750 against the f32 reference: {err:.3e}", flush=True)
    assert err <= 1e-3


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
