"""Granite Speech's encoder block and self-conditioning on the device (telmo_amd.granite:
Granite::block_span, src/granite.rs:800-952, and Granite::self_conditioning, src/granite.rs:1040-1069)
against the same sequence composed from the oracle's functions (tests/layer_oracle.py), on an MI355X.

* Bit for bit against the composition with the integer oracle, and within 1e-3 row-normwise of the
  composition with the reference's fused f32 products.
* Granite's shapes (src/granite.rs:1153-1170): d 1024, feed-forward 4096, 2048 convolution channels,
  kernel 7, vocabulary 16384. A strided block at T0 = 4 T input frames, a stack of the two strided
  blocks, a plain block and the self-conditioning (T0 = 1000 -> 250), batches of utterances, an odd
  frame count.
* The row kernels the block adds: softmax (src/kernels/avx512.rs:382-407) bit for bit against the
  oracle on rows of 1 to 20000 values, and the strided block's pooling.
"""
import numpy as np
import pytest

import bench
import layer_oracle
from helpers import rel_norm_err

pytestmark = pytest.mark.gpu

D = bench.G_D


def say(*args):
    print("[case]", *args, flush=True)


def run_blocks(tk, blocks, x, utterances, selfcond=None, paired=False):
    """The device blocks in order over x (numpy [t, d]); selfcond = (head, head_b, mid, mid_b) host
    parameters applied after the last block. paired: each block boundary's two LayerNorms in one
    launch (forward's prepared and next_norm). Returns the output rows."""
    import torch

    from telmo_amd.granite import GraniteBlock, self_conditioning

    t = x.shape[0]
    blk = GraniteBlock(tk, D, bench.G_FF, bench.G_CC, bench.G_KERNEL, t)
    cur = torch.from_numpy(x.copy()).cuda()
    n = t
    ws = [bench.upload_granite_block(tk, params) for params in blocks]
    if paired and ws:
        blk.prepare(cur, n, ws[0])
    for i, w in enumerate(ws):
        nxt = ws[i + 1].norms["ff1_norm"] if paired and i + 1 < len(ws) else None
        y, n = blk.forward(cur, n, w, utterances=utterances, prepared=paired, next_norm=nxt)
        cur = y
    if selfcond is not None:
        import telmo_amd

        head, head_b, mid, mid_b = selfcond
        H = telmo_amd.PackedWeights.from_parts(tk, head[2], head[3], telmo_amd.Precision.INT8, head[0], head[1])
        M = telmo_amd.PackedWeights.from_parts(tk, mid[2], mid[3], telmo_amd.Precision.INT8, mid[0], mid[1])
        logits = torch.empty(n * head[2], dtype=torch.float32, device="cuda")
        self_conditioning(tk, cur, n, H, torch.from_numpy(head_b).cuda(), M, torch.from_numpy(mid_b).cuda(), logits)
        tk.synchronize()
        H.close()
        M.close()
    tk.synchronize()
    for w in ws:
        for m in w.mats.values():
            m.close()
    return cur[:n].cpu().numpy()


def oracle_blocks(orc, blocks, x, utterances, fast, selfcond=None):
    for mats, biases, norms, dw_w, dw_b, strided in blocks:
        x = layer_oracle.oracle_granite_block(orc, x, mats, biases, norms, dw_w, dw_b, strided, utterances, fast)
    if selfcond is not None:
        x = layer_oracle.oracle_self_conditioning(orc, x, *selfcond, fast=fast)
    return x


def check(orc, got, blocks, x, utterances, what, selfcond=None):
    want = oracle_blocks(orc, blocks, x, utterances, True, selfcond)
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), what
    ref = oracle_blocks(orc, blocks, x, utterances, False, selfcond)
    err = rel_norm_err(got, ref)
    print(f"[err] {what} against the f32 reference: {err:.3e}", flush=True)
    assert err <= 1e-3


@pytest.mark.parametrize("frames,utterances", [(1000, 1), (500, 2), (333, 3)])
def test_strided_block(tk, orc, frames, utterances):
    p = bench.granite_block_params(1100, True)
    x = bench.synth_normal((frames * utterances, D), 11)
    say("granite strided block", frames, utterances)
    got = run_blocks(tk, [p], x, utterances)
    assert got.shape[0] == utterances * (frames // 2)
    check(orc, got, [p], x, utterances, f"strided block, {utterances} x {frames} frames")


@pytest.mark.parametrize("frames,utterances", [(250, 1), (125, 4)])
def test_plain_block(tk, orc, frames, utterances):
    p = bench.granite_block_params(1300, False)
    x = bench.synth_normal((frames * utterances, D), 12)
    say("granite block", frames, utterances)
    got = run_blocks(tk, [p], x, utterances)
    check(orc, got, [p], x, utterances, f"block, {utterances} x {frames} frames")


def test_block_boundaries_in_one_launch(tk):
    """Two strided blocks and a plain one with each boundary's norm_out and the next block's ff1
    LayerNorm in one launch, the first block's taken by prepare: the bits of the blocks run one
    LayerNorm at a time (which the oracle tests pin), over 2 x 500 frames."""
    blocks = [bench.granite_block_params(1700, True), bench.granite_block_params(1800, True),
              bench.granite_block_params(1900, False)]
    x = bench.synth_normal((1000, D), 15)
    say("granite paired boundaries", 1000)
    want = run_blocks(tk, blocks, x, 2)
    got = run_blocks(tk, blocks, x, 2, paired=True)
    assert got.shape == want.shape == (250, D)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_self_conditioning(tk, orc):
    h = bench.granite_head_params(1500)
    x = bench.synth_normal((250, D), 13)
    say("granite self-conditioning", 250)
    got = run_blocks(tk, [], x, 1, selfcond=h)
    check(orc, got, [], x, 1, "self-conditioning at 250 frames", selfcond=h)


def test_encoder_start_at_four_times_the_frames(tk, orc):
    """The encoder's first two strided blocks, a plain block and the self-conditioning after it, as
    Granite::encode runs them (src/granite.rs:628-650): T0 = 1000 input frames, T = 250 out. Bit for
    bit against the integer oracle's chain; each stage within 1e-3 of the fused f32 reference on the
    same input rows (the contract of a product). The chain's end-to-end distance from the f32
    reference is printed: the softmax of the self-conditioning multiplies its input's differences
    (its logits have a spread of about 14), so it is not a per-stage bound."""
    blocks = [bench.granite_block_params(1700, True), bench.granite_block_params(1800, True),
              bench.granite_block_params(1900, False)]
    h = bench.granite_head_params(2000)
    x = bench.synth_normal((1000, D), 14)
    say("granite encoder start", 1000)
    got = run_blocks(tk, blocks, x, 1, selfcond=h)
    assert got.shape == (250, D)
    stage_in = x
    for i, p in enumerate(blocks):
        fast = layer_oracle.oracle_granite_block(orc, stage_in, *p[:5], p[5], 1, True)
        ref = layer_oracle.oracle_granite_block(orc, stage_in, *p[:5], p[5], 1, False)
        err = rel_norm_err(fast, ref)
        print(f"[err] block {i} of the chain against the f32 reference on its input: {err:.3e}", flush=True)
        assert err <= 1e-3
        stage_in = fast
    fast = layer_oracle.oracle_self_conditioning(orc, stage_in, *h, fast=True)
    ref = layer_oracle.oracle_self_conditioning(orc, stage_in, *h, fast=False)
    err = rel_norm_err(fast, ref)
    print(f"[err] self-conditioning of the chain against the f32 reference on its input: {err:.3e}", flush=True)
    assert err <= 1e-3
    assert np.array_equal(got.view(np.uint32), fast.view(np.uint32))
    end = rel_norm_err(got, oracle_blocks(orc, blocks, x, 1, False, h))
    print(f"[err] the chain end to end against the f32 reference chain: {end:.3e}", flush=True)


# Row lengths for each register-held instance (up to 1024, 4096, 8192, 16384 values, 16384 itself
# without masks) and the chunked kernel beyond.
@pytest.mark.parametrize("n", [1, 3, 16, 17, 1030, 4096, 4097, 6000, 12345, 16384, 20000])
def test_softmax_matches_the_oracle(tk, orc, n):
    import torch

    rows = 7
    x = (bench.synth_normal((rows, n), 40 + n) * np.float32(8.0)).astype(np.float32)
    x[1] = -np.inf
    x[2] = np.float32(3.0)
    if n > 4:
        x[3, 3] = np.inf
        x[4, :] = -1000.0
        x[4, n // 2] = 5.0
        x[5, n // 3] = np.nan  # the reference's lane order for the maximum (NaN rows: see the oracle)
    xd = torch.from_numpy(x.copy()).cuda()
    say("softmax", rows, n)
    tk.softmax_device(xd, n, rows, n)
    tk.synchronize()
    got = xd.cpu().numpy()
    want = orc.softmax(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), n


def test_softmax_of_the_self_conditioning_shape(tk, orc):
    """750 rows of 16384 (60 s of Granite's frames over the CTC vocabulary), more rows than CUs."""
    import torch

    x = (bench.synth_normal((750, 16384), 47) * np.float32(6.0)).astype(np.float32)
    xd = torch.from_numpy(x.copy()).cuda()
    say("softmax", 750, 16384)
    tk.softmax_device(xd, 16384, 750, 16384)
    tk.synchronize()
    assert np.array_equal(xd.cpu().numpy().view(np.uint32), orc.softmax(x).view(np.uint32))


def test_softmax_strided_rows_and_refusals(tk, orc):
    import torch

    import telmo_amd

    x = bench.synth_normal((5, 300), 50) * np.float32(4.0)
    xd = torch.from_numpy(x.copy()).cuda()
    tk.softmax_device(xd, 300, 5, 257)
    tk.synchronize()
    got = xd.cpu().numpy()
    want = x.copy()
    want[:, :257] = orc.softmax(x[:, :257])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    with pytest.raises(telmo_amd.TelmoError):
        tk.softmax_device(xd, 256, 5, 257)  # ldx < n
    with pytest.raises(telmo_amd.TelmoError):
        tk.softmax_device(xd, 300, 6, 257)  # past the buffer


def test_average_pairs(tk):
    import torch

    import telmo_amd

    x = bench.synth_normal((2 * 7, 40), 60)
    xd = torch.from_numpy(x).cuda()
    out = torch.full((6, 40), -1.0, device="cuda")
    tk.average_pairs_device(xd, 40, 7, 40, out, 40, batch=2)  # 7 frames: 3 rows each, the last dropped
    tk.synchronize()
    want = np.concatenate([(x[s * 7:s * 7 + 6:2] + x[s * 7 + 1:s * 7 + 6:2]) / np.float32(2.0) for s in (0, 1)])
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.astype(np.float32).view(np.uint32))
    with pytest.raises(telmo_amd.TelmoError):
        tk.average_pairs_device(xd, 40, 7, 40, xd, 40, batch=1)  # out overlaps x
    with pytest.raises(telmo_amd.TelmoError):
        tk.average_pairs_device(xd, 40, 8, 40, out, 40, batch=2)  # 16 input rows of 14
