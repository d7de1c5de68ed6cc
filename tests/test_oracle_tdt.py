"""The oracle's TDT decoder: predict_rows (src/parakeet.rs:1524-1577) and decode_inner (1412-1513).

The reference pins these only through model goldens (tests/goldens, real checkpoints). Here:
- predict_rows against an f64 numpy restatement on dequantised weights (which gate is which, the
  [x; h] order, the embedding row and the [h, c] state layout), within the fast path's error;
- a zero-weight network, whose gates are exactly the biases, against the closed-form cell update;
- decode_inner's control flow on a zero joint, whose logits are exactly the joint bias: blank runs
  moving max(duration, 1) frames, tokens of duration 0 up to max_symbols per frame, tokens moving
  by their duration, a start part-way through a frame, the first-largest tie rule and a NaN first
  logit (never beaten), all against token lists written out by hand.
"""
import numpy as np
import pytest

from helpers import tdt_network


def dequant(values, scales, n, k):
    panels = -(-n // 16)
    q = values.view(np.int8).reshape(panels, k, 16).transpose(0, 2, 1).reshape(panels * 16, k)[:n]
    return q.astype(np.float64) * scales[:n, None].astype(np.float64)


def predict_f64(net, tokens, states, preds):
    h, L = net["h"], len(net["lstm"])
    sig = lambda x: 1.0 / (1.0 + np.exp(-x))
    states = states.astype(np.float64).copy()
    out = np.zeros((len(tokens), h))
    for r, tok in enumerate(tokens):
        x = net["emb"][tok].astype(np.float64)
        for l in range(L):
            W = dequant(*net["lstm"][l], 4 * h, 2 * h)
            hs, cs = states[r, l * 2 * h:l * 2 * h + h], states[r, l * 2 * h + h:(l + 1) * 2 * h]
            g = W @ np.concatenate([x, hs]) + net["lstm_b"][l]
            i, f, gg, o = sig(g[:h]), sig(g[h:2 * h]), np.tanh(g[2 * h:3 * h]), sig(g[3 * h:])
            c = f * cs + i * gg
            hn = o * np.tanh(c)
            states[r, l * 2 * h:l * 2 * h + h], states[r, l * 2 * h + h:(l + 1) * 2 * h] = hn, c
            x = hn
        out[r] = dequant(*net["proj"], h, h) @ x + net["proj_b"]
    return states, out


@pytest.mark.parametrize("layers,rows", [(1, 1), (2, 3), (2, 16)])
def test_predict_rows_matches_an_f64_restatement(orc, layers, rows):
    rng = np.random.default_rng(layers * 10 + rows)
    net = tdt_network(rng, 64, 50, [0, 1, 2], layers=layers)
    tokens = rng.integers(0, 50, size=rows)
    states = (0.5 * rng.standard_normal((rows, layers * 2 * 64))).astype(np.float32)
    preds = np.zeros((rows, 64), np.float32)
    want_states, want_preds = predict_f64(net, tokens, states, preds)
    orc.tdt_predict(net, tokens, states, preds)
    assert np.max(np.abs(states - want_states)) < 2e-4
    assert np.max(np.abs(preds - want_preds)) < 2e-4


def test_zero_weights_give_the_closed_form_cell(orc):
    rng = np.random.default_rng(4)
    h = 32
    net = tdt_network(rng, h, 10, [0, 1], layers=1)
    net["lstm"] = [(np.zeros_like(net["lstm"][0][0]), net["lstm"][0][1])]
    states = (0.5 * rng.standard_normal((1, 2 * h))).astype(np.float32)
    c0 = states[0, h:].astype(np.float64)
    b = net["lstm_b"][0].astype(np.float64)
    sig = lambda x: 1.0 / (1.0 + np.exp(-x))
    c = sig(b[h:2 * h]) * c0 + sig(b[:h]) * np.tanh(b[2 * h:3 * h])
    hn = sig(b[3 * h:]) * np.tanh(c)
    orc.tdt_predict(net, [3], states, np.zeros((1, h), np.float32))
    assert np.max(np.abs(states[0, h:] - c)) < 1e-6
    assert np.max(np.abs(states[0, :h] - hn)) < 1e-6


def zero_joint(net, bias):
    net = dict(net)
    net["joint"] = (np.zeros_like(net["joint"][0]), net["joint"][1])
    net["joint_b"] = np.asarray(bias, np.float32)
    return net


def joint_bias(vocab, ndur, token, dur_index):
    b = np.zeros(vocab + ndur, np.float32)
    b[token] = 5.0
    b[vocab + dur_index] = 5.0
    return b


@pytest.fixture(scope="module")
def small():
    return tdt_network(np.random.default_rng(7), 32, 20, [0, 1, 2, 3, 4], layers=2, max_symbols=3)


def decode(orc, net, frames, frame=0, on_frame=0):
    rng = np.random.default_rng(frames)
    enc = rng.standard_normal((frames, net["h"])).astype(np.float32)
    state = np.zeros(len(net["lstm"]) * 2 * net["h"], np.float32)
    pred = np.zeros(net["h"], np.float32)
    return orc.tdt_decode(net, enc, state, pred, frame, on_frame)


@pytest.mark.parametrize("dur_index,step", [(0, 1), (1, 1), (3, 3), (4, 4)])
def test_blank_runs_move_max_duration_1(orc, small, dur_index, step):
    net = zero_joint(small, joint_bias(20, 5, 19, dur_index))
    toks, frame, on = decode(orc, net, 23)
    assert toks == [] and on == 0
    assert frame == -(-23 // step) * step


def test_duration_0_tokens_stop_at_max_symbols(orc, small):
    net = zero_joint(small, joint_bias(20, 5, 7, 0))
    toks, frame, on = decode(orc, net, 6)
    assert toks == [(7, t, 0) for t in range(6) for _ in range(3)]
    assert (frame, on) == (6, 0)


def test_tokens_move_by_their_duration(orc, small):
    net = zero_joint(small, joint_bias(20, 5, 11, 2))
    toks, frame, on = decode(orc, net, 9)
    assert toks == [(11, t, 2) for t in range(0, 9, 2)]
    assert (frame, on) == (10, 0)


def test_a_start_part_way_through_a_frame(orc, small):
    net = zero_joint(small, joint_bias(20, 5, 4, 0))
    toks, frame, on = decode(orc, net, 3, frame=1, on_frame=2)
    assert toks == [(4, 1, 0), (4, 2, 0), (4, 2, 0), (4, 2, 0)]
    assert (frame, on) == (3, 0)


def test_ties_go_to_the_first_and_a_nan_first_logit_wins(orc, small):
    b = joint_bias(20, 5, 9, 2)
    b[6] = b[9]  # a tie: the first of the two
    b[20 + 4] = b[20 + 2]  # a duration tie: index 2 stays
    toks, _, _ = decode(orc, zero_joint(small, b), 4)
    assert toks == [(6, 0, 2), (6, 2, 2)]
    b = joint_bias(20, 5, 9, 1)
    b[0] = np.nan  # nothing is larger than a NaN at index 0 in the reference's scan
    toks, _, _ = decode(orc, zero_joint(small, b), 2)
    assert toks == [(0, 0, 1), (0, 1, 1)]


def test_a_start_past_the_frames_does_nothing(orc, small):
    toks, frame, on = decode(orc, small, 5, frame=5, on_frame=1)
    assert toks == [] and (frame, on) == (5, 1)


def test_random_networks_emit_and_skip(orc):
    """Sanity of the random decode the GPU tests compare against: both branches are taken."""
    rng = np.random.default_rng(3)
    net = tdt_network(rng, 64, 100, [0, 1, 2, 3, 4], blank_bias=3.0)
    toks, frame, _ = decode(orc, net, 60)
    assert len(toks) > 5 and frame >= 60
    assert len({f for _, f, _ in toks}) < 60  # some frames were skipped by blanks or durations
    assert all(0 <= t < 99 for t, _, _ in toks)
