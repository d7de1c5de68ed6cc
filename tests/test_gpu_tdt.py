"""Parity of the device TDT decoder (tg_tdt_predict_device, tg_tdt_decode_device) with the oracle's
predict_rows and decode_inner, through the C ABI, on an MI355X.

The GEMVs are the fast path's, bit-identical to the integer oracle for the same inputs. The gate
math uses the GPU's expf / tanhf where the oracle (like the reference) uses the host libm, so a
gate output can differ by an ulp. That can move a rounding of the next product's two-digit input by
one unit (1/32639 of the row's largest |value|), a step of about |q| s / 32639 in each output it
feeds (1e-6 to 1e-5 here). States and predictions are therefore held to the fast path's own bound,
1e-4 (absolute for states, row-normwise for predictions; the parity bound for f32 outputs is 1e-3), and the
emitted tokens, frames and durations must be identical.
"""
import numpy as np
import pytest

from helpers import INT8_P, Q8_0_P, rel_norm_err, tdt_network

pytestmark = pytest.mark.gpu

TOL = 1e-4


def say(*args):
    print("[case]", *args, flush=True)


def upload(tk, net, durations=None):
    import torch

    import telmo_amd

    P = telmo_amd.Precision(net["p"])
    h, vocab, nd = net["h"], net["vocab"], len(net["durations"])
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    joint = telmo_amd.PackedWeights.from_parts(tk, vocab + nd, h, P, *net["joint"])
    lstm = [telmo_amd.PackedWeights.from_parts(tk, 4 * h, 2 * h, P, *w) for w in net["lstm"]]
    proj = telmo_amd.PackedWeights.from_parts(tk, h, h, P, *net["proj"])
    durations = net["durations"] if durations is None else durations
    return telmo_amd.TdtDecoder(tk, h, vocab, durations, net["max_symbols"], joint, dev(net["joint_b"]),
                                dev(net["emb"]), lstm, [dev(b) for b in net["lstm_b"]], proj, dev(net["proj_b"]))


@pytest.mark.parametrize("p,rows", [(INT8_P, 1), (INT8_P, 4), (INT8_P, 16), (Q8_0_P, 1), (Q8_0_P, 16)])
def test_predict_rows_matches_the_oracle(tk, orc, p, rows):
    import torch

    rng = np.random.default_rng(100 + rows + p)
    net = tdt_network(rng, 640, 1025, [0, 1, 2, 3, 4], layers=2, precision=p)
    dec = upload(tk, net)
    assert dec.max_rows() == 16
    tokens = rng.integers(0, 1025, size=rows)
    states = (0.5 * rng.standard_normal((rows, 2 * 2 * 640))).astype(np.float32)
    preds = np.zeros((rows, 640), np.float32)
    say("predict", p, rows)
    sd, pd = torch.from_numpy(states.copy()).cuda(), torch.zeros((rows, 640), device="cuda")
    dec.predict_rows(list(tokens), sd, pd)
    tk.synchronize()
    orc.tdt_predict(net, tokens, states, preds)
    assert np.max(np.abs(sd.cpu().numpy() - states)) <= TOL
    assert rel_norm_err(pd.cpu().numpy(), preds) <= TOL
    dec.close()


DECODE_CASES = [  # h, vocab, durations, layers, precision, frames, blank_bias, max_symbols
    (64, 100, [0, 1, 2, 3, 4], 2, INT8_P, 60, 3.0, 10),
    (64, 100, [0, 1, 2, 3, 4], 2, INT8_P, 200, 6.0, 3),
    (128, 300, [0, 2, 4], 1, INT8_P, 77, 4.0, 2),
    (64, 100, [1, 2], 3, Q8_0_P, 50, 2.0, 5),
    (640, 8193, [0, 1, 2, 3, 4], 2, INT8_P, 120, 6.0, 10),
    (640, 8193, [0, 1, 2, 3, 4], 2, Q8_0_P, 60, 6.0, 10),
]


@pytest.mark.parametrize("resident", [True, False], ids=["resident", "steps"])
@pytest.mark.parametrize("case", DECODE_CASES)
def test_decode_matches_the_oracle(tk, orc, case, resident):
    """Both ways of running the steps: resident and the graph of step kernels, int8 and Q8_0."""
    import torch

    h, vocab, durs, layers, p, frames, blank_bias, ms = case
    rng = np.random.default_rng(frames + h + layers)
    net = tdt_network(rng, h, vocab, durs, layers=layers, precision=p, max_symbols=ms, blank_bias=blank_bias)
    dec = upload(tk, net)
    # networks run resident unless told otherwise
    assert dec.resident
    dec.set_resident(resident)
    assert dec.resident == resident
    enc = rng.standard_normal((frames, h)).astype(np.float32)
    state = (0.3 * rng.standard_normal(layers * 2 * h)).astype(np.float32)
    pred = (0.3 * rng.standard_normal(h)).astype(np.float32)
    sd, pdv = torch.from_numpy(state.copy()).cuda(), torch.from_numpy(pred.copy()).cuda()
    say("decode", case, "resident" if resident else "steps")
    toks, frame, on = dec.decode(torch.from_numpy(enc).cuda(), sd, pdv)
    assert dec.last_resident == resident
    want, wframe, won = orc.tdt_decode(net, enc, state, pred)
    assert [tuple(t) for t in toks] == want
    assert (frame, on) == (wframe, won)
    assert np.max(np.abs(sd.cpu().numpy() - state)) <= TOL
    assert rel_norm_err(pdv.cpu().numpy()[None], pred[None]) <= TOL
    dec.close()


def test_decode_known_answers(tk, orc):
    """Zero joints, so the logits are the bias: blank runs, duration-0 tokens up to max_symbols, a
    start part-way through a frame, ties and a NaN first logit, as the oracle's pinned cases."""
    import torch

    rng = np.random.default_rng(7)
    base = tdt_network(rng, 32, 20, [0, 1, 2, 3, 4], layers=2, max_symbols=3)
    enc = torch.from_numpy(rng.standard_normal((23, 32)).astype(np.float32)).cuda()

    def run(bias, frames, frame=0, on_frame=0):
        net = dict(base)
        net["joint"] = (np.zeros_like(base["joint"][0]), base["joint"][1])
        net["joint_b"] = np.asarray(bias, np.float32)
        dec = upload(tk, net)
        state = torch.zeros(2 * 2 * 32, device="cuda")
        pred = torch.zeros(32, device="cuda")
        out = dec.decode(enc[:frames], state, pred, frame, on_frame)
        dec.close()
        return out

    def bias(token, d):
        b = np.zeros(25, np.float32)
        b[token] = 5.0
        b[20 + d] = 5.0
        return b

    say("decode known answers")
    assert run(bias(19, 3), 23) == ([], 24, 0)
    assert run(bias(19, 0), 23) == ([], 23, 0)
    assert [tuple(t) for t in run(bias(7, 0), 6)[0]] == [(7, t, 0) for t in range(6) for _ in range(3)]
    assert [tuple(t) for t in run(bias(11, 2), 9)[0]] == [(11, t, 2) for t in range(0, 9, 2)]
    toks, frame, on = run(bias(4, 0), 3, frame=1, on_frame=2)
    assert [tuple(t) for t in toks] == [(4, 1, 0), (4, 2, 0), (4, 2, 0), (4, 2, 0)] and (frame, on) == (3, 0)
    b = bias(9, 2)
    b[6] = b[9]
    b[24] = b[22]
    assert [tuple(t) for t in run(b, 4)[0]] == [(6, 0, 2), (6, 2, 2)]
    b = bias(9, 1)
    b[0] = np.nan
    assert [tuple(t) for t in run(b, 2)[0]] == [(0, 0, 1), (0, 1, 1)]
    assert run(bias(7, 0), 5, frame=5, on_frame=1) == ([], 5, 1)


def test_decode_refusals(tk):
    import torch

    import telmo_amd

    rng = np.random.default_rng(8)
    net = tdt_network(rng, 32, 20, [0, 1, 2], layers=1, max_symbols=2)
    with pytest.raises(telmo_amd.TelmoError):  # the joint has 23 outputs, 20 tokens + 2 durations need 22
        upload(tk, net, durations=[0, 1])
    with pytest.raises(telmo_amd.TelmoError):  # a negative duration
        upload(tk, net, durations=[0, -1, 2])
    dec = upload(tk, net)
    with pytest.raises(telmo_amd.TelmoError):
        dec.predict_rows([20], torch.zeros((1, 64), device="cuda"), torch.zeros((1, 32), device="cuda"))
    with pytest.raises(telmo_amd.TelmoError):
        dec.predict_rows([0] * 17, torch.zeros((17, 64), device="cuda"), torch.zeros((17, 32), device="cuda"))
    b = np.zeros(23, np.float32)
    b[5] = b[20] = 5.0  # token 5, duration 0: two tokens per frame
    net2 = dict(net)
    net2["joint"] = (np.zeros_like(net["joint"][0]), net["joint"][1])
    net2["joint_b"] = b
    dec2 = upload(tk, net2)
    enc = torch.zeros((4, 32), device="cuda")
    with pytest.raises(telmo_amd.TelmoError):  # 8 tokens, room for 3
        dec2.decode(enc, torch.zeros(64, device="cuda"), torch.zeros(32, device="cuda"), cap=3)
    dec.close()
    dec2.close()



def test_decode_fixture(tk):
    """The committed TDT fixture (a small int8 network from telmo's generator): predict_rows and the
    decode from the start state; tokens exact, states within TOL."""
    import torch

    from golden_cases import load, rows, tdt_net

    meta = [r for r in rows() if r["kind"] == "tdt"][0]
    g = load(meta)
    net = tdt_net(meta, g)
    dec = upload(tk, net)
    say("tdt fixture", meta["name"])
    sd = torch.from_numpy(g["states0"].copy()).cuda()
    pd = torch.zeros(g["preds"].shape, device="cuda")
    dec.predict_rows(list(g["tokens_in"]), sd, pd)
    tk.synchronize()
    assert np.max(np.abs(sd.cpu().numpy() - g["states"])) <= TOL
    assert rel_norm_err(pd.cpu().numpy(), g["preds"]) <= TOL
    state, pred = torch.from_numpy(g["state0"].copy()).cuda(), torch.from_numpy(g["pred0"].copy()).cuda()
    toks, frame, on = dec.decode(torch.from_numpy(g["enc"]).cuda(), state, pred)
    assert np.array_equal(np.asarray([tuple(t) for t in toks], np.int32).reshape(-1, 3), g["tokens"])
    assert [frame, on] == list(g["end"])
    assert np.max(np.abs(state.cpu().numpy() - g["state"])) <= TOL
    dec.close()


def zero_joint_network(rng, token, duration, h=32, vocab=20, durs=(0, 1, 2, 3, 4), max_symbols=3):
    """A network whose joint weights are zero, so every logit is its bias: the decode emits `token`
    with `duration` at every step (the closed form of decode_inner's loop)."""
    net = tdt_network(rng, h, vocab, list(durs), layers=2, max_symbols=max_symbols)
    net["joint"] = (np.zeros_like(net["joint"][0]), net["joint"][1])
    b = np.zeros(vocab + len(durs), np.float32)
    b[token] = 5.0
    b[vocab + list(durs).index(duration)] = 5.0
    net["joint_b"] = b
    return net


def test_resident_decode_crosses_the_relaunch_boundary(tk):
    """More steps than one resident launch makes (16384): 6000 frames of three duration-0 tokens each
    are 18000 steps, so the host relaunches from the control block once; tokens are the closed form,
    and state and prediction equal the step kernels' run of the same decode."""
    import torch

    rng = np.random.default_rng(11)
    net = zero_joint_network(rng, 7, 0)
    frames = 6000
    enc = torch.from_numpy(rng.standard_normal((frames, 32)).astype(np.float32)).cuda()
    dec = upload(tk, net)
    results = []
    for resident in (True, False):
        dec.set_resident(resident)
        state, pred = torch.zeros(2 * 2 * 32, device="cuda"), torch.zeros(32, device="cuda")
        say("decode across the relaunch boundary", "resident" if resident else "steps")
        toks, frame, on = dec.decode(enc, state, pred)
        assert dec.last_resident == resident
        assert [tuple(t) for t in toks] == [(7, t, 0) for t in range(frames) for _ in range(3)]
        assert (frame, on) == (frames, 0)
        results.append((state.cpu().numpy(), pred.cpu().numpy()))
    assert np.max(np.abs(results[0][0] - results[1][0])) <= TOL
    assert np.max(np.abs(results[0][1] - results[1][1])) <= TOL
    dec.close()


@pytest.mark.parametrize("steps", [1, 3, 16])
def test_resident_decode_relaunches_every_few_steps(tk, orc, steps):
    """The same decodes with a relaunch every `steps` steps: every launch resumes from the control
    block, the hand-over words and the state the previous one wrote back; the oracle's tokens."""
    import torch

    for case in (DECODE_CASES[0], DECODE_CASES[2]):
        h, vocab, durs, layers, p, frames, blank_bias, ms = case
        rng = np.random.default_rng(frames + h + layers)
        net = tdt_network(rng, h, vocab, durs, layers=layers, precision=p, max_symbols=ms, blank_bias=blank_bias)
        dec = upload(tk, net)
        dec.set_resident_limits(steps_per_launch=steps)
        enc = rng.standard_normal((frames, h)).astype(np.float32)
        state = (0.3 * rng.standard_normal(layers * 2 * h)).astype(np.float32)
        pred = (0.3 * rng.standard_normal(h)).astype(np.float32)
        sd, pdv = torch.from_numpy(state.copy()).cuda(), torch.from_numpy(pred.copy()).cuda()
        say("decode relaunching every", steps, "steps", case)
        toks, frame, on = dec.decode(torch.from_numpy(enc).cuda(), sd, pdv)
        assert dec.last_resident
        want, wframe, won = orc.tdt_decode(net, enc, state, pred)
        assert [tuple(t) for t in toks] == want
        assert (frame, on) == (wframe, won)
        assert np.max(np.abs(sd.cpu().numpy() - state)) <= TOL
        assert rel_norm_err(pdv.cpu().numpy()[None], pred[None]) <= TOL
        dec.close()


def test_resident_decode_past_its_deadline_leaves_the_state_as_passed(tk, orc):
    """A one-microsecond limit on every wait between workgroups (forced from the host; every wait
    still ends, at its deadline): the decode fails with an error, and state and prediction are the
    caller's values, not a mix of the steps the workgroups had reached. With the default limit the
    same call then gives the oracle's decode."""
    import torch

    import telmo_amd

    h, vocab, durs, layers, p, frames, blank_bias, ms = DECODE_CASES[0]
    rng = np.random.default_rng(frames + h + layers)
    net = tdt_network(rng, h, vocab, durs, layers=layers, precision=p, max_symbols=ms, blank_bias=blank_bias)
    dec = upload(tk, net)
    enc = rng.standard_normal((frames, h)).astype(np.float32)
    state = (0.3 * rng.standard_normal(layers * 2 * h)).astype(np.float32)
    pred = (0.3 * rng.standard_normal(h)).astype(np.float32)
    encd = torch.from_numpy(enc).cuda()
    sd, pdv = torch.from_numpy(state.copy()).cuda(), torch.from_numpy(pred.copy()).cuda()
    dec.set_resident_limits(wait_us=1)
    say("resident decode with a 1 us wait limit")
    with pytest.raises(telmo_amd.TelmoError):
        dec.decode(encd, sd, pdv)
    tk.synchronize()
    assert np.array_equal(sd.cpu().numpy(), state)
    assert np.array_equal(pdv.cpu().numpy(), pred)
    dec.set_resident_limits()
    say("the same decode with the default limits")
    toks, frame, on = dec.decode(encd, sd, pdv)
    assert dec.last_resident
    want, wframe, won = orc.tdt_decode(net, enc, state, pred)
    assert [tuple(t) for t in toks] == want
    assert (frame, on) == (wframe, won)
    assert np.max(np.abs(sd.cpu().numpy() - state)) <= TOL
    dec.close()


def test_concurrent_decodes_on_two_contexts_share_the_device(orc, gpu_stream):
    """Two threads, each with its own context, stream and network, decode at the same time, five
    times each: one resident decode holds the device at a time, the other runs on the step kernels,
    and every decode equals the oracle's. The threads touch only their own streams (no device-wide
    synchronisation), so their decodes overlap."""
    import threading

    import torch

    import telmo_amd

    h, vocab, durs, layers, p, frames, blank_bias, ms = DECODE_CASES[4]
    reps = 5
    cases = []
    for i in range(2):
        rng = np.random.default_rng(300 + i)
        net = tdt_network(rng, h, vocab, durs, layers=layers, precision=p, max_symbols=ms, blank_bias=blank_bias)
        enc = rng.standard_normal((frames, h)).astype(np.float32)
        state = (0.3 * rng.standard_normal(layers * 2 * h)).astype(np.float32)
        pred = (0.3 * rng.standard_normal(h)).astype(np.float32)
        ws, wp = state.copy(), pred.copy()
        want = orc.tdt_decode(net, enc, ws, wp)
        cases.append((net, enc, state, pred, want, ws))
    kerns = [telmo_amd.Kernels(0) for _ in range(2)]
    decs = [upload(k, c[0]) for k, c in zip(kerns, cases)]
    encs = [torch.from_numpy(c[1]).cuda() for c in cases]
    ins = [[(torch.from_numpy(c[2].copy()).cuda(), torch.from_numpy(c[3].copy()).cuda()) for _ in range(reps)]
           for c in cases]
    torch.cuda.synchronize()
    start = threading.Barrier(2)
    results = [[], []]
    errors = []

    def run(i):
        try:
            start.wait()
            for r in range(reps):
                sd, pdv = ins[i][r]
                toks, frame, on = decs[i].decode(encs[i], sd, pdv)
                results[i].append(([tuple(t) for t in toks], frame, on, decs[i].last_resident))
            kerns[i].synchronize()
        except Exception as e:  # reported by the main thread
            errors.append(e)

    say("two concurrent decodes")
    threads = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads)
    assert not errors, errors
    torch.cuda.synchronize()
    for i in range(2):
        want, wframe, won = cases[i][4]
        assert len(results[i]) == reps
        for r, (toks, frame, on, _) in enumerate(results[i]):
            assert toks == want and (frame, on) == (wframe, won)
            assert np.max(np.abs(ins[i][r][0].cpu().numpy() - cases[i][5])) <= TOL
    ran = [r[3] for i in range(2) for r in results[i]]
    print("[case] resident decodes:", sum(ran), "of", len(ran), flush=True)
    for d in decs:
        d.close()
    for k in kerns:
        k.close()


MULTI_CASES = [  # h, vocab, durations, layers, streams, frames per stream, blank_bias, max_symbols
    (64, 100, [0, 1, 2, 3, 4], 2, 2, [60, 45], 3.0, 10),
    (64, 100, [0, 1, 2, 3, 4], 2, 4, [60, 7, 33, 60], 6.0, 3),
    (128, 300, [0, 2, 4], 1, 8, [77, 20, 77, 1, 50, 64, 9, 70], 4.0, 2),
    (640, 8193, [0, 1, 2, 3, 4], 2, 8, [120, 90, 120, 60, 100, 120, 75, 110], 6.0, 10),
]


@pytest.mark.parametrize("case", MULTI_CASES)
def test_multi_stream_decode_matches_each_stream(tk, orc, case):
    """Several streams in one resident launch (tg_tdt_decode_streams_device). Each stream's tokens,
    frame, on_frame, state and prediction equal, bit for bit, the single-stream resident decode of
    that stream alone, and its tokens equal the oracle's decode of it. In the case of Parakeet's
    shapes, with eight streams of 60 to 120 frames, one stream meets a near tie: there the single-stream
    decode and the oracle part ways. The device's expf / tanhf and the host's libm differ by an ulp in
    a gate, as the module docstring describes, so the multi-stream decode follows the single-stream
    one. That case asserts the oracle's tokens for all streams but at most one."""
    import torch

    h, vocab, durs, layers, m, frames, blank_bias, ms = case
    rng = np.random.default_rng(300 + h + m)
    net = tdt_network(rng, h, vocab, durs, layers=layers, max_symbols=ms, blank_bias=blank_bias)
    dec = upload(tk, net)
    encs = [rng.standard_normal((f, h)).astype(np.float32) for f in frames]
    states = [(0.3 * rng.standard_normal(layers * 2 * h)).astype(np.float32) for _ in range(m)]
    preds = [(0.3 * rng.standard_normal(h)).astype(np.float32) for _ in range(m)]
    dev = lambda a: torch.from_numpy(a.copy()).cuda()  # noqa: E731
    sd, pd = [dev(s) for s in states], [dev(p) for p in preds]
    say("multi-stream decode", case)
    got = dec.decode_streams([dev(e) for e in encs], sd, pd)
    assert dec.last_resident == 2
    steps_multi = dec.last_steps
    apart = []
    for q in range(m):
        toks, frame, on = got[q]
        s1, p1 = dev(states[q]), dev(preds[q])
        t1, f1, o1 = dec.decode(dev(encs[q]), s1, p1)
        assert dec.last_resident == 1
        assert (t1, f1, o1) == got[q], q
        assert np.array_equal(sd[q].cpu().numpy().view(np.uint32), s1.cpu().numpy().view(np.uint32)), q
        assert np.array_equal(pd[q].cpu().numpy().view(np.uint32), p1.cpu().numpy().view(np.uint32)), q
        want, wframe, won = orc.tdt_decode(net, encs[q], states[q].copy(), preds[q].copy())
        if [tuple(t) for t in toks] != want or (frame, on) != (wframe, won):
            apart.append(q)
    print(f"[steps] {m} streams: {steps_multi} steps in one launch; streams apart from the oracle: {apart}",
          flush=True)
    assert len(apart) <= (1 if h == 640 else 0)
    dec.close()


def test_multi_stream_decode_falls_back_and_refuses(tk, orc):
    """With the resident decode off the streams run one after another on the step kernels, with the
    same tokens; a stream past its frames takes no part; shared states are refused."""
    import torch

    import telmo_amd

    rng = np.random.default_rng(77)
    net = tdt_network(rng, 64, 100, [0, 1, 2, 3, 4], layers=2, max_symbols=4, blank_bias=3.0)
    dec = upload(tk, net)
    encs = [rng.standard_normal((f, 64)).astype(np.float32) for f in (30, 40, 25)]
    dev = lambda a: torch.from_numpy(a.copy()).cuda()  # noqa: E731
    zero_s, zero_p = np.zeros(2 * 2 * 64, np.float32), np.zeros(64, np.float32)
    runs = []
    for resident in (True, False):
        dec.set_resident(resident)
        say("multi-stream decode", "resident" if resident else "steps")
        got = dec.decode_streams([dev(e) for e in encs], [dev(zero_s) for _ in encs], [dev(zero_p) for _ in encs],
                                 frames=[0, 40, 0])
        assert dec.last_resident == (2 if resident else 0)
        assert got[1] == ([], 40, 0)  # started past its frames
        runs.append(got)
    assert runs[0] == runs[1]
    for q in (0, 2):
        want, wframe, won = orc.tdt_decode(net, encs[q], zero_s.copy(), zero_p.copy())
        assert [tuple(t) for t in runs[0][q][0]] == want
    dec.set_resident(True)
    shared = dev(zero_s)
    with pytest.raises(telmo_amd.TelmoError, match="share"):
        dec.decode_streams([dev(e) for e in encs[:2]], [shared, shared], [dev(zero_p), dev(zero_p)])
    dec.close()
