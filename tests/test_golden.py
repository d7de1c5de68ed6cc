"""The golden fixtures: the oracle still reproduces them, bit for bit, from their inputs; and the
inputs are what telmo's generator gives for their seeds (src/kernels/mod.rs:795-805)."""
import os
import sys

import numpy as np
import pytest

from golden_cases import ACT, GOLDEN, PREC, cases, load, rows, tdt_net

CASES = cases()


@pytest.mark.parametrize("meta", CASES, ids=[c["name"] for c in CASES])
def test_the_oracle_reproduces_the_fixture(orc, meta):
    g = load(meta)
    m, k, n, lda, ldc = meta["m"], meta["k"], meta["n"], meta["lda"], meta["ldc"]
    bias = g["bias"] if meta["bias"] else None
    c = g["c0"].copy()
    assert orc.matmul(True, g["a"], lda, m, g["values"], g["scales"], PREC[meta["precision"]], n, k, c, ldc, bias,
                      ACT[meta["act"]], meta["scale"], meta["accumulate"]) == 0
    assert np.array_equal(c.view(np.uint32), g["c_fused"].view(np.uint32))
    if meta["precision"] in ("int8", "q8_0"):
        c = g["c0"].copy()
        fast = orc.matmul_fast if meta["precision"] == "int8" else orc.matmul_fast_q8
        fast(g["a"], lda, m, g["values"], g["scales"], n, k, c, ldc, bias, ACT[meta["act"]],
             meta["scale"], meta["accumulate"])
        assert np.array_equal(c.view(np.uint32), g["c_fast"].view(np.uint32))
        # the fast path stays within the gate of the fused sums on every fixture
        got, want = g["c_fast"].reshape(m, ldc)[:, :n], g["c_fused"].reshape(m, ldc)[:, :n]
        scale = np.maximum(np.abs(want).max(axis=1, keepdims=True), 1e-30)
        assert (np.abs(got - want) / scale).max() <= 1e-3


def test_the_inputs_come_from_the_generator(orc):
    sys.path.insert(0, GOLDEN)
    import make_golden

    for i, case in enumerate(make_golden.CASES):
        meta, arrays = make_golden.make(case, i + 1)
        g = load(meta)
        for key in ("a", "values", "scales", "bias", "c0"):
            assert np.array_equal(arrays[key], g[key]), (meta["name"], key)
    assert os.path.exists(os.path.join(GOLDEN, "cases.json"))


ROWS = rows()


@pytest.mark.parametrize("meta", ROWS, ids=[c["name"] for c in ROWS])
def test_the_oracle_reproduces_the_row_and_tdt_fixtures(orc, meta):
    g = load(meta)
    kind = meta["kind"]
    if kind == "layer_norm":
        got = np.stack([orc.layer_norm(r, g["gamma"], g["beta"], meta["eps"]) for r in g["x"]])
        assert np.array_equal(got.view(np.uint32), g["out"].view(np.uint32))
    elif kind == "glu":
        h = meta["half"]
        got = np.stack([orc.glu(r[:h], r[h:]) for r in g["x"]])
        assert np.array_equal(got.view(np.uint32), g["out"].view(np.uint32))
    elif kind == "dwconv":
        got = orc.dwconv1d(g["x"], g["w"], g["bias"], rows=meta["rows"], t0=meta["t0"], stride=meta["stride"],
                           silu=meta["silu"])
        assert np.array_equal(got.view(np.uint32), g["out"].view(np.uint32))
    else:
        net = tdt_net(meta, g)
        states, preds = g["states0"].copy(), np.zeros_like(g["preds"])
        orc.tdt_predict(net, g["tokens_in"], states, preds)
        assert np.array_equal(states.view(np.uint32), g["states"].view(np.uint32))
        assert np.array_equal(preds.view(np.uint32), g["preds"].view(np.uint32))
        state, pred = g["state0"].copy(), g["pred0"].copy()
        toks, frame, on = orc.tdt_decode(net, g["enc"], state, pred)
        assert np.array_equal(np.asarray(toks, np.int32).reshape(-1, 3), g["tokens"])
        assert [frame, on] == list(g["end"])
        assert np.array_equal(state.view(np.uint32), g["state"].view(np.uint32))
        assert np.array_equal(pred.view(np.uint32), g["pred"].view(np.uint32))


def test_the_row_inputs_come_from_the_generator(orc):
    sys.path.insert(0, GOLDEN)
    import make_golden

    inputs = {"layer_norm": ("x", "gamma", "beta"), "glu": ("x",), "dwconv": ("x", "w", "bias"),
              "tdt": ("joint_values", "joint_scales", "joint_b", "emb", "tokens_in", "states0", "enc")}
    for i, case in enumerate(make_golden.ROW_CASES):
        meta, arrays = make_golden.make_row(case, i + 1)
        g = load(meta)
        for key in inputs[meta["kind"]]:
            assert np.array_equal(arrays[key], g[key]), (meta["name"], key)
