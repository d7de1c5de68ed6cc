"""The golden fixtures: the oracle still reproduces them, bit for bit, from their inputs; and the
inputs are what telmo's generator gives for their seeds (src/kernels/mod.rs:795-805)."""
import os
import sys

import numpy as np
import pytest

from golden_cases import ACT, GOLDEN, PREC, cases, load

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
