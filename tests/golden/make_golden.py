"""Writes the golden fixtures of the matrix product: inputs and expected outputs.

Inputs come from telmo's test generator (xorshift64, src/kernels/mod.rs:795-805) through the
oracle: uniform u in [-1, 1), normals by Box-Muller, int8 weights floor(u01 * 255) - 127 and
scales 0.001 + 0.009 u01. Expected outputs are the oracle's fused sums (the reference's AVX2 /
AVX-512 / NEON semantics, src/kernels/mod.rs:530-688) and, for int8 and Q8_0 weights, the
integer oracle of the two-digit fast path. Each case is one .npz (no pickled objects) plus an entry in
cases.json. The row kernels (LayerNorm, GLU, the depthwise convolution) and the TDT decoder
(predict_rows, decode_inner on a small int8 network) get fixtures of their own, listed in rows.json.

    python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as orc  # noqa: E402

PREC = {"f32": orc.F32, "f16": orc.F16, "bf16": orc.BF16, "int8": orc.INT8, "q8_0": orc.Q8_0}
ACT = {"none": orc.NONE, "relu": orc.RELU, "silu": orc.SILU}


class Stream:
    """Consecutive draws of telmo's generator: seed s gives the s-th block."""

    def __init__(self, seed):
        self.seed = seed

    def uniform(self, n):
        self.seed += 1
        return orc.random(n, self.seed)

    def u01(self, n):
        return ((self.uniform(n).astype(np.float64) + 1.0) / 2.0)

    def normal(self, n):
        u1 = self.u01(n)
        u2 = self.u01(n)
        u1 = np.maximum(u1, 2.0 ** -24)
        return (np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)).astype(np.float32)


def weights(st, prec, n, k):
    """Panel values and scales for precision prec (int8: telmo's random int8 and scales)."""
    if prec == "int8":
        q = (np.floor(st.u01(n * k) * 255.0) - 127.0).astype(np.int8).reshape(n, k)
        s = (0.001 + 0.009 * st.u01(n)).astype(np.float32)
        panels = -(-n // 16)
        pad = np.zeros((panels * 16, k), np.int8)
        pad[:n] = q
        values = pad.reshape(panels, 16, k).transpose(0, 2, 1).reshape(-1).view(np.uint8).copy()
        scales = np.zeros(panels * 16, np.float32)
        scales[:n] = s
        return values, scales
    w = st.normal(n * k) * np.float32(0.05)
    return orc.encode(w.reshape(n, k), n, k, PREC[prec])


CASES = [
    # (name, m, k, n, precision, act, scale, accumulate, bias, lda_pad, ldc_pad)
    ("shape_1x1x1", 1, 1, 1, "int8", "none", 1.0, False, False, 0, 0),
    ("shape_3x7x5", 3, 7, 5, "int8", "relu", 1.0, False, True, 0, 0),
    ("shape_8x64x16", 8, 64, 16, "int8", "silu", 1.0, False, True, 0, 0),
    ("shape_9x64x16", 9, 64, 16, "int8", "none", 0.5, True, False, 0, 0),
    ("shape_13x100x50", 13, 100, 50, "int8", "silu", 2.0, True, True, 3, 5),
    ("shape_64x128x96", 64, 128, 96, "int8", "relu", 1.0, False, True, 0, 0),
    ("gemv_4x640x200", 4, 640, 200, "int8", "none", 1.0 / 16, False, True, 0, 0),
    ("config1_slice_16x1024x64", 16, 1024, 64, "int8", "none", 1.0, False, False, 0, 0),
    ("f32_13x64x40", 13, 64, 40, "f32", "silu", 1.0, False, True, 0, 0),
    ("f16_13x64x40", 13, 64, 40, "f16", "relu", 1.0, True, False, 0, 0),
    ("bf16_13x64x40", 13, 64, 40, "bf16", "none", 0.5, False, True, 0, 0),
    ("q8_0_13x64x40", 13, 64, 40, "q8_0", "silu", 1.0, False, True, 0, 0),
    ("q8_0_4x96x33", 4, 96, 33, "q8_0", "relu", 0.5, True, True, 0, 0),
    ("q8_0_40x256x70", 40, 256, 70, "q8_0", "none", 1.0, False, True, 2, 3),
]


def make(case, seed):
    name, m, k, n, prec, act, scale, acc, with_bias, lpad, cpad = case
    st = Stream(seed * 1000)
    lda, ldc = k + lpad, n + cpad
    if name.startswith("config1"):
        a = st.normal(m * lda)
    else:
        a = st.uniform(m * lda)
    values, scales = weights(st, prec, n, k)
    bias = st.uniform(n) if with_bias else np.zeros(0, np.float32)
    c0 = st.uniform(m * ldc)
    fused = c0.copy()
    rc = orc.matmul(True, a, lda, m, values, scales, PREC[prec], n, k, fused, ldc,
                    bias if with_bias else None, ACT[act], scale, acc)
    assert rc == 0, (name, rc)
    out = {"a": a, "values": values, "scales": scales, "bias": bias, "c0": c0, "c_fused": fused}
    if prec in ("int8", "q8_0"):
        fast = c0.copy()
        fn = orc.matmul_fast if prec == "int8" else orc.matmul_fast_q8
        fn(a, lda, m, values, scales, n, k, fast, ldc, bias if with_bias else None, ACT[act], scale, acc)
        out["c_fast"] = fast
    meta = {"name": name, "m": m, "k": k, "n": n, "lda": lda, "ldc": ldc, "precision": prec, "act": act,
            "scale": scale, "accumulate": acc, "bias": with_bias, "seed": seed}
    return meta, out


ROW_CASES = [
    # (name, kind, params)
    ("layer_norm_5x1000", "layer_norm", {"m": 5, "n": 1000, "eps": 1e-5}),
    ("glu_3x600", "glu", {"m": 3, "half": 300}),
    ("dwconv_40x96_k9", "dwconv", {"frames": 40, "channels": 96, "kernel": 9, "t0": 0, "stride": 1, "rows": 40,
                                   "silu": True}),
    ("dwconv_37x70_k15_s2", "dwconv", {"frames": 37, "channels": 70, "kernel": 15, "t0": 1, "stride": 2,
                                       "rows": 18, "silu": False}),
    ("tdt_h32_v20", "tdt", {"h": 32, "vocab": 20, "durations": [0, 1, 2, 3, 4], "layers": 2, "max_symbols": 3,
                            "frames": 30, "rows": 3}),
]


def int8_panels(st, n, k, lo, hi):
    q = (np.floor(st.u01(n * k) * 255.0) - 127.0).astype(np.int8).reshape(n, k)
    s = (lo + (hi - lo) * st.u01(n)).astype(np.float32)
    panels = -(-n // 16)
    pad = np.zeros((panels * 16, k), np.int8)
    pad[:n] = q
    values = pad.reshape(panels, 16, k).transpose(0, 2, 1).reshape(-1).view(np.uint8).copy()
    scales = np.zeros(panels * 16, np.float32)
    scales[:n] = s
    return values, scales


def make_row(case, seed):
    name, kind, p = case
    st = Stream(seed * 1000 + 500)
    out = {}
    if kind == "layer_norm":
        x = (st.normal(p["m"] * p["n"]) * np.float32(3.0) + np.float32(2.0)).reshape(p["m"], p["n"])
        gamma, beta = np.float32(1.0) + st.uniform(p["n"]) * np.float32(0.1), st.uniform(p["n"]) * np.float32(0.1)
        out = {"x": x, "gamma": gamma, "beta": beta,
               "out": np.stack([orc.layer_norm(r, gamma, beta, p["eps"]) for r in x])}
    elif kind == "glu":
        x = (st.normal(p["m"] * 2 * p["half"]) * np.float32(4.0)).reshape(p["m"], 2 * p["half"])
        out = {"x": x, "out": np.stack([orc.glu(r[:p["half"]], r[p["half"]:]) for r in x])}
    elif kind == "dwconv":
        x = st.normal(p["frames"] * p["channels"]).reshape(p["frames"], p["channels"])
        w = (st.uniform(p["kernel"] * p["channels"]) * np.float32(0.5)).reshape(p["kernel"], p["channels"])
        bias = st.uniform(p["channels"])
        out = {"x": x, "w": w, "bias": bias,
               "out": orc.dwconv1d(x, w, bias, rows=p["rows"], t0=p["t0"], stride=p["stride"], silu=p["silu"])}
    else:  # a small int8 TDT network: predict_rows on a few rows, then a decode from the start state
        h, vocab, nd, L = p["h"], p["vocab"], len(p["durations"]), p["layers"]
        net = {"p": orc.INT8, "h": h, "vocab": vocab, "durations": p["durations"], "max_symbols": p["max_symbols"]}
        net["joint"] = int8_panels(st, vocab + nd, h, 0.001, 0.01)
        net["joint_b"] = st.uniform(vocab + nd) * np.float32(0.5)
        net["joint_b"][vocab - 1] += np.float32(1.0)  # the blank: runs of blanks between tokens
        net["emb"] = (st.normal(vocab * h) * np.float32(0.5)).reshape(vocab, h)
        net["lstm"] = [int8_panels(st, 4 * h, 2 * h, 0.004, 0.008) for _ in range(L)]
        net["lstm_b"] = [st.uniform(4 * h) * np.float32(0.1) for _ in range(L)]
        net["proj"] = int8_panels(st, h, h, 0.01, 0.03)
        net["proj_b"] = st.uniform(h) * np.float32(0.1)
        tokens = (np.floor(st.u01(p["rows"]) * vocab)).astype(np.int32)
        states0 = (st.uniform(p["rows"] * L * 2 * h) * np.float32(0.5)).reshape(p["rows"], L * 2 * h)
        states, preds = states0.copy(), np.zeros((p["rows"], h), np.float32)
        orc.tdt_predict(net, tokens, states, preds)
        enc = st.normal(p["frames"] * h).reshape(p["frames"], h)
        state = np.zeros(L * 2 * h, np.float32)
        pred = np.zeros(h, np.float32)
        orc.tdt_predict(net, [vocab - 1], state.reshape(1, -1), pred.reshape(1, -1))  # the start state
        state0, pred0 = state.copy(), pred.copy()
        toks, frame, on = orc.tdt_decode(net, enc, state, pred)
        out = {"joint_values": net["joint"][0], "joint_scales": net["joint"][1], "joint_b": net["joint_b"],
               "emb": net["emb"], "proj_values": net["proj"][0], "proj_scales": net["proj"][1],
               "proj_b": net["proj_b"], "tokens_in": tokens, "states0": states0, "states": states, "preds": preds,
               "enc": enc, "state0": state0, "pred0": pred0, "state": state, "pred": pred,
               "tokens": np.asarray(toks, np.int32).reshape(-1, 3), "end": np.asarray([frame, on], np.int64)}
        for l in range(L):
            out[f"lstm{l}_values"], out[f"lstm{l}_scales"] = net["lstm"][l]
            out[f"lstm{l}_b"] = net["lstm_b"][l]
    meta = {"name": name, "kind": kind, "seed": seed, **p}
    return meta, out


def main():
    metas = []
    for i, case in enumerate(CASES):
        meta, arrays = make(case, i + 1)
        np.savez_compressed(os.path.join(HERE, meta["name"] + ".npz"), **arrays)
        metas.append(meta)
    with open(os.path.join(HERE, "cases.json"), "w") as f:
        json.dump(metas, f, indent=1)
    rows = []
    for i, case in enumerate(ROW_CASES):
        meta, arrays = make_row(case, i + 1)
        np.savez_compressed(os.path.join(HERE, meta["name"] + ".npz"), **arrays)
        rows.append(meta)
    with open(os.path.join(HERE, "rows.json"), "w") as f:
        json.dump(rows, f, indent=1)
    print(f"wrote {len(metas)} product cases and {len(rows)} row and TDT cases")


if __name__ == "__main__":
    main()
