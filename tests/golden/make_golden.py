"""Writes the golden fixtures of the matrix product: inputs and expected outputs.

Inputs come from telmo's test generator (xorshift64, src/kernels/mod.rs:795-805) through the
oracle: uniform u in [-1, 1), normals by Box-Muller, int8 weights floor(u01 * 255) - 127 and
scales 0.001 + 0.009 u01. Expected outputs are the oracle's fused sums (the reference's AVX2 /
AVX-512 / NEON semantics, src/kernels/mod.rs:530-688) and, for int8 and Q8_0 weights, the
integer oracle of the two-digit fast path. Each case is one .npz (no pickled objects) plus an entry in
cases.json.

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


def main():
    metas = []
    for i, case in enumerate(CASES):
        meta, arrays = make(case, i + 1)
        np.savez_compressed(os.path.join(HERE, meta["name"] + ".npz"), **arrays)
        metas.append(meta)
    with open(os.path.join(HERE, "cases.json"), "w") as f:
        json.dump(metas, f, indent=1)
    print(f"wrote {len(metas)} cases")


if __name__ == "__main__":
    main()
