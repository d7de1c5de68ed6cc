"""Loading the golden fixtures of tests/golden (inputs and expected outputs, no pickles)."""
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
PREC = {"f32": 0, "f16": 1, "bf16": 2, "int8": 3, "q8_0": 4}
ACT = {"none": 0, "relu": 1, "silu": 2}


def cases():
    with open(os.path.join(GOLDEN, "cases.json")) as f:
        return json.load(f)


def load(meta):
    with np.load(os.path.join(GOLDEN, meta["name"] + ".npz")) as z:
        return {key: z[key] for key in z.files}


def rows():
    """The row-kernel and TDT fixtures (rows.json)."""
    with open(os.path.join(GOLDEN, "rows.json")) as f:
        return json.load(f)


def tdt_net(meta, g):
    """The oracle's network dict of a TDT fixture."""
    L = meta["layers"]
    return {"p": PREC["int8"], "h": meta["h"], "vocab": meta["vocab"], "durations": meta["durations"],
            "max_symbols": meta["max_symbols"], "joint": (g["joint_values"], g["joint_scales"]), "joint_b": g["joint_b"],
            "emb": g["emb"], "lstm": [(g[f"lstm{l}_values"], g[f"lstm{l}_scales"]) for l in range(L)],
            "lstm_b": [g[f"lstm{l}_b"] for l in range(L)], "proj": (g["proj_values"], g["proj_scales"]),
            "proj_b": g["proj_b"]}
