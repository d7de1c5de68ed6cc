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
