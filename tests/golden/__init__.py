"""Golden fixtures for the NF4 path (written by make_golden.py from the CPU oracle)."""

import glob
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def load_dequant_fixtures():
    out = []
    for path in sorted(glob.glob(os.path.join(HERE, "dequant_*.npz"))):
        with np.load(path, allow_pickle=False) as f:
            out.append((os.path.basename(path), {k: f[k] for k in f.files}))
    return out
