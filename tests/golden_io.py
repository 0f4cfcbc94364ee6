"""Loader for the committed golden fixtures (tests/golden/*.npz).

Fixtures are plain arrays (numpy's default allow_pickle=False); inputs of bf16
cases are stored as raw 16-bit patterns under ``<name>_bf16`` and come back as
the float32 values they encode."""
import glob
import os

import numpy as np

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def names():
    return sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN_DIR, "*.npz")))


def load(name):
    with np.load(os.path.join(GOLDEN_DIR, name + ".npz")) as z:
        out = {}
        for k in z.files:
            a = z[k]
            if k.endswith("_bf16"):
                out[k[:-5]] = (a.astype(np.uint32) << 16).view(np.float32)
            elif a.dtype.kind == "U":
                out[k] = str(a)
            else:
                out[k] = a
    return out
