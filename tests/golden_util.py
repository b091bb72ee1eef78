"""Loads the committed fixtures of tests/golden/ back into Case objects."""
from __future__ import annotations

import glob
import json
import os

import numpy as np

import cases

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def names():
    return sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN_DIR, "*.npz")))


def load(name):
    """Returns (Case, expected float64 [B, Nq, Hq, D])."""
    with np.load(os.path.join(GOLDEN_DIR, f"{name}.npz"), allow_pickle=False) as z:
        meta = json.loads(str(z["meta"]))
        c = cases.Case(meta["name"], float(meta["scale"]))
        for key in z.files:
            if key.startswith("buf_"):
                c.bufs[key[4:]] = np.ascontiguousarray(z[key])
        for role, (b, t, ne, nb, off) in meta["views"].items():
            c.views[role] = (b, int(t), tuple(ne), tuple(nb), int(off))
        return c, np.array(z["expected"])
