"""Writes the committed fixtures tests/golden/*.npz.

Each fixture holds the input bytes of one flash_attn_ext call laid out as
voxtral.cpp lays them out (tests/cases.py builders, small sizes), the ggml
views (type, ne, nb, offset) per operand, the scale, and the expected output
computed by torch's scaled_dot_product_attention in float64 on the CPU (a
library routine independent of the oracle), with Q rounded to f16 first as
ggml does for an f16 K. The reference holds no vectors for this op (its
arithmetic lives in ggml, absent here), so these are this repository's own.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import cases  # noqa: E402
import refmath  # noqa: E402


def builders():
    yield "decode_gqa4_hd128", cases.decode_case(80, hq=8, hkv=2, hd=128, capacity=96, seed=501)
    yield "decode_window_hd128", cases.decode_case(200, hq=4, hkv=1, hd=128, seed=502, window=64)
    yield "decode_batched_ragged", cases.batched_case(3, hq=4, hkv=1, capacity=64, lo=5, hi=64, seed=503)
    yield "encoder_hd64_nomask", cases.encoder_case(48, 2, 64, seed=504)
    yield "encoder_hd64_window", cases.encoder_case(40, 2, 64, seed=505, window=12)
    yield "prefill_causal_hd128", cases.prefill_case(24, hq=8, hkv=2, seed=506)
    yield "prefill_causal_offset", cases.prefill_case(10, hq=4, hkv=1, seed=507, kv_offset=30)
    c = cases.prefill_case(12, hq=2, hkv=1, seed=508)
    c.bufs["mask"].reshape(12, 12)[3, :] = cases.NEG_INF_F16   # a fully masked row -> zeros
    c.name = "prefill_fully_masked_row"
    yield c.name, c


def save(name, c):
    want, live = refmath.sdpa_f64(c, q_f16=True)
    want = np.where(live[..., None], want, 0.0)
    arrays = {f"buf_{k}": v for k, v in c.bufs.items()}
    meta = {"name": name, "scale": c.scale,
            "views": {r: [b, t, list(ne), list(nb), off] for r, (b, t, ne, nb, off) in c.views.items()}}
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), meta=np.array(json.dumps(meta)),
                        expected=want.astype(np.float64), **arrays)
    print(f"{name}: out {want.shape}")


if __name__ == "__main__":
    for n, c in builders():
        save(n, c)
