"""Independent float64 restatements used to pin the oracle on the CPU.

`logical` reads a ggml view into a [ne3, ne2, ne1, ne0] numpy array through
its byte strides; `sdpa_f64` runs torch's scaled_dot_product_attention in
float64 on those arrays (a library routine, CPU only).
"""
from __future__ import annotations

import numpy as np

from oracle.oracle import F16, F32


def logical(case, role) -> np.ndarray | None:
    if not case.has(role):
        return None
    b, t, ne, nb, off = case.views[role]
    buf = case.bufs[b]
    dt = np.float32 if t == F32 else np.float16
    arr = np.ndarray(shape=ne[::-1], dtype=dt, buffer=buf, offset=off, strides=nb[::-1])
    return arr.astype(np.float64)


def expand(case):
    """Q, K, V, mask as float64 [B, H, N, D] / [B, Hq, Nq, Nkv] with the GQA,
    batch and mask-plane broadcasts of the ggml contract made explicit."""
    q = logical(case, "q")
    k = logical(case, "k")
    v = logical(case, "v")
    m = logical(case, "mask")
    B, Hq, Nq, D = q.shape
    Bk, Hkv = k.shape[0], k.shape[1]
    k = np.repeat(np.repeat(k, Hq // Hkv, axis=1), B // Bk, axis=0)
    v = np.repeat(np.repeat(v, Hq // Hkv, axis=1), B // Bk, axis=0)
    if m is not None:
        Bm, Hm = m.shape[0], m.shape[1]
        m = m[:, :, :Nq, :]
        m = np.tile(m, (B // Bm, Hq // Hm, 1, 1))  # plane index h % Hm, batch b % Bm
    return q, k, v, m


def sdpa_f64(case, q_f16=None):
    """torch SDPA in float64; returns [B, Nq, Hq, D] and a mask of live rows.
    Q is rounded to f16 first when q_f16, by default when K is f16 (ggml
    converts Q to K's dot type)."""
    import torch

    if q_f16 is None:
        q_f16 = case.views["k"][1] == F16
    q, k, v, m = expand(case)
    if q_f16:
        q = q.astype(np.float16).astype(np.float64)
    tq, tk, tv = (torch.from_numpy(np.ascontiguousarray(x)) for x in (q, k, v))
    tm = torch.from_numpy(np.ascontiguousarray(m)) if m is not None else None
    out = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=tm, scale=case.scale)
    out = out.numpy().transpose(0, 2, 1, 3)  # [B, Nq, Hq, D]
    if m is None:
        live = np.ones(out.shape[:3], dtype=bool)
    else:
        live = np.isfinite(m).any(axis=-1).transpose(0, 2, 1)  # [B, Nq, Hq]
    return out, live
