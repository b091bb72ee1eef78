"""Seeded attention inputs laid out exactly as voxtral.cpp lays them out.

A Case holds contiguous host buffers (numpy) and, per operand, the ggml view
(type, ne, nb, byte offset) into one of them. The same bytes go to the oracle
(host) and, in GPU tests, to the device, so both see identical inputs.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from conftest import load_package
from oracle.oracle import F16, F32, View

views = load_package().views

NEG_INF_F16 = np.uint16(0xFC00)


def f16_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def f32(x: float) -> float:
    """ggml stores the scale as a float op param; keep it float32-exact."""
    return float(np.float32(x))


def normal(rng, shape, sigma=1.0):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma)).astype(np.float32)


@dataclass
class Case:
    name: str
    scale: float
    bufs: dict = field(default_factory=dict)       # name -> contiguous np.ndarray
    views: dict = field(default_factory=dict)      # role -> (buf, type, ne, nb, offset)
    meta: dict = field(default_factory=dict)

    def add(self, role, buf_name, arr, type_, ne, nb, offset=0):
        if buf_name not in self.bufs:
            self.bufs[buf_name] = np.ascontiguousarray(arr)
        self.views[role] = (buf_name, type_, tuple(ne), tuple(nb), offset)

    def has(self, role):
        return role in self.views

    def oracle_view(self, role):
        if role not in self.views:
            return None
        b, t, ne, nb, off = self.views[role]
        return View(self.bufs[b], t, ne, nb, off)

    @property
    def out_shape(self):
        _, _, qne, _, _ = self.views["q"]
        _, _, vne, _, _ = self.views["v"]
        return (qne[3], qne[1], qne[2], vne[0])  # [B, Nq, Hq, D]

    def dst_ne_nb(self):
        B, Nq, Hq, D = self.out_shape
        return views.dst(D, Hq, Nq, B)


# ---------------------------------------------------------------------------
# builders for the shapes voxtral.cpp produces


def decode_case(n_kv, hq=32, hkv=8, hd=128, capacity=None, seed=1, q_sigma=1.0, kv_sigma=1.0,
                batch=1, window=None, name=None, q_f16=False, kv_f32=False):
    """Single-token decode against a token-major f16 cache (src/voxtral.cpp:1736-1805).
    window: if set, additive mask [n_kv, 1] with -inf outside the last `window` rows.
    kv_f32: the cache is F32, the reference's own cache type (:1126-1136)."""
    rng = np.random.default_rng(seed)
    cap = capacity or n_kv
    c = Case(name or f"decode_nkv{n_kv}_b{batch}", f32(1.0 / math.sqrt(hd)))
    q = normal(rng, (batch, 1, hq, hd), q_sigma)
    if q_f16:
        c.add("q", "q", f16_bits(q), F16, *_batched_q(1, hq, hd, 2, batch))
    else:
        c.add("q", "q", q, F32, *_batched_q(1, hq, hd, 4, batch))
    k = f16_bits(normal(rng, (batch, cap, hkv, hd), kv_sigma))
    v = f16_bits(normal(rng, (batch, cap, hkv, hd), kv_sigma))
    if kv_f32:
        k, v = _widen(k), _widen(v)
    ne, nb = views.kv_cache(n_kv, hkv, hd, cap, elt=4 if kv_f32 else 2, batch=batch)
    c.add("k", "k", k, F32 if kv_f32 else F16, ne, nb)
    c.add("v", "v", v, F32 if kv_f32 else F16, ne, nb)
    if window is not None:
        m = np.zeros((batch, 1, n_kv), dtype=np.uint16)
        m[:, :, : max(0, n_kv - window)] = NEG_INF_F16
        c.add("mask", "mask", m, F16, *views.mask(n_kv, 1, 1, batch))
    return c


def _widen(h, perturb=True):
    """f16 bits -> F32 values. With perturb, each value moves by a few f16 ulps
    of pseudo-random F32 detail, so F32 inputs are not f16-valued (the path
    must round them itself, as it rounds Q)."""
    x = h.view(np.float16).astype(np.float32)
    if perturb:
        r = np.random.default_rng(x.size).uniform(-1.0, 1.0, size=x.shape).astype(np.float32)
        x = (x + r * np.abs(x) * np.float32(2.0 ** -9)).astype(np.float32)
    return np.ascontiguousarray(x)


def _batched_q(n_tokens, heads, hd, elt, batch):
    ne, nb = views.decoder_q(n_tokens, heads, hd, elt)
    return (ne[0], ne[1], ne[2], batch), (nb[0], nb[1], nb[2], n_tokens * heads * hd * elt)


def encoder_case(seq=1500, heads=20, hd=64, seed=2, name=None, window=None, scale=None, q_f16=False,
                 k_ramp=0.0, q_sigma=1.0, kv_f32=False):
    """Encoder self-attention (src/voxtral.cpp:1580-1613): q/k/v [hd, seq, heads]
    views of [seq][heads][hd] buffers. q is f16-valued, stored as F32 (the
    reference's q is a mul_mat output) or, with q_f16, as F16; window: realtime
    sliding-causal mask (src/voxtral.cpp:2179-2190). k_ramp > 0 scales key row
    j by 1 + k_ramp * j / seq, so row maxima keep growing along the KV axis.
    scale defaults to 1/sqrt(hd). kv_f32: K/V are F32, as the reference's
    mul_mat outputs are (src/voxtral.cpp:1581-1605)."""
    rng = np.random.default_rng(seed)
    c = Case(name or f"encoder_seq{seq}", f32(1.0 / math.sqrt(hd) if scale is None else scale))
    qh = f16_bits(normal(rng, (seq, heads, hd), q_sigma))
    q = qh.view(np.float16).astype(np.float32)
    kf = normal(rng, (seq, heads, hd))
    if k_ramp:
        kf = kf * (1.0 + k_ramp * np.arange(seq, dtype=np.float32) / seq)[:, None, None]
    k = f16_bits(kf)
    v = f16_bits(normal(rng, (seq, heads, hd)))
    if q_f16:
        c.add("q", "q", qh, F16, *views.encoder_qkv(seq, heads, hd, 2))
    else:
        c.add("q", "q", q, F32, *views.encoder_qkv(seq, heads, hd, 4))
    if kv_f32:
        c.add("k", "k", _widen(k), F32, *views.encoder_qkv(seq, heads, hd, 4))
        c.add("v", "v", _widen(v), F32, *views.encoder_qkv(seq, heads, hd, 4))
    else:
        c.add("k", "k", k, F16, *views.encoder_qkv(seq, heads, hd, 2))
        c.add("v", "v", v, F16, *views.encoder_qkv(seq, heads, hd, 2))
    if window is not None:
        qi = np.arange(seq)[:, None]
        ki = np.arange(seq)[None, :]
        allow = (ki <= qi) & (ki >= qi - (window - 1))
        m = np.where(allow, np.uint16(0), NEG_INF_F16).astype(np.uint16)
        c.add("mask", "mask", m, F16, *views.mask(seq, seq))
    return c


def prefill_case(n=439, hq=32, hkv=8, hd=128, seed=3, causal=True, kv_offset=0, capacity=None, name=None,
                 kv_f32=False):
    """Decoder prefill (src/voxtral.cpp:1736-1805) with the causal mask of
    fill_causal_mask (:2104-2111); kv_offset > 0 gives n_kv = kv_offset + n.
    kv_f32: the reference's F32 cache (:1126-1136)."""
    rng = np.random.default_rng(seed)
    n_kv = kv_offset + n
    cap = capacity or n_kv
    c = Case(name or f"prefill_n{n}_off{kv_offset}", f32(1.0 / math.sqrt(hd)))
    q = normal(rng, (n, hq, hd))
    c.add("q", "q", q, F32, *views.decoder_q(n, hq, hd))
    k = f16_bits(normal(rng, (cap, hkv, hd)))
    v = f16_bits(normal(rng, (cap, hkv, hd)))
    if kv_f32:
        k, v = _widen(k), _widen(v)
    ne, nb = views.kv_cache(n_kv, hkv, hd, cap, elt=4 if kv_f32 else 2)
    c.add("k", "k", k, F32 if kv_f32 else F16, ne, nb)
    c.add("v", "v", v, F32 if kv_f32 else F16, ne, nb)
    if causal:
        qi = np.arange(n)[:, None] + kv_offset
        ki = np.arange(n_kv)[None, :]
        m = np.where(ki <= qi, np.uint16(0), NEG_INF_F16).astype(np.uint16)
        c.add("mask", "mask", m, F16, *views.mask(n_kv, n))
    return c


def implicit_mask(nq, nkv, offset, window=0):
    """The explicit F16 mask [nq, nkv] that an implicit causal / window mask
    descriptor stands for (include/vxfa.h): row i attends j iff
    j <= i + offset and, for window > 0, j >= i + offset - window + 1."""
    qi = np.arange(nq, dtype=np.int64)[:, None] + offset
    ki = np.arange(nkv, dtype=np.int64)[None, :]
    allow = ki <= qi
    if window > 0:
        allow &= ki >= qi - window + 1
    return np.where(allow, np.uint16(0), NEG_INF_F16).astype(np.uint16)


def with_mask(c: Case, m: np.ndarray) -> Case:
    """Attach (or replace) an explicit mask [nq, nkv] broadcast over heads and batch."""
    nq, nkv = m.shape
    c.bufs.pop("mask", None)
    c.views.pop("mask", None)
    c.add("mask", "mask", np.ascontiguousarray(m), F16, *views.mask(nkv, nq))
    return c


def ring_case(c: Case, capacity: int, start: int, seed=0) -> Case:
    """The decode case c (a linear cache whose k/v views hold n_kv rows) laid
    out as a ring of `capacity` rows: logical row p at cache row
    (start + p) % capacity, every other row random f16. k/v views cover the
    whole ring [D, capacity, Hkv, Bk]."""
    import copy
    rng = np.random.default_rng(seed)
    r = copy.deepcopy(c)
    r.name = f"{c.name}_ring{capacity}_at{start}"
    for role in ("k", "v"):
        b, t, ne, nb, off = c.views[role]
        D, nkv, hkv, bk = ne
        assert off == 0 and nkv <= capacity
        lin = c.bufs[b].reshape(bk, -1, hkv, D)
        ring = f16_bits(normal(rng, (bk, capacity, hkv, D)))
        rows = (start + np.arange(nkv)) % capacity
        ring[:, rows] = lin[:, :nkv]
        r.bufs[b] = ring
        rne, rnb = views.kv_cache(capacity, hkv, D, capacity, batch=bk)
        r.views[role] = (b, t, rne, rnb, 0)
    return r


def _powf(x, y):
    """libm's powf, the function ggml's CPU rope uses for its theta scale."""
    import ctypes
    import ctypes.util
    m = ctypes.CDLL(ctypes.util.find_library("m"))
    m.powf.restype = ctypes.c_float
    m.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    return np.float32(m.powf(np.float32(x), np.float32(y)))


def rope_ggml(x, positions, n_dims, freq_base):
    """ggml_rope_ext, mode 0, freq_scale 1, ext_factor 0, attn_factor 1 (the
    arguments of src/voxtral.cpp:1746-1749): x [..., n_tok, heads, D] float32,
    token t at positions[t]. Pair j of a head turns by theta_j with
    theta_0 = p and theta_{j+1} = theta_j * powf(freq_base, -2 / n_dims) in
    float32 (ggml's running product); cos / sin of the float32 angle."""
    x = np.asarray(x, dtype=np.float32)
    ts = _powf(freq_base, np.float32(-2.0) / np.float32(n_dims))
    out = x.copy()
    for t, p in enumerate(positions):
        th = np.float32(p)
        for j in range(n_dims // 2):
            c = np.float32(np.cos(np.float64(th)))
            s = np.float32(np.sin(np.float64(th)))
            x0 = x[..., t, :, 2 * j]
            x1 = x[..., t, :, 2 * j + 1]
            out[..., t, :, 2 * j] = x0 * c - x1 * s
            out[..., t, :, 2 * j + 1] = x0 * s + x1 * c
            th = np.float32(th * ts)
    return out


def batched_case(n_streams=32, hq=32, hkv=8, hd=128, capacity=8192, lo=512, hi=8192, seed=5,
                 kv_sigma=0.5, name=None, kv_f32=False):
    """32 independent decode streams along ne[3] with ragged valid lengths
    drawn from U{lo..hi} and a per-stream length mask [cap, 1, 1, B]."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=n_streams)
    c = decode_case(capacity, hq, hkv, hd, capacity=capacity, seed=seed + 1000, kv_sigma=kv_sigma,
                    batch=n_streams, name=name or f"batched_{n_streams}", kv_f32=kv_f32)
    m = np.zeros((n_streams, 1, capacity), dtype=np.uint16)
    for b, L in enumerate(lens):
        m[b, 0, L:] = NEG_INF_F16
    c.add("mask", "mask", m, F16, *views.mask(capacity, 1, 1, n_streams))
    c.meta["lens"] = lens
    return c


def oracle_ggml(c: Case, vkq_f16=False, flags=0, threads=None):
    """ggml-faithful restatement; fp32 V accumulation unless vkq_f16 (the one-row
    kernel's f16 accumulator, used as the bracket)."""
    from oracle import oracle
    return oracle.fa_ggml(c.oracle_view("q"), c.oracle_view("k"), c.oracle_view("v"), c.oracle_view("mask"),
                          c.scale, vkq_f16=vkq_f16, flags=flags, threads=threads)


def q_rounded(c: Case) -> bool:
    """ggml converts Q to K's dot type: f16 for an f16 K, none for an F32 K."""
    return c.views["k"][1] == F16


def oracle_f64(c: Case, threads=None, q_f16=None):
    """Exact float64 attention; Q rounded to f16 when K is f16 (ggml's Q
    conversion), unless q_f16 says otherwise."""
    from oracle import oracle
    return oracle.fa_f64(c.oracle_view("q"), c.oracle_view("k"), c.oracle_view("v"), c.oracle_view("mask"),
                         c.scale, q_f16=q_rounded(c) if q_f16 is None else q_f16, threads=threads)
