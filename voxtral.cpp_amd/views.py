"""The tensor views voxtral.cpp hands to ggml_flash_attn_ext, as (ne, nb).

Each function restates the ggml_reshape / ggml_permute / ggml_view chain of
the reference graph builder for one operand, so callers (tests, bench, a
host executor) place data in exactly the byte layout the real app produces.
ne is ggml order (ne[0] fastest); nb are byte strides.
"""
from __future__ import annotations

F32_SIZE, F16_SIZE = 4, 2


def encoder_qkv(seq: int, heads: int, hd: int, elt: int):
    """Encoder q/k/v: mul_mat output [heads*hd, seq] reshaped to [hd, heads, seq]
    and permuted (0,2,1,3) to [hd, seq, heads] (src/voxtral.cpp:1581-1605).
    Backing buffer: [seq][heads][hd] contiguous."""
    ne = (hd, seq, heads, 1)
    nb = (elt, heads * hd * elt, hd * elt, seq * heads * hd * elt)
    return ne, nb


def decoder_q(n_tokens: int, heads: int, hd: int, elt: int = F32_SIZE):
    """Decoder q: contiguous [heads*hd, n_tokens] reshaped to [hd, heads, n_tokens]
    and permuted to [hd, n_tokens, heads] (src/voxtral.cpp:1775-1776).
    Backing buffer: [n_tokens][heads][hd]."""
    ne = (hd, n_tokens, heads, 1)
    nb = (elt, heads * hd * elt, hd * elt, n_tokens * heads * hd * elt)
    return ne, nb


def kv_cache(n_kv: int, kv_heads: int, hd: int, capacity: int, elt: int = F16_SIZE, batch: int = 1):
    """K or V of one layer: a view of the first n_kv rows of the token-major
    cache [kv_dim, capacity] (kv_dim = kv_heads*hd), reshaped to
    [hd, kv_heads, n_kv] and permuted to [hd, n_kv, kv_heads]
    (src/voxtral.cpp:1773-1794; cache allocated at :1126-1136).
    Backing buffer: [batch][capacity][kv_heads][hd]; batch > 1 stacks
    independent streams along ne[3]."""
    ne = (hd, n_kv, kv_heads, batch)
    nb = (elt, kv_heads * hd * elt, hd * elt, capacity * kv_heads * hd * elt)
    return ne, nb


def mask(n_kv: int, rows: int, planes: int = 1, batch: int = 1, row_stride: int | None = None):
    """Additive F16 mask [n_kv, rows, planes, batch], rows contiguous
    (causal [n, n] at src/voxtral.cpp:2104-2111, cast to F16 at :1801)."""
    rs = row_stride if row_stride is not None else n_kv
    ne = (n_kv, rows, planes, batch)
    nb = (F16_SIZE, rs * F16_SIZE, rs * rows * F16_SIZE, rs * rows * planes * F16_SIZE)
    return ne, nb


def dst(hd: int, heads: int, n_tokens: int, batch: int = 1):
    """Output of flash_attn_ext: F32 [hd, heads, n_tokens, batch], contiguous
    (already permuted; voxtral then applies cont + reshape, :1612, :1804)."""
    ne = (hd, heads, n_tokens, batch)
    nb = (F32_SIZE, hd * F32_SIZE, hd * heads * F32_SIZE, hd * heads * n_tokens * F32_SIZE)
    return ne, nb
