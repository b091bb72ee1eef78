"""TEST INFRASTRUCTURE ONLY: ctypes binding of the CPU oracle (fa_oracle.c).

Used by tests/ as the parity checker and by bench.py's cpu_baseline leg.
The product path never imports this module.

A tensor is described ggml-style by `View`: a host numpy buffer plus element
type, ne[4] (ne[0] fastest) and nb[4] (byte strides), exactly the fields the
C ABI's vxfa_tensor carries.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16 = 0, 1  # ggml's GGML_TYPE_F32 / GGML_TYPE_F16

VKQ_F16 = 1
MUT_GQA_MOD = 1 << 8
MUT_NO_MASK = 1 << 9
MUT_NO_SCALE = 1 << 10
MUT_V_SHIFT = 1 << 11
MUT_NO_MAXSUB = 1 << 12


class VxfaTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("type", ctypes.c_int32),
        ("pad_", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_size_t * 4),
    ]


@dataclass
class View:
    """A ggml tensor view over a host numpy buffer."""

    base: np.ndarray
    type: int
    ne: tuple
    nb: tuple
    offset: int = 0

    def desc(self) -> VxfaTensor:
        t = VxfaTensor()
        t.data = self.base.ctypes.data + self.offset
        t.type = self.type
        for i in range(4):
            t.ne[i] = int(self.ne[i])
            t.nb[i] = int(self.nb[i])
        return t


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER(VxfaTensor)
        L.oracle_fa_ggml.argtypes = [P, P, P, P, P, ctypes.c_float, ctypes.c_float,
                                     ctypes.c_float, ctypes.c_int, ctypes.c_int]
        L.oracle_fa_ggml.restype = ctypes.c_int
        L.oracle_fa_f64.argtypes = [P, P, P, P, ctypes.POINTER(ctypes.c_double), ctypes.c_float,
                                    ctypes.c_float, ctypes.c_float, ctypes.c_int, ctypes.c_int]
        L.oracle_fa_f64.restype = ctypes.c_int
        L.oracle_fa_cpu_simd.argtypes = [P, P, P, P, P, ctypes.c_float, ctypes.c_int]
        L.oracle_fa_cpu_simd.restype = ctypes.c_int
        L.oracle_f32_to_f16_array.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.oracle_f16_to_f32_array.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        _lib = L
    return _lib


def host_threads() -> int:
    """Hardware threads this process may run on (its CPU affinity set)."""
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except (AttributeError, OSError):
        return max(1, os.cpu_count() or 1)


def default_threads() -> int:
    """voxtral's default: min(hardware threads, 16) (src/voxtral.cpp:1046-1051)."""
    return max(1, min(host_threads(), 16))


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_f16_array(x.ctypes.data, out.ctypes.data, x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().oracle_f16_to_f32_array(h.ctypes.data, out.ctypes.data, h.size)
    return out


def _out_shape(q: View, v: View):
    # dst [DV, Hq, Nq, B] contiguous -> numpy [B, Nq, Hq, DV]
    return (int(q.ne[3]), int(q.ne[1]), int(q.ne[2]), int(v.ne[0]))


def fa_ggml(q: View, k: View, v: View, mask: View | None, scale: float,
            max_bias: float = 0.0, logit_softcap: float = 0.0,
            vkq_f16: bool = True, flags: int = 0, threads: int | None = None) -> np.ndarray:
    """ggml-faithful flash_attn_ext; returns float32 [B, Nq, Hq, DV]."""
    shape = _out_shape(q, v)
    out = np.zeros(shape, dtype=np.float32)
    DV, Hq, Nq, B = shape[3], shape[2], shape[1], shape[0]
    dst = View(out, F32, (DV, Hq, Nq, B), (4, 4 * DV, 4 * DV * Hq, 4 * DV * Hq * Nq))
    qd, kd, vd, dd = q.desc(), k.desc(), v.desc(), dst.desc()
    md = mask.desc() if mask is not None else None
    fl = flags | (VKQ_F16 if vkq_f16 else 0)
    rc = lib().oracle_fa_ggml(ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(vd),
                              ctypes.byref(md) if md is not None else None, ctypes.byref(dd),
                              scale, max_bias, logit_softcap, fl,
                              threads if threads else default_threads())
    if rc != 0:
        raise ValueError("oracle_fa_ggml: contract violation")
    return out


def fa_cpu_simd(q: View, k: View, v: View, mask: View | None, scale: float,
                threads: int | None = None, out: np.ndarray | None = None) -> np.ndarray:
    """ggml's one-row algorithm with its AVX2/F16C vector kernels (the timed
    CPU baseline); returns float32 [B, Nq, Hq, DV]."""
    shape = _out_shape(q, v)
    if out is None:
        out = np.zeros(shape, dtype=np.float32)
    DV, Hq, Nq, B = shape[3], shape[2], shape[1], shape[0]
    dst = View(out, F32, (DV, Hq, Nq, B), (4, 4 * DV, 4 * DV * Hq, 4 * DV * Hq * Nq))
    qd, kd, vd, dd = q.desc(), k.desc(), v.desc(), dst.desc()
    md = mask.desc() if mask is not None else None
    rc = lib().oracle_fa_cpu_simd(ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(vd),
                                  ctypes.byref(md) if md is not None else None, ctypes.byref(dd),
                                  scale, threads if threads else default_threads())
    if rc != 0:
        raise ValueError("oracle_fa_cpu_simd: contract violation")
    return out


def fa_f64(q: View, k: View, v: View, mask: View | None, scale: float,
           max_bias: float = 0.0, logit_softcap: float = 0.0, q_f16: bool = True,
           threads: int | None = None) -> np.ndarray:
    """Exact double-precision attention; returns float64 [B, Nq, Hq, DV]."""
    out = np.zeros(_out_shape(q, v), dtype=np.float64)
    qd, kd, vd = q.desc(), k.desc(), v.desc()
    md = mask.desc() if mask is not None else None
    rc = lib().oracle_fa_f64(ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(vd),
                             ctypes.byref(md) if md is not None else None,
                             out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
                             scale, max_bias, logit_softcap, 1 if q_f16 else 0,
                             threads if threads else default_threads())
    if rc != 0:
        raise ValueError("oracle_fa_f64: contract violation")
    return out
