"""ctypes binding of libvxfa.so, the C ABI declared in include/vxfa.h.

This is the Python face of the drop-in boundary: it builds the same
ggml-style tensor descriptors (type, ne[4], nb[4], data) that a ggml backend
would pass for a GGML_OP_FLASH_ATTN_EXT node, and calls the library. It holds
no compute of its own: when libvxfa.so is missing every entry point raises.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libvxfa.so")

F32, F16 = 0, 1  # equal to ggml's GGML_TYPE_F32 / GGML_TYPE_F16

OK, UNSUPPORTED, INVALID_ARG, NO_WORKSPACE, HIP_ERROR = 0, 1, 2, 3, 4

MASK_NONE, MASK_CAUSAL = 0, 1  # enum vxfa_mask_kind

# every symbol include/vxfa.h declares
EXPORTS = (
    "vxfa_ctx_create",
    "vxfa_ctx_destroy",
    "vxfa_supports",
    "vxfa_flash_attn_ext",
    "vxfa_check_mask_desc",
    "vxfa_flash_attn_ext_implicit",
    "vxfa_kv_append",
    "vxfa_flash_attn_ext_append",
    "vxfa_flash_attn_ext_ring",
    "vxfa_flash_attn_ext_rope",
    "vxfa_flash_attn_ext_noalloc",
    "vxfa_status_str",
    "vxfa_last_error",
    "vxfa_version",
)


class VxfaTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("type", ctypes.c_int32),
        ("pad_", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_size_t * 4),
    ]


class VxfaMaskDesc(ctypes.Structure):
    """vxfa_mask_desc: query row i attends kv j iff j <= i + offset and, for
    window > 0, j >= i + offset - window + 1."""
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("offset", ctypes.c_int64),
    ]


def mask_desc(kind: int = MASK_CAUSAL, window: int = 0, offset: int = 0) -> VxfaMaskDesc:
    m = VxfaMaskDesc()
    m.kind, m.window, m.offset = int(kind), int(window), int(offset)
    return m


class VxfaRing(ctypes.Structure):
    """vxfa_ring: logical position p lives in cache row (start + p) mod capacity."""
    _fields_ = [
        ("start", ctypes.c_int64),
        ("n_kv", ctypes.c_int64),
    ]


def ring(start: int, n_kv: int) -> VxfaRing:
    r = VxfaRing()
    r.start, r.n_kv = int(start), int(n_kv)
    return r


class VxfaRope(ctypes.Structure):
    """vxfa_rope: ggml_rope_ext mode 0 with freq_scale 1 (positions: device int32 pointer)."""
    _fields_ = [
        ("positions", ctypes.c_void_p),
        ("n_dims", ctypes.c_int32),
        ("mode", ctypes.c_int32),
        ("freq_base", ctypes.c_float),
        ("freq_scale", ctypes.c_float),
    ]


def rope(positions_ptr: int, n_dims: int, freq_base: float, mode: int = 0, freq_scale: float = 1.0) -> VxfaRope:
    r = VxfaRope()
    r.positions, r.n_dims, r.mode, r.freq_base, r.freq_scale = positions_ptr, n_dims, mode, freq_base, freq_scale
    return r


class VxfaError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"vxfa status {status} ({status_str(status)}): {msg}")
        self.status = status


_lib = None


def load() -> ctypes.CDLL:
    """Load libvxfa.so; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C {HERE}` "
                           "(or __graft_entry__.build()); there is no fallback path")
    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.POINTER(VxfaTensor)
    L.vxfa_ctx_create.argtypes = [ctypes.c_int]
    L.vxfa_ctx_create.restype = ctypes.c_void_p
    L.vxfa_ctx_destroy.argtypes = [ctypes.c_void_p]
    L.vxfa_ctx_destroy.restype = None
    L.vxfa_supports.argtypes = [P, P, P, P, P, ctypes.c_float, ctypes.c_float, ctypes.c_float]
    L.vxfa_supports.restype = ctypes.c_int
    L.vxfa_flash_attn_ext.argtypes = [ctypes.c_void_p, P, P, P, P, P, ctypes.c_float, ctypes.c_float,
                                      ctypes.c_float, ctypes.c_void_p]
    L.vxfa_flash_attn_ext.restype = ctypes.c_int
    M = ctypes.POINTER(VxfaMaskDesc)
    L.vxfa_check_mask_desc.argtypes = [M]
    L.vxfa_check_mask_desc.restype = ctypes.c_int
    L.vxfa_flash_attn_ext_implicit.argtypes = [ctypes.c_void_p, P, P, P, M, P, ctypes.c_float, ctypes.c_float,
                                               ctypes.c_float, ctypes.c_void_p]
    L.vxfa_flash_attn_ext_implicit.restype = ctypes.c_int
    L.vxfa_kv_append.argtypes = [ctypes.c_void_p, P, P, P, P, ctypes.c_void_p]
    L.vxfa_kv_append.restype = ctypes.c_int
    L.vxfa_flash_attn_ext_append.argtypes = [ctypes.c_void_p, P, P, P, P, P, P, P, ctypes.c_float, ctypes.c_float,
                                             ctypes.c_float, ctypes.c_void_p]
    L.vxfa_flash_attn_ext_append.restype = ctypes.c_int
    L.vxfa_flash_attn_ext_ring.argtypes = [ctypes.c_void_p, P, P, P, ctypes.POINTER(VxfaRing), P, P, P,
                                           ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_void_p]
    L.vxfa_flash_attn_ext_ring.restype = ctypes.c_int
    L.vxfa_flash_attn_ext_rope.argtypes = [ctypes.c_void_p, P, P, P, P, P, ctypes.POINTER(VxfaRope), P, P,
                                           ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_void_p]
    L.vxfa_flash_attn_ext_rope.restype = ctypes.c_int
    L.vxfa_flash_attn_ext_noalloc.argtypes = [P, P, P, P, P, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                              ctypes.c_void_p]
    L.vxfa_flash_attn_ext_noalloc.restype = ctypes.c_int
    L.vxfa_status_str.argtypes = [ctypes.c_int]
    L.vxfa_status_str.restype = ctypes.c_char_p
    L.vxfa_last_error.argtypes = [ctypes.c_void_p]
    L.vxfa_last_error.restype = ctypes.c_char_p
    L.vxfa_version.argtypes = []
    L.vxfa_version.restype = ctypes.c_int
    _lib = L
    return L


def status_str(status: int) -> str:
    try:
        return load().vxfa_status_str(status).decode()
    except RuntimeError:
        return str(status)


def desc(ptr: int, type_: int, ne, nb) -> VxfaTensor:
    """Descriptor of a ggml view: ptr (device address), type, ne[4], nb[4] (bytes)."""
    t = VxfaTensor()
    t.data = ptr
    t.type = type_
    for i in range(4):
        t.ne[i] = int(ne[i])
        t.nb[i] = int(nb[i])
    return t


def _ref(t):
    return ctypes.byref(t) if t is not None else None


def check_mask_desc(m) -> int:
    """Host-only validation of a mask descriptor (VxfaMaskDesc or None)."""
    return load().vxfa_check_mask_desc(_ref(m))


def flash_attn_ext_noalloc(q, k, v, mask, dst, scale: float, max_bias: float = 0.0, logit_softcap: float = 0.0,
                           stream: int = 0, check: bool = True) -> int:
    """vxfa_flash_attn_ext_noalloc: the op on the current device without a
    context; scratch in the library's static per-GPU array (calls that
    overlap on one GPU race)."""
    L = load()
    rc = L.vxfa_flash_attn_ext_noalloc(_ref(q), _ref(k), _ref(v), _ref(mask), _ref(dst), scale, max_bias,
                                       logit_softcap, ctypes.c_void_p(stream))
    if check and rc != OK:
        raise VxfaError(rc, L.vxfa_last_error(None).decode())
    return rc


def supports(q, k, v, mask, dst, scale: float, max_bias: float = 0.0, logit_softcap: float = 0.0) -> int:
    """Host-only capability check (ggml supports_op analogue)."""
    return load().vxfa_supports(_ref(q), _ref(k), _ref(v), _ref(mask), _ref(dst), scale, max_bias, logit_softcap)


class Context:
    """vxfa_ctx: one per stream; owns the split-KV workspace."""

    def __init__(self, device: int = 0):
        self._lib = load()
        self._h = self._lib.vxfa_ctx_create(device)
        if not self._h:
            raise RuntimeError(f"vxfa_ctx_create({device}) failed (no such HIP device?)")

    def flash_attn_ext(self, q, k, v, mask, dst, scale: float, max_bias: float = 0.0,
                       logit_softcap: float = 0.0, stream: int = 0, check: bool = True) -> int:
        rc = self._lib.vxfa_flash_attn_ext(self._h, _ref(q), _ref(k), _ref(v), _ref(mask), _ref(dst),
                                           scale, max_bias, logit_softcap, ctypes.c_void_p(stream))
        if check and rc != OK:
            raise VxfaError(rc, self.last_error())
        return rc

    def flash_attn_ext_implicit(self, q, k, v, mask_desc, dst, scale: float, max_bias: float = 0.0,
                                logit_softcap: float = 0.0, stream: int = 0, check: bool = True) -> int:
        """The op with an implicit causal / window mask (a VxfaMaskDesc, or None)."""
        rc = self._lib.vxfa_flash_attn_ext_implicit(self._h, _ref(q), _ref(k), _ref(v), _ref(mask_desc), _ref(dst),
                                                    scale, max_bias, logit_softcap, ctypes.c_void_p(stream))
        if check and rc != OK:
            raise VxfaError(rc, self.last_error())
        return rc

    def kv_append(self, k_new, v_new, k, v, stream: int = 0, check: bool = True) -> int:
        """F32 -> F16 append of new K/V rows into the last rows of the cache views k, v."""
        rc = self._lib.vxfa_kv_append(self._h, _ref(k_new), _ref(v_new), _ref(k), _ref(v), ctypes.c_void_p(stream))
        if check and rc != OK:
            raise VxfaError(rc, self.last_error())
        return rc

    def flash_attn_ext_append(self, q, k, v, k_new, v_new, mask, dst, scale: float, max_bias: float = 0.0,
                              logit_softcap: float = 0.0, stream: int = 0, check: bool = True) -> int:
        """kv_append then flash_attn_ext, fused for a single-token decode step."""
        rc = self._lib.vxfa_flash_attn_ext_append(self._h, _ref(q), _ref(k), _ref(v), _ref(k_new), _ref(v_new),
                                                  _ref(mask), _ref(dst), scale, max_bias, logit_softcap,
                                                  ctypes.c_void_p(stream))
        if check and rc != OK:
            raise VxfaError(rc, self.last_error())
        return rc

    def flash_attn_ext_ring(self, q, k, v, ring_desc, k_new, v_new, dst, scale: float, max_bias: float = 0.0,
                            logit_softcap: float = 0.0, stream: int = 0, check: bool = True) -> int:
        """A decode step over a ring-buffer cache (k_new / v_new: the step's new row, or None)."""
        rc = self._lib.vxfa_flash_attn_ext_ring(self._h, _ref(q), _ref(k), _ref(v), _ref(ring_desc), _ref(k_new),
                                                _ref(v_new), _ref(dst), scale, max_bias, logit_softcap,
                                                ctypes.c_void_p(stream))
        if check and rc != OK:
            raise VxfaError(rc, self.last_error())
        return rc

    def flash_attn_ext_rope(self, q, k, v, k_new, v_new, rope_desc, mask, dst, scale: float, max_bias: float = 0.0,
                            logit_softcap: float = 0.0, stream: int = 0, check: bool = True) -> int:
        """Rotate q and the new K rows (mode 0), append the new rows, attend."""
        rc = self._lib.vxfa_flash_attn_ext_rope(self._h, _ref(q), _ref(k), _ref(v), _ref(k_new), _ref(v_new),
                                                _ref(rope_desc), _ref(mask), _ref(dst), scale, max_bias,
                                                logit_softcap, ctypes.c_void_p(stream))
        if check and rc != OK:
            raise VxfaError(rc, self.last_error())
        return rc

    def last_error(self) -> str:
        return self._lib.vxfa_last_error(self._h).decode()

    def close(self) -> None:
        if self._h:
            self._lib.vxfa_ctx_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
