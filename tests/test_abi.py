"""The C ABI without a GPU: libvxfa.so loads, exports every function that
include/vxfa.h declares, and its host-only capability check (the supports_op
analogue) accepts voxtral.cpp's views and rejects what the path does not do.
No call here launches work or touches a device."""
import ctypes
import os
import re

import numpy as np
import pytest

import cases
from conftest import ROOT, load_package

vxfa = load_package().vxfa
views = load_package().views

HEADER = os.path.join(ROOT, "include", "vxfa.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vxfa_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_what_the_binding_binds():
    assert declared_functions() == sorted(vxfa.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = vxfa.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert ctypes.cast(getattr(lib, name), ctypes.c_void_p).value


def test_version_and_status_strings():
    lib = vxfa.load()
    assert lib.vxfa_version() >= 10000
    for s in (vxfa.OK, vxfa.UNSUPPORTED, vxfa.INVALID_ARG, vxfa.NO_WORKSPACE, vxfa.HIP_ERROR):
        assert lib.vxfa_status_str(s).decode() not in ("", "unknown status")
    assert lib.vxfa_status_str(99).decode() == "unknown status"
    assert lib.vxfa_last_error(None).decode() == ""


def test_struct_layout_matches_header():
    # void* data; int32 type; int32 pad_; int64 ne[4]; size_t nb[4]
    assert ctypes.sizeof(vxfa.VxfaTensor) == 8 + 4 + 4 + 32 + 32
    assert vxfa.VxfaTensor.ne.offset == 16 and vxfa.VxfaTensor.nb.offset == 48


ADDR = 1 << 20   # a 16-byte aligned fake device address: supports() never dereferences it


def descs(c):
    d = {}
    for role, (b, t, ne, nb, off) in c.views.items():
        d[role] = vxfa.desc(ADDR + off, t, ne, nb)
    B, Nq, Hq, D = c.out_shape
    d["dst"] = vxfa.desc(ADDR, vxfa.F32, *views.dst(D, Hq, Nq, B))
    return d


def supports(c, **over):
    d = descs(c)
    d.update({k: v for k, v in over.items() if k in d or k == "mask"})
    return vxfa.supports(d["q"], d["k"], d["v"], d.get("mask"), d["dst"], c.scale,
                         over.get("max_bias", 0.0), over.get("softcap", 0.0))


@pytest.mark.parametrize("make", [
    lambda: cases.decode_case(1024, seed=1),
    lambda: cases.decode_case(100, seed=1, window=10),
    lambda: cases.encoder_case(64, 20, 64, seed=1),
    lambda: cases.prefill_case(40, seed=1),
    lambda: cases.batched_case(4, capacity=64, lo=2, hi=64, seed=1),
    # the reference's own F32 cache and F32 encoder K/V (src/voxtral.cpp:1126-1136, :1581-1605)
    lambda: cases.decode_case(1024, seed=1, kv_f32=True),
    lambda: cases.encoder_case(64, 20, 64, seed=1, kv_f32=True),
    lambda: cases.prefill_case(40, seed=1, kv_f32=True),
])
def test_voxtral_views_are_supported(make):
    assert supports(make()) == vxfa.OK


def test_unsupported_features_report_unsupported():
    c = cases.decode_case(64, seed=2)
    assert supports(c, max_bias=8.0) == vxfa.UNSUPPORTED
    assert supports(c, softcap=30.0) == vxfa.UNSUPPORTED
    d = descs(c)
    # F32 K with f16 V: mixed K/V types are not implemented
    k32 = vxfa.desc(ADDR, vxfa.F32, d["k"].ne, [4, 4096, 512, 4096 * 64])
    assert vxfa.supports(d["q"], k32, d["v"], None, d["dst"], c.scale) == vxfa.UNSUPPORTED
    v32 = vxfa.desc(ADDR, vxfa.F32, d["v"].ne, [4, 4096, 512, 4096 * 64])
    assert vxfa.supports(d["q"], k32, v32, None, d["dst"], c.scale) == vxfa.OK
    # head dim 96 is a valid op but not one this path implements
    c96 = cases.decode_case(64, hq=4, hkv=1, hd=96, seed=3)
    assert supports(c96) == vxfa.UNSUPPORTED


def test_contract_violations_report_invalid():
    c = cases.decode_case(64, hq=8, hkv=2, seed=4)
    d = descs(c)
    bad_k = vxfa.desc(ADDR, vxfa.F16, (128, 64, 3, 1), d["k"].nb)          # 8 % 3 != 0
    bad_v = vxfa.desc(ADDR, vxfa.F16, (128, 63, 2, 1), d["v"].nb)          # n_kv mismatch
    bad_dst = vxfa.desc(ADDR, vxfa.F32, (128, 1, 8, 1), (4, 512, 512, 4096))  # not permuted
    assert vxfa.supports(d["q"], bad_k, d["v"], None, d["dst"], c.scale) == vxfa.INVALID_ARG
    assert vxfa.supports(d["q"], d["k"], bad_v, None, d["dst"], c.scale) == vxfa.INVALID_ARG
    assert vxfa.supports(d["q"], d["k"], d["v"], None, bad_dst, c.scale) == vxfa.INVALID_ARG
    short_mask = vxfa.desc(ADDR, vxfa.F16, (63, 1, 1, 1), (2, 126, 126, 126))
    assert vxfa.supports(d["q"], d["k"], d["v"], short_mask, d["dst"], c.scale) == vxfa.INVALID_ARG
    assert vxfa.supports(None, d["k"], d["v"], None, d["dst"], c.scale) == vxfa.INVALID_ARG


def test_unaligned_views_are_unsupported_not_invalid():
    c = cases.decode_case(64, seed=5)
    d = descs(c)
    q_odd = vxfa.desc(ADDR + 4, vxfa.F32, d["q"].ne, d["q"].nb)
    assert vxfa.supports(q_odd, d["k"], d["v"], None, d["dst"], c.scale) == vxfa.UNSUPPORTED


def test_unpadded_odd_mask_rows_are_accepted():
    """voxtral passes an unpadded [n, n] mask (src/voxtral.cpp:2024, :1880):
    439-wide rows are 878 bytes, not 16-byte aligned."""
    c = cases.prefill_case(439, seed=6)
    assert c.views["mask"][3][1] == 878
    assert supports(c) == vxfa.OK


def test_zero_sized_query_is_accepted():
    c = cases.decode_case(16, seed=7)
    b, t, ne, nb, off = c.views["q"]
    c.views["q"] = (b, t, (ne[0], ne[1], ne[2], 0), nb, off)
    assert supports(c) == vxfa.OK


# --- implicit masks (vxfa_flash_attn_ext_implicit) ----------------------------

def test_mask_desc_layout_matches_header():
    # int32 kind; int32 window; int64 offset
    assert ctypes.sizeof(vxfa.VxfaMaskDesc) == 16
    assert vxfa.VxfaMaskDesc.window.offset == 4 and vxfa.VxfaMaskDesc.offset.offset == 8


def test_mask_desc_validation():
    assert vxfa.check_mask_desc(None) == vxfa.OK
    assert vxfa.check_mask_desc(vxfa.mask_desc(vxfa.MASK_NONE)) == vxfa.OK
    assert vxfa.check_mask_desc(vxfa.mask_desc(vxfa.MASK_CAUSAL, 0, 0)) == vxfa.OK
    assert vxfa.check_mask_desc(vxfa.mask_desc(vxfa.MASK_CAUSAL, 750, -5)) == vxfa.OK
    assert vxfa.check_mask_desc(vxfa.mask_desc(2)) == vxfa.INVALID_ARG
    assert vxfa.check_mask_desc(vxfa.mask_desc(vxfa.MASK_CAUSAL, -1, 0)) == vxfa.INVALID_ARG


def test_implicit_entry_rejects_a_null_context():
    # returns before any HIP call
    lib = vxfa.load()
    m = vxfa.mask_desc()
    assert lib.vxfa_flash_attn_ext_implicit(None, None, None, None, ctypes.byref(m), None,
                                            0.125, 0.0, 0.0, None) == vxfa.INVALID_ARG


def test_implicit_mask_formula_matches_voxtral_masks():
    """The descriptor's formula reproduces the masks voxtral.cpp fills:
    fill_causal_mask (src/voxtral.cpp:2104-2111, built by prefill_case), the
    realtime encoder window (:2179-2190, built by encoder_case), the decode
    window of the streaming workload (built by decode_case) and a causal
    prefill against a filled cache (kv_offset rows before the chunk)."""
    def mask_of(c):
        b, _, ne, _, _ = c.views["mask"]
        return c.bufs[b].reshape(-1, ne[0])
    n = 75
    assert np.array_equal(cases.implicit_mask(n, n, 0), mask_of(cases.prefill_case(n, hq=4, hkv=1, hd=64)))
    pc = cases.prefill_case(20, hq=4, hkv=1, hd=64, kv_offset=33)
    assert np.array_equal(cases.implicit_mask(20, 53, 33), mask_of(pc))
    ec = cases.encoder_case(90, 2, 64, window=17)
    assert np.array_equal(cases.implicit_mask(90, 90, 0, 17), mask_of(ec))
    dc = cases.decode_case(300, hq=4, hkv=1, hd=64, window=64)
    assert np.array_equal(cases.implicit_mask(1, 300, 299, 64), mask_of(dc))
    # closed forms: window 1 keeps only the diagonal; a negative offset empties the first rows
    assert (cases.implicit_mask(8, 8, 0, 1) == 0).sum() == 8
    m = cases.implicit_mask(8, 8, -3)
    assert (m[:3] == cases.NEG_INF_F16).all() and (m[3] == 0).sum() == 1


def test_append_entries_reject_a_null_context():
    lib = vxfa.load()
    assert lib.vxfa_kv_append(None, None, None, None, None, None) == vxfa.INVALID_ARG
    assert lib.vxfa_flash_attn_ext_append(None, None, None, None, None, None, None, None,
                                          0.1, 0.0, 0.0, None) == vxfa.INVALID_ARG


def test_ring_struct_and_null_context():
    assert ctypes.sizeof(vxfa.VxfaRing) == 16 and vxfa.VxfaRing.n_kv.offset == 8
    lib = vxfa.load()
    r = vxfa.ring(0, 1)
    assert lib.vxfa_flash_attn_ext_ring(None, None, None, None, ctypes.byref(r), None, None, None,
                                        0.1, 0.0, 0.0, None) == vxfa.INVALID_ARG


def test_rope_struct_and_null_context():
    # const int32_t* positions; int32 n_dims; int32 mode; float freq_base; float freq_scale
    assert ctypes.sizeof(vxfa.VxfaRope) == 24 and vxfa.VxfaRope.freq_base.offset == 16
    lib = vxfa.load()
    r = vxfa.rope(0, 128, 1e6)
    assert lib.vxfa_flash_attn_ext_rope(None, None, None, None, None, None, ctypes.byref(r), None, None,
                                        0.1, 0.0, 0.0, None) == vxfa.INVALID_ARG


def test_rope_restatement_closed_forms():
    """Position 0 leaves vectors unchanged; one pair at position p turns by p
    radians (theta_0 = p); the rotation keeps each pair's norm."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 2, 8)).astype(np.float32)
    y = cases.rope_ggml(x, [0, 1, 7], 8, 10000.0)
    assert np.array_equal(y[0], x[0])
    c, s = np.cos(1.0), np.sin(1.0)
    assert np.allclose(y[1, :, 0], x[1, :, 0] * c - x[1, :, 1] * s, atol=1e-6)
    n0 = np.hypot(x[..., 0::2], x[..., 1::2])
    n1 = np.hypot(y[..., 0::2], y[..., 1::2])
    assert np.allclose(n0, n1, rtol=1e-5)
    ts = cases._powf(10000.0, np.float32(-2.0) / np.float32(8))
    assert abs(float(ts) - 10000.0 ** (-0.25)) < 1e-7


def test_ggml_binding_loads_and_declines_without_a_gpu():
    """The ggml-side binding (tests/ggml_binding/binding.c, compiled as C by
    the build) links against libvxfa.so and loads; its supports_op declines
    a node with attention sinks before any device access."""
    path = os.path.join(ROOT, "tests", "ggml_binding", "libvxfa_ggml_binding.so")
    if not os.path.exists(path):
        pytest.skip("the binding library is built by __graft_entry__.build()")
    lib = ctypes.CDLL(path)
    f = lib.vxfa_test_decoder_node
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 8 + [ctypes.c_void_p] * 2 + [ctypes.c_int]
    buf = (ctypes.c_float * 4096)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    assert f(None, None, p, p, p, 30, 8192, 0, 32, 8, 128, 1, 16, None, p, 1) == 0
