"""The ggml-side binding, compiled as C (tests/ggml_binding/binding.c against
ggml_min.h, linked to libvxfa.so), driven through the nodes voxtral.cpp's
decoder builds (src/voxtral.cpp:1772-1802) on the reference's own F32 KV
cache (kv_self_k / kv_self_v [1024, 8192, 30], :1126-1136):

  * 30 decoder layers of one decode step at n_kv 8192 (no mask), every node
    through backend_supports_flash_attn_ext and backend_flash_attn_ext on
    one stream, then checked against the oracle layer by layer;
  * a causal prefill of 339 tokens after 100 cached rows (n_kv 439, the F16
    causal mask of fill_causal_mask, :2104-2111, cast at :1801);
  * supports_op declines a node with attention sinks (src[4]) and one with a
    head dim the path does not implement, without touching the GPU.
"""
import ctypes
import os

import numpy as np
import pytest

import cases
from oracle import oracle

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "tests", "ggml_binding", "libvxfa_ggml_binding.so")
LAYERS, WINDOW, HQ, HKV, HD = 30, 8192, 32, 8, 128


@pytest.fixture(scope="module")
def env():
    import torch
    import gpu_util
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(LIB)
    f = lib.vxfa_test_decoder_node
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 8 + [ctypes.c_void_p] * 2 + [ctypes.c_int]
    ctx = gpu_util.vxfa.Context(0)
    g = torch.Generator(device="cuda")
    g.manual_seed(1234)
    kc = torch.randn((LAYERS, WINDOW, HKV * HD), device="cuda", generator=g, dtype=torch.float32)
    vc = torch.randn((LAYERS, WINDOW, HKV * HD), device="cuda", generator=g, dtype=torch.float32)
    yield f, ctx, kc, vc
    ctx.close()


def _call(f, ctx, kc, vc, layer, q, n_tokens, n_kv, mask, dst, sinks=0, head_dim=HD):
    import torch
    return f(ctypes.c_void_p(ctx._h), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
             ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(kc.data_ptr()), ctypes.c_void_p(vc.data_ptr()),
             LAYERS, WINDOW, layer, HQ, HKV, head_dim, n_tokens, n_kv,
             ctypes.c_void_p(mask.data_ptr() if mask is not None else None), ctypes.c_void_p(dst.data_ptr()), sinks)


def _oracle_case(q, k_layer, v_layer, n_tokens, n_kv, mask):
    """The node's views (the ggml reshape/permute of the driver) over host
    copies: q [128, n, 32] of a [4096, n] buffer, k/v [128, n_kv, 8] of the
    layer's [1024, 8192] cache slice, mask [n_kv, n]."""
    c = cases.Case(f"ggml_node_n{n_tokens}_nkv{n_kv}", cases.f32(1.0 / np.sqrt(HD)))
    c.add("q", "q", q, oracle.F32, (HD, n_tokens, HQ, 1), (4, 4 * HQ * HD, 4 * HD, 4 * HQ * HD * n_tokens))
    kvnb = (4, 4 * HKV * HD, 4 * HD, 4 * HKV * HD * n_kv)
    c.add("k", "k", k_layer, oracle.F32, (HD, n_kv, HKV, 1), kvnb)
    c.add("v", "v", v_layer, oracle.F32, (HD, n_kv, HKV, 1), kvnb)
    if mask is not None:
        c.add("mask", "mask", mask, oracle.F16, (n_kv, n_tokens, 1, 1), (2, 2 * n_kv, 2 * n_kv * n_tokens,
                                                                         2 * n_kv * n_tokens))
    return c


def _check(out, c, tag):
    import gpu_util
    for ref in (cases.oracle_ggml(c), cases.oracle_f64(c)):
        mx, r, ok = gpu_util.parity(out, ref, ATOL, RTOL)
        assert ok, (tag, mx, r)
    return mx


def test_binding_thirty_decode_layers_f32_cache(env):
    import torch
    f, ctx, kc, vc = env
    g = torch.Generator(device="cuda")
    g.manual_seed(99)
    qs = torch.randn((LAYERS, HQ * HD), device="cuda", generator=g, dtype=torch.float32)
    dst = torch.full((LAYERS, HQ * HD), float("nan"), device="cuda", dtype=torch.float32)
    for layer in range(LAYERS):
        rc = _call(f, ctx, kc, vc, layer, qs[layer], 1, WINDOW, None, dst[layer])
        assert rc == 1, (layer, rc, ctx.last_error())
    torch.cuda.synchronize()
    out_all = dst.cpu().numpy()
    q_all = qs.cpu().numpy()
    worst = 0.0
    for layer in range(LAYERS):
        c = _oracle_case(q_all[layer], kc[layer].cpu().numpy(), vc[layer].cpu().numpy(), 1, WINDOW, None)
        worst = max(worst, _check(out_all[layer].reshape(c.out_shape), c, f"layer {layer}"))
    print(f"[ggml binding] 30 decode layers, F32 cache n_kv 8192: max |gpu - f64 oracle| = {worst:.3e}", flush=True)


def test_binding_causal_prefill_f32_cache(env):
    import torch
    f, ctx, kc, vc = env
    n, off, layer = 339, 100, 5
    n_kv = off + n
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    q = torch.randn((n, HQ * HD), device="cuda", generator=g, dtype=torch.float32)
    m = np.where(np.arange(n_kv)[None, :] <= np.arange(n)[:, None] + off, 0, cases.NEG_INF_F16).astype(np.uint16)
    dm = torch.from_numpy(m.view(np.int16)).cuda()
    dst = torch.full((n, HQ * HD), float("nan"), device="cuda", dtype=torch.float32)
    rc = _call(f, ctx, kc, vc, layer, q, n, n_kv, dm, dst)
    assert rc == 1, (rc, ctx.last_error())
    torch.cuda.synchronize()
    c = _oracle_case(q.cpu().numpy(), kc[layer, :n_kv].cpu().numpy(), vc[layer, :n_kv].cpu().numpy(), n, n_kv, m)
    mx = _check(dst.cpu().numpy().reshape(c.out_shape), c, "prefill")
    print(f"[ggml binding] causal prefill 339 after 100 rows, F32 cache: max |gpu - f64 oracle| = {mx:.3e}",
          flush=True)


def test_binding_supports_op_declines(env):
    import torch
    f, ctx, kc, vc = env
    q = torch.zeros(HQ * HD, device="cuda", dtype=torch.float32)
    dst = torch.zeros(HQ * HD, device="cuda", dtype=torch.float32)
    assert _call(f, ctx, kc, vc, 0, q, 1, 16, None, dst, sinks=1) == 0
    assert _call(f, ctx, kc, vc, 0, q, 1, 16, None, dst, head_dim=80) == 0
