"""vxfa_flash_attn_ext_noalloc: the op with no context and no allocation,
its scratch in the library's static per-GPU array. Each call is checked
against vxfa_flash_attn_ext on the same device bytes (same kernels, same
split choice: identical bits) and, for the decode steps, against the oracle
at the parity bar; calls come in a row with the later ones smaller, so the
array keeps an earlier call's contents."""
import numpy as np
import pytest

import cases

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


@pytest.fixture(scope="module")
def runner():
    import gpu_util
    r = gpu_util.Runner()
    yield r
    r.close()


def _same(runner, c, oracle=False):
    import gpu_util
    dev = gpu_util.to_device(c)
    rc, ref = runner.run(c, dev=dev)
    assert rc == 0
    rc, out = runner.run_noalloc(c, dev=dev)
    assert rc == 0
    print(f"[noalloc] {c.name}: max |noalloc - ctx| = {float(np.abs(out - ref).max()):.3e}", flush=True)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    if oracle:
        m, r, ok = gpu_util.parity(out, cases.oracle_f64(c), ATOL, RTOL)
        assert ok, (m, r)


def test_noalloc_decode_then_smaller_decode(runner):
    """n_kv 8192 (64 split records in the scratch), then n_kv 1000 (16)."""
    _same(runner, cases.decode_case(8192, seed=301), oracle=True)
    _same(runner, cases.decode_case(1000, seed=302), oracle=True)


def test_noalloc_f32_cache_decode(runner):
    """The reference's F32 cache (F32 products, its split records in the
    scratch): n_kv 8192, then an hd 64 call with fewer splits."""
    _same(runner, cases.decode_case(8192, seed=317, kv_f32=True), oracle=True)
    _same(runner, cases.decode_case(700, hq=16, hkv=8, hd=64, seed=318, kv_f32=True), oracle=True)


def test_noalloc_batched_then_single(runner):
    _same(runner, cases.batched_case(16, capacity=2048, lo=100, hi=2048, seed=303))
    _same(runner, cases.decode_case(333, hq=16, hkv=8, hd=64, seed=304))


def test_noalloc_prefill_and_f32_staging(runner):
    """Causal prefill (no scratch), F32 encoder K/V (7.7 MB of f16 staging in
    the scratch), then a smaller F32 causal prefill (the short masked prefill
    whose mask row intervals, found in the staging launch, sit in the scratch
    after the staged K/V)."""
    _same(runner, cases.prefill_case(439, seed=305))
    _same(runner, cases.encoder_case(1500, 20, 64, seed=306, kv_f32=True))
    _same(runner, cases.prefill_case(100, seed=307, kv_f32=True))


def test_noalloc_mask_tensor_after_staging(runner):
    """hd 64 prefill with a mask tensor: the pre-pass's row intervals sit in
    the scratch after the f16 staging of F32 K/V (a context keeps them in its
    own region): the same bits either way, then a smaller masked call."""
    _same(runner, cases.encoder_case(600, 20, 64, seed=309, window=300, kv_f32=True), oracle=True)
    _same(runner, cases.encoder_case(200, 4, 64, seed=310, window=50), oracle=True)


def test_noalloc_rejects_staging_beyond_the_scratch(runner):
    """F32 K and V of 16384 rows x 8 x 128 need 64 MiB of f16 staging: beyond
    the 8 MiB scratch, the call returns VXFA_NO_WORKSPACE and launches nothing."""
    from conftest import load_package
    vx = load_package().vxfa
    c = cases.prefill_case(2, seed=308, causal=False, kv_offset=16382, kv_f32=True)
    rc, _ = runner.run_noalloc(c, check=False)
    assert rc == vx.NO_WORKSPACE
    msg = vx.load().vxfa_last_error(None).decode()
    assert "staging" in msg, msg


def test_noalloc_graph_capture_replays(runner):
    """No-alloc calls captured into a HIP graph, after eager no-alloc calls on
    the device (the first call on a device looks up the scratch, which may
    load the code object, so it is made outside capture): decode n_kv 8192
    (split records in the scratch), an F32 K/V prefill (f16 staging in the
    scratch) and an hd 64 F32 K/V prefill with a window mask tensor (staging
    and the mask pre-pass in one launch, the interval table after the staged
    K/V). Three replays, each followed by eager no-alloc calls of other
    shapes, match the eager bits."""
    import torch
    import gpu_util
    vx = gpu_util.vxfa
    cs = [cases.decode_case(8192, seed=311), cases.prefill_case(300, seed=312, kv_f32=True),
          cases.encoder_case(600, 8, 64, seed=316, window=300, kv_f32=True)]
    devs = [gpu_util.to_device(c) for c in cs]
    eager = []
    for c, d in zip(cs, devs):
        rc, ref = runner.run_noalloc(c, dev=d)
        assert rc == 0
        eager.append(ref)
    outs = []
    for c in cs:
        B, Nq, Hq, D = c.out_shape
        outs.append(torch.zeros(B * Nq * Hq * D, device="cuda", dtype=torch.float32))
    descs = [gpu_util.descs(c, d) for c, d in zip(cs, devs)]
    stream = torch.cuda.Stream()

    def step():
        for c, dd, o in zip(cs, descs, outs):
            ne, nb = c.dst_ne_nb()
            dst = vx.desc(o.data_ptr(), vx.F32, ne, nb)
            rc = vx.flash_attn_ext_noalloc(dd["q"], dd["k"], dd["v"], dd.get("mask"), dst, c.scale,
                                           stream=stream.cuda_stream)
            assert rc == 0

    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        step()
    torch.cuda.synchronize()
    others = [cases.decode_case(1000, seed=313), cases.batched_case(16, capacity=2048, lo=100, hi=2048, seed=314),
              cases.encoder_case(400, 20, 64, seed=315, kv_f32=True)]
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        with torch.cuda.stream(stream):
            g.replay()
        torch.cuda.synchronize()
        for o, ref, c in zip(outs, eager, cs):
            got = o.cpu().numpy().reshape(c.out_shape)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (rep, c.name)
        rc, _ = runner.run_noalloc(others[rep])
        assert rc == 0
