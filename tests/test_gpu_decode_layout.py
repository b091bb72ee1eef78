"""GPU: decode with its K tiles read as whole rows and turned through LDS
into the MFMA operand layout, over split counts, and graph capture of calls
that use the split-KV records.

  * Every decode variant (plain f16 and F32 caches, head dims 64 and 128, GQA
    groups 1, 2, 4, a mask tensor, ragged batches, F16 q) at split counts 1
    (the split kernel writes the output itself), 3 and 64 (VXFA_DECODE_SPLIT)
    and the default choice, each within the parity bar of the float64
    oracle.
  * HIP graphs: decode calls with 64 and 8 split records per (batch, kv head)
    and an F32 K/V prefill (f16 staging in the workspace) captured once and
    replayed three times, with eager calls of other shapes between the
    replays, replay to the eager bits.
"""
import contextlib
import os
import sys

import numpy as np
import pytest

import cases

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@contextlib.contextmanager
def _env(**kw):
    old = {k: os.environ.get(k) for k in kw}
    os.environ.update({k: str(v) for k, v in kw.items()})
    try:
        yield
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


@pytest.fixture(scope="module")
def runners():
    """the default context and contexts with 1, 3 and 64 decode splits (the
    environment is read when a context is created)"""
    import gpu_util
    rs = {"default": gpu_util.Runner()}
    for n in (1, 3, 64):
        with _env(VXFA_DECODE_SPLIT=n):
            rs[n] = gpu_util.Runner()
    yield rs
    for r in rs.values():
        r.close()


def _oracle_ok(out, c):
    import gpu_util
    m, r, ok = gpu_util.parity(out, cases.oracle_f64(c), ATOL, RTOL)
    _say(f"    vs f64 maxabs={m:.3e} rel={r:.3e}")
    return ok


DECODE_CASES = {
    "nkv8192": lambda: cases.decode_case(8192, seed=501),
    "nkv77": lambda: cases.decode_case(77, seed=503),
    "nkv5000_hd64_g2": lambda: cases.decode_case(5000, hq=16, hkv=8, hd=64, seed=504),
    "nkv3000_g1": lambda: cases.decode_case(3000, hq=8, hkv=8, seed=505),
    "nkv999_hd64_g4": lambda: cases.decode_case(999, hq=8, hkv=2, hd=64, seed=506),
    "f32_cache_4096": lambda: cases.decode_case(4096, seed=507, kv_f32=True),
    "f32_cache_300_hd64": lambda: cases.decode_case(300, hq=16, hkv=4, hd=64, seed=508, kv_f32=True),
    "window_mask_8k": lambda: cases.decode_case(8192, seed=509, window=1000),
    "batch4_ragged": lambda: cases.batched_case(4, capacity=4096, lo=100, hi=4096, seed=510),
    "q_f16_batch2": lambda: cases.decode_case(2500, seed=512, batch=2, q_f16=True),
}


@pytest.mark.parametrize("splits", ["default", 1, 3, 64])
@pytest.mark.parametrize("name", sorted(DECODE_CASES))
def test_decode_split_counts(runners, name, splits):
    c = DECODE_CASES[name]()
    _say(f"[case] {name} splits={splits}")
    rc, out = runners[splits].run(c)
    assert rc == 0
    assert _oracle_ok(out, c)


def test_graph_capture_with_split_records(runners):
    """decode n_kv 8192 (64 records per pair), n_kv 1024 (8), an F32 K/V
    prefill (staging) and an hd 64 F32 K/V prefill with a window mask tensor
    (staging and the mask pre-pass in one launch, the interval table in the
    record region) captured together; replayed three times with eager calls
    of other shapes between the replays"""
    import torch
    import gpu_util
    r = runners["default"]
    cs = [cases.decode_case(8192, seed=541), cases.decode_case(1024, seed=542),
          cases.prefill_case(200, seed=543, kv_f32=True),
          cases.encoder_case(500, 8, 64, seed=544, window=200, kv_f32=True)]
    devs = [gpu_util.to_device(c) for c in cs]
    eager = []
    outs = []
    for c, d in zip(cs, devs):
        rc, ref = r.run(c, dev=d)
        assert rc == 0
        eager.append(ref)
        B, Nq, Hq, D = c.out_shape
        outs.append(torch.zeros(B * Nq * Hq * D, device="cuda", dtype=torch.float32))
    descs = [gpu_util.descs(c, d) for c, d in zip(cs, devs)]
    stream = torch.cuda.Stream()

    def step():
        for c, dd, o in zip(cs, descs, outs):
            ne, nb = c.dst_ne_nb()
            dst = gpu_util.vxfa.desc(o.data_ptr(), gpu_util.vxfa.F32, ne, nb)
            rc = r.ctx.flash_attn_ext(dd["q"], dd["k"], dd["v"], dd.get("mask"), dst, c.scale,
                                      stream=stream.cuda_stream)
            assert rc == 0

    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        step()
    torch.cuda.synchronize()
    others = [cases.batched_case(32, capacity=2048, lo=512, hi=2048, seed=544), cases.decode_case(3000, seed=545),
              cases.encoder_case(300, 20, 64, seed=546, kv_f32=True)]
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        with torch.cuda.stream(stream):
            g.replay()
        torch.cuda.synchronize()
        for o, ref, c in zip(outs, eager, cs):
            got = o.cpu().numpy().reshape(c.out_shape)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (rep, c.name)
        rc, _ = r.run(others[rep], verify_inputs=False)   # eager work between replays
        assert rc == 0
