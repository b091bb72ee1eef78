"""GPU parity: the HIP path through the C ABI against the CPU oracle.

Tolerance (the stated bar for this op): max-abs <= 2e-3 and relative
Frobenius error <= 1e-2, against the ggml-faithful restatement with fp32
accumulation and against the exact float64 reference; besides, every output
element of at least 5% of the largest magnitude is within 1e-2 relative
(gpu_util.elem_rel). The ggml one-row kernel's f16 V accumulator is checked
as a bracket: the GPU result may not be further from it than that mode is
from exact, plus 2e-3.
"""
import sys

import numpy as np
import pytest

import cases
import golden_util
from oracle import oracle

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


@pytest.fixture(scope="module")
def runner():
    import gpu_util
    r = gpu_util.Runner()
    yield r
    r.close()


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def check_case(runner, c, bracket=False, dev=None):
    import gpu_util
    _say(f"[case] {c.name} views={ {k: v[2] for k, v in c.views.items()} }")
    rc, out = runner.run(c, dev=dev)
    assert rc == 0
    ref = cases.oracle_ggml(c)
    exact = cases.oracle_f64(c)
    m1, r1, ok1 = gpu_util.parity(out, ref, ATOL, RTOL)
    m2, r2, ok2 = gpu_util.parity(out, exact, ATOL, RTOL)
    _say(f"    vs ggml-fp32 maxabs={m1:.3e} rel={r1:.3e} elem={gpu_util.elem_rel(out, ref):.3e}; "
         f"vs f64 maxabs={m2:.3e} rel={r2:.3e} elem={gpu_util.elem_rel(out, exact):.3e}")
    assert np.isfinite(out).all()
    assert ok1, (m1, r1)
    assert ok2, (m2, r2)
    if bracket:
        g16 = cases.oracle_ggml(c, vkq_f16=True)
        own = np.abs(g16.astype(np.float64) - exact)
        assert (np.abs(out - g16) <= own + ATOL).all()
    return out


# --- the five workloads at full size ------------------------------------------

def test_decode_nkv1024(runner):
    check_case(runner, cases.decode_case(1024, seed=11), bracket=True)


def test_decode_nkv8192(runner):
    check_case(runner, cases.decode_case(8192, capacity=8192, seed=12), bracket=True)


def test_encoder_prefill_1500x20_hd64(runner):
    check_case(runner, cases.encoder_case(1500, 20, 64, seed=13), bracket=True)


def test_decoder_prefill_439_causal(runner):
    check_case(runner, cases.prefill_case(439, seed=14), bracket=True)


def test_sliding_window_decode_100_steps(runner):
    """Cache of 16384 rows, window 2048, one appended row per step (config 4)."""
    import torch
    import gpu_util
    cap, n0, window, steps = 16384, 16284, 2048, 100
    rng = np.random.default_rng(15)
    base = cases.decode_case(n0, capacity=cap, seed=16)
    dev = gpu_util.to_device(base)
    worst = 0.0
    for t in range(steps):
        n_kv = n0 + t + 1
        # append the new K/V row at position n0 + t (host and device)
        for name in ("k", "v"):
            row = cases.f16_bits(cases.normal(rng, (8, 128)))
            base.bufs[name].reshape(cap, 8, 128)[n0 + t] = row
            dev[name].view(torch.int16).view(cap, 8, 128)[n0 + t] = torch.from_numpy(row.view(np.int16)).to("cuda")
        q = cases.normal(rng, (1, 1, 32, 128))
        base.bufs["q"][...] = q
        dev["q"].copy_(torch.from_numpy(q.view(np.uint8).reshape(-1)).to("cuda"))
        m = np.zeros((1, 1, n_kv), dtype=np.uint16)
        m[..., : n_kv - window] = cases.NEG_INF_F16
        c = cases.Case(f"sliding_step{t}", base.scale, bufs=dict(base.bufs), views=dict(base.views))
        ne, nb = cases.views.kv_cache(n_kv, 8, 128, cap)
        c.views["k"] = ("k", oracle.F16, ne, nb, 0)
        c.views["v"] = ("v", oracle.F16, ne, nb, 0)
        c.bufs["mask"] = m
        c.views["mask"] = ("mask", oracle.F16) + cases.views.mask(n_kv, 1) + (0,)
        d2 = dict(dev)
        d2["mask"] = gpu_util.guarded(m)
        rc, out = runner.run(c, dev=d2, verify_inputs=(t == steps - 1))
        ref = cases.oracle_ggml(c)
        m1, r1, ok = gpu_util.parity(out, ref, ATOL, RTOL)
        worst = max(worst, m1)
        assert ok, (t, m1, r1)
    _say(f"    sliding window: worst maxabs over {steps} steps = {worst:.3e}")


def test_batched_ragged_32_streams(runner):
    c = cases.batched_case(32, seed=17)
    _say(f"    lengths {c.meta['lens'].tolist()}")
    check_case(runner, c)


# --- the committed fixtures (expected = torch float64 SDPA) --------------------

@pytest.mark.parametrize("name", golden_util.names())
def test_golden_fixture(runner, name):
    import gpu_util
    c, want = golden_util.load(name)
    _say(f"[golden] {name}")
    rc, out = runner.run(c)
    assert rc == 0
    m, r, ok = gpu_util.parity(out, want, ATOL, RTOL)
    _say(f"    maxabs={m:.3e} rel={r:.3e}")
    assert ok, (m, r)


# --- contract edge cases --------------------------------------------------------

@pytest.mark.parametrize("n_kv", [1, 2, 15, 16, 17, 31, 33, 63, 64, 65, 127, 129, 1000, 4097])
def test_decode_lengths(runner, n_kv):
    check_case(runner, cases.decode_case(n_kv, capacity=n_kv + 7, seed=100 + n_kv))


@pytest.mark.parametrize("hq,hkv,hd", [(32, 32, 128), (16, 8, 128), (8, 2, 64), (20, 20, 64), (32, 4, 128)])
def test_decode_groups(runner, hq, hkv, hd):
    # G = 1, 2, 4 use the decode kernel; G = 8 goes through the prefill kernel
    check_case(runner, cases.decode_case(777, hq, hkv, hd, seed=hq * 7 + hkv))


def test_decode_q_f16(runner):
    check_case(runner, cases.decode_case(300, seed=21, q_f16=True))


def test_decode_window_small(runner):
    check_case(runner, cases.decode_case(5000, window=100, seed=22))


@pytest.mark.parametrize("n,off", [(1, 0), (2, 0), (33, 0), (64, 0), (65, 0), (200, 57), (128, 1000)])
def test_prefill_causal_shapes(runner, n, off):
    check_case(runner, cases.prefill_case(n, kv_offset=off, seed=200 + n + off))


def test_prefill_no_mask_gqa(runner):
    check_case(runner, cases.prefill_case(300, causal=False, seed=23))


def _sparse_mask(rng, nq, nkv):
    """-inf everywhere but a few live entries per row, many on the first and
    last entries of 8-entry groups (where a row's 16-byte chunks straddle
    64-entry tiles), a fully zero 32 x 64 block, and rows with no live entry."""
    m = np.full((nq, nkv), cases.NEG_INF_F16, dtype=np.uint16)
    live_vals = cases.f16_bits(np.array([0.0, 0.0, -1.5, 0.25], dtype=np.float32))
    for i in range(nq):
        if i % 11 == 5:
            continue                      # row without a live entry: output 0
        cols = set(rng.integers(0, nkv, size=int(rng.integers(1, 4))).tolist())
        for t in range(0, nkv, 64):       # tile edges and 8-entry group edges
            for c in (t, t + 7, t + 8, t + 63):
                if c < nkv and rng.random() < 0.15:
                    cols.add(c)
        cols.add(nkv - 1) if rng.random() < 0.3 else None
        for c in cols:
            m[i, c] = live_vals[int(rng.integers(0, len(live_vals)))]
    r1, c1 = min(32, nq), min(64, nkv)
    m[:r1, :c1] = 0                       # a tile whose entries are all zero
    return m


@pytest.mark.parametrize("n,nkv,hq,hkv,hd", [(71, 133, 32, 8, 128), (129, 511, 32, 8, 128), (64, 65, 32, 8, 128),
                                           (100, 257, 20, 20, 64), (33, 1001, 16, 8, 128)])
def test_prefill_sparse_mask_scan(runner, n, nkv, hq, hkv, hd):
    """The prefill mask scan's tile classes and live range on unpadded rows of
    odd length (every row misaligned differently), isolated live entries at
    chunk and tile edges, a partial last tile and a partial last row block;
    compared with the oracle on the same mask."""
    rng = np.random.default_rng(1000 + n + nkv)
    c = cases.prefill_case(n, hq=hq, hkv=hkv, hd=hd, causal=False, kv_offset=nkv - n, seed=900 + n,
                           name=f"sparse_mask_n{n}_kv{nkv}_hd{hd}")
    check_case(runner, cases.with_mask(c, _sparse_mask(rng, n, nkv)))


@pytest.mark.parametrize("seq", [1, 31, 100, 750, 1501])
def test_encoder_shapes(runner, seq):
    check_case(runner, cases.encoder_case(seq, 4, 64, seed=300 + seq))


@pytest.mark.parametrize("seq", [32, 64, 96, 128, 161, 1024])
def test_encoder_block_splits(runner, seq):
    """hd 64 unmasked prefill: KV ranges that leave KV groups of a workgroup
    empty (32, 64, 96), exact multiples of the 32-position block (no partial
    block), and short groups next to full ones (161)."""
    check_case(runner, cases.encoder_case(seq, 3, 64, seed=500 + seq))


def test_encoder_rising_maxima(runner):
    """Key norms grow along the KV axis (up to 5x), so the running row max is
    raised in many blocks: the rescale path of the pipelined softmax."""
    check_case(runner, cases.encoder_case(700, 4, 64, seed=26, k_ramp=4.0, q_sigma=2.0))


def test_encoder_negative_and_f16_q(runner):
    check_case(runner, cases.encoder_case(300, 4, 64, seed=27, scale=-0.125))
    check_case(runner, cases.encoder_case(300, 4, 64, seed=28, q_f16=True))


def test_encoder_zero_scale(runner):
    """scale 0: every unmasked position weighs the same (mean of V)."""
    check_case(runner, cases.encoder_case(200, 2, 64, seed=29, scale=0.0))


def test_prefill_hd64_gqa_no_mask(runner):
    check_case(runner, cases.prefill_case(257, hq=8, hkv=2, hd=64, causal=False, seed=30))


def test_encoder_realtime_window(runner):
    """realtime encoder: sliding-causal window 750 (src/voxtral.cpp:2179-2190)"""
    check_case(runner, cases.encoder_case(1000, 4, 64, seed=24, window=750))


def test_realtime_encoder_full_size(runner):
    """The realtime encoder's attention at its real shape: 1500 frames x 32
    heads, hd 64, the 750 sliding-causal window as the F16 mask tensor
    voxtral fills (3000-byte rows: not 16-byte aligned), as the implicit mask
    (same bits as the tensor), and with F32 K/V as the application passes them
    (src/voxtral.cpp:1580-1611, mask :2179-2190, cast :1564)."""
    from conftest import load_package
    vx = load_package().vxfa
    import gpu_util
    c = cases.encoder_case(1500, 32, 64, seed=25, window=750)
    out = check_case(runner, c)
    rc, imp = runner.run_implicit(c, vx.mask_desc(vx.MASK_CAUSAL, 750, 0))
    assert rc == 0
    if HD64_MASK_BITWISE:
        assert np.array_equal(imp.view(np.uint32), out.view(np.uint32))
    mx, r, ok = gpu_util.parity(imp, cases.oracle_f64(c), ATOL, RTOL)
    assert ok, (mx, r)
    check_case(runner, cases.encoder_case(1500, 32, 64, seed=26, window=750, kv_f32=True))


def test_fully_masked_rows_are_zero(runner):
    c = cases.prefill_case(70, hq=4, hkv=2, seed=25)
    m = c.bufs["mask"].reshape(70, 70)
    m[5, :] = cases.NEG_INF_F16
    m[69, :] = cases.NEG_INF_F16
    out = check_case(runner, c)
    assert (out[0, 5] == 0).all() and (out[0, 69] == 0).all()


def test_decode_fully_masked_is_zero(runner):
    c = cases.decode_case(500, window=0, seed=26)
    out = check_case(runner, c)
    assert (out == 0).all()


def test_finite_additive_mask(runner):
    """non-binary additive mask values (e.g. a bias) are added, not thresholded"""
    c = cases.prefill_case(90, hq=8, hkv=2, seed=27)
    rng = np.random.default_rng(27)
    m = c.bufs["mask"].reshape(90, 90)
    bias = cases.f16_bits(rng.uniform(-3, 3, size=m.shape).astype(np.float32))
    c.bufs["mask"] = np.where(m == cases.NEG_INF_F16, m, bias).astype(np.uint16)
    check_case(runner, c)


def test_mask_head_planes_and_batch_broadcast(runner):
    """mask with 2 head planes (plane h % 2) and K/V shared by 2 q batches"""
    rng = np.random.default_rng(28)
    c = cases.decode_case(600, hq=8, hkv=2, hd=128, seed=28, batch=2)
    # K/V: keep only batch 0 and broadcast it (Bk = 1)
    for name in ("k", "v"):
        b, t, ne, nb, off = c.views[name]
        c.views[name] = (b, t, (ne[0], ne[1], ne[2], 1), nb, off)
    m = np.where(rng.uniform(size=(1, 2, 1, 600)) < 0.3, cases.NEG_INF_F16, np.uint16(0)).astype(np.uint16)
    c.bufs["mask"] = m
    c.views["mask"] = ("mask", oracle.F16, (600, 1, 2, 1), (2, 1200, 1200, 2400), 0)
    check_case(runner, c)


def test_deterministic_and_reusable(runner):
    """same inputs give identical bits; the split-KV counters reset themselves"""
    import gpu_util
    c = cases.decode_case(8192, seed=29)
    dev = gpu_util.to_device(c)
    _, a = runner.run(c, dev=dev)
    for _ in range(3):
        _, b = runner.run(c, dev=dev)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    c2 = cases.decode_case(3000, hq=16, hkv=4, seed=30, batch=3)
    check_case(runner, c2)
    _, b = runner.run(c, dev=dev)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_unsupported_types_are_reported(runner):
    import gpu_util
    c = cases.decode_case(64, seed=31)
    c.bufs["k32"] = c.bufs["k"].view(np.float16).astype(np.float32)
    b, t, ne, nb, off = c.views["k"]
    c.views["k"] = ("k32", oracle.F32, ne, tuple(x * 2 for x in nb), 0)
    rc, _ = runner.run(c, check=False)
    assert rc == gpu_util.vxfa.UNSUPPORTED


def test_graph_capture_replays_match_eager(runner):
    """Calls captured into a HIP graph (decode split+merge, masked prefill)
    replay to the same bits as eager calls, with eager work between replays."""
    import torch
    import gpu_util
    cs = [cases.decode_case(8192, seed=41), cases.prefill_case(100, hq=8, hkv=2, seed=42)]
    devs = [gpu_util.to_device(c) for c in cs]
    outs = []
    eager = []
    for c, d in zip(cs, devs):
        _, ref = runner.run(c, dev=d)
        eager.append(ref)
        B, Nq, Hq, D = c.out_shape
        outs.append(torch.zeros(B * Nq * Hq * D, device="cuda", dtype=torch.float32))
    stream = torch.cuda.Stream()
    descs = [gpu_util.descs(c, d) for c, d in zip(cs, devs)]

    def step():
        for c, dd, o in zip(cs, descs, outs):
            ne, nb = c.dst_ne_nb()
            dst = gpu_util.vxfa.desc(o.data_ptr(), gpu_util.vxfa.F32, ne, nb)
            runner.ctx.flash_attn_ext(dd["q"], dd["k"], dd["v"], dd.get("mask"), dst, c.scale,
                                      stream=stream.cuda_stream)

    with torch.cuda.stream(stream):
        step()  # first launches outside the capture (code objects load on first use)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        step()
    torch.cuda.synchronize()
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        with torch.cuda.stream(stream):
            g.replay()
        torch.cuda.synchronize()
        runner.run(cs[0], dev=devs[0])  # eager work between replays
        for o, ref, c in zip(outs, eager, cs):
            got = o.cpu().numpy().reshape(c.out_shape)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (rep, c.name)


# --- implicit masks: vxfa_flash_attn_ext_implicit ------------------------------
# The descriptor path against the explicit mask tensor it stands for (same
# case, same device bytes) and against the oracle run with that tensor.
# Prefill takes the same kernel path with the same step order, so the bits
# must agree exactly; decode sizes its splits to the live range instead of
# n_kv, which changes the summation order, so it is held to the parity bar.

def _implicit(runner, c, offset, window=0, bitwise=True):
    import gpu_util
    from conftest import load_package
    vx = load_package().vxfa
    B, Nq, Hq, D = c.out_shape
    nkv = c.views["k"][2][1]
    cases.with_mask(c, cases.implicit_mask(Nq, nkv, offset, window))
    _say(f"[implicit] {c.name} offset={offset} window={window}")
    explicit = check_case(runner, c)
    dev = gpu_util.to_device(c)
    rc, out = runner.run_implicit(c, vx.mask_desc(vx.MASK_CAUSAL, window, offset), dev=dev)
    assert rc == 0
    assert np.isfinite(out).all()
    if bitwise:
        assert np.array_equal(out.view(np.uint32), explicit.view(np.uint32))
    m, r, ok = gpu_util.parity(out, cases.oracle_f64(c), ATOL, RTOL)
    _say(f"    implicit vs f64 maxabs={m:.3e} rel={r:.3e}; vs explicit maxabs={np.abs(out - explicit).max():.3e}")
    assert ok, (m, r)
    return out


def test_implicit_decoder_prefill_439_causal(runner):
    _implicit(runner, cases.prefill_case(439, seed=41, causal=False), offset=0)


@pytest.mark.parametrize("n,kv_offset", [(64, 448), (1, 100), (200, 37)])
def test_implicit_causal_against_filled_cache(runner, n, kv_offset):
    c = cases.prefill_case(n, seed=42 + n, causal=False, kv_offset=kv_offset)
    _implicit(runner, c, offset=kv_offset, bitwise=(n > 1))


def test_implicit_realtime_encoder_window(runner):
    """Realtime encoder: 32 heads, hd 64, causal window 750 (src/voxtral.cpp:2179-2190)."""
    _implicit(runner, cases.encoder_case(1100, 32, 64, seed=43), offset=0, window=750, bitwise=HD64_MASK_BITWISE)


# hd 64 under an implicit mask and under a mask tensor runs the pipelined
# encoder kernel; a tensor whose rows are live intervals (a pre-pass finds
# them) takes the implicit mask's path with the same bounds: bitwise equal
HD64_MASK_BITWISE = True


@pytest.mark.parametrize("seq,heads,window,offset", [(1500, 4, 750, 0), (1500, 2, 0, 0), (333, 3, 1, 0),
                                                     (257, 2, 31, 5), (700, 2, 100, 600), (129, 2, 0, -100),
                                                     (64, 1, 33, 0), (1, 2, 0, 0), (161, 2, 64, 0),
                                                     (700, 8, 200, 0), (300, 16, 0, 50)])
def test_implicit_hd64_windows(runner, seq, heads, window, offset):
    """The pipelined hd 64 kernel under implicit causal / window masks: row
    ranges that start and end inside a block, windows of one position and of
    one block less one, offsets past the KV length and before it (rows with
    no live position give zeros), partial last blocks; 8 and 16 heads take
    the heavy-tiles-first grid order."""
    from conftest import load_package
    import gpu_util
    vx = load_package().vxfa
    c = cases.encoder_case(seq, heads, 64, seed=700 + seq + window)
    m = cases.implicit_mask(seq, seq, offset, window)
    rc, out = runner.run_implicit(c, vx.mask_desc(vx.MASK_CAUSAL, window, offset))
    assert rc == 0
    assert np.isfinite(out).all()
    cases.with_mask(c, m)
    for ref in (cases.oracle_ggml(c), cases.oracle_f64(c)):
        mx, r, ok = gpu_util.parity(out, ref, ATOL, RTOL)
        _say(f"    implicit hd64 seq={seq} w={window} off={offset}: maxabs={mx:.3e} rel={r:.3e}")
        assert ok, (mx, r)
    dead = ~(m != cases.NEG_INF_F16).any(axis=1)
    assert (out[:, dead] == 0).all()
    # the same mask as an F16 tensor
    rc, mt = runner.run(c)
    assert rc == 0
    assert np.array_equal(mt.view(np.uint32), out.view(np.uint32))


def _mask_planes(c, planes):
    """Replace c's mask by the [nkv, nq, P, 1] tensor of the P planes (uint16
    [nq, nkv] each); head h reads plane h % P."""
    nq, nkv = planes[0].shape
    m = np.ascontiguousarray(np.stack(planes))
    c.bufs.pop("mask", None)
    c.views.pop("mask", None)
    c.add("mask", "mask", m, oracle.F16, (nkv, nq, len(planes), 1),
          (2, 2 * nkv, 2 * nkv * nq, 2 * nkv * nq * len(planes)))
    return c


def _hd64_mask(kind, seq, rng):
    m = cases.implicit_mask(seq, seq, 0, 100)
    if kind == "holes":           # -inf holes inside the window of rows 130 .. 140
        for r in range(min(130, seq - 1), min(141, seq)):
            if r >= 2:
                m[r, r - 1] = cases.NEG_INF_F16
    elif kind == "bias":          # finite values on every live entry
        bias = cases.f16_bits(rng.uniform(-3, 3, size=m.shape).astype(np.float32))
        m = np.where(m == cases.NEG_INF_F16, m, bias).astype(np.uint16)
    elif kind == "minus_zero":    # -0 entries are live
        m = np.where(m == 0, np.uint16(0x8000), m).astype(np.uint16)
    elif kind == "empty_rows":    # rows with no live entry
        m[::7] = cases.NEG_INF_F16
    elif kind == "islands":       # one live run per row, anywhere
        m[:] = cases.NEG_INF_F16
        for r in range(seq):
            lo = int(rng.integers(0, seq))
            m[r, lo:int(rng.integers(lo, seq)) + 1] = 0
    return m


@pytest.mark.parametrize("kind", ["holes", "bias", "minus_zero", "empty_rows", "islands"])
@pytest.mark.parametrize("seq", [300, 161])
def test_hd64_mask_tensor(runner, kind, seq):
    """hd 64 prefill with a mask tensor on the pipelined kernel: rows that are
    live intervals (window, islands, -0, empty rows) take the interval path;
    a workgroup with holes or finite values adds the mask per element. An odd
    n_kv (161) puts the mask rows off 16-byte alignment."""
    rng = np.random.default_rng(900 + seq + len(kind))
    c = cases.encoder_case(seq, 4, 64, seed=900 + seq)
    cases.with_mask(c, _hd64_mask(kind, seq, rng))
    out = check_case(runner, c)
    m = c.bufs["mask"]
    dead = ~(m != cases.NEG_INF_F16).any(axis=1)
    assert (out[:, dead] == 0).all()


def test_hd64_mask_tensor_planes(runner):
    """Two mask planes (head h reads plane h % 2): a window on one, finite
    values on the other, so one plane's workgroups take the interval path
    and the other's the per-element path."""
    rng = np.random.default_rng(950)
    c = cases.encoder_case(400, 4, 64, seed=950)
    _mask_planes(c, [_hd64_mask("window", 400, rng), _hd64_mask("bias", 400, rng)])
    check_case(runner, c)


@pytest.mark.parametrize("window", [1, 100, 512])
def test_implicit_prefill_windows(runner, window):
    _implicit(runner, cases.prefill_case(333, seed=44, causal=False), offset=0, window=window)


def test_implicit_negative_offset_empties_rows(runner):
    out = _implicit(runner, cases.prefill_case(130, seed=45, causal=False), offset=-5)
    assert (out[:, :5] == 0).all()


def test_implicit_decode_sliding_window(runner):
    """Config 4 shape: cache 16384, n_kv 16285, window 2048 as a descriptor."""
    c = cases.decode_case(16285, capacity=16384, seed=46)
    _implicit(runner, c, offset=16284, window=2048, bitwise=False)


@pytest.mark.parametrize("n_kv,offset,window", [(1024, 1023, 0), (777, 500, 64), (300, 5000, 0), (300, -1, 0)])
def test_implicit_decode_ranges(runner, n_kv, offset, window):
    c = cases.decode_case(n_kv, seed=47 + n_kv)
    out = _implicit(runner, c, offset=offset, window=window, bitwise=False)
    if offset < 0:
        assert (out == 0).all()


def test_implicit_none_equals_no_mask(runner):
    import gpu_util
    from conftest import load_package
    vx = load_package().vxfa
    c = cases.encoder_case(300, 4, 64, seed=48)
    dev = gpu_util.to_device(c)
    rc1, a = runner.run(c, dev=dev)
    rc2, b = runner.run_implicit(c, vx.mask_desc(vx.MASK_NONE), dev=dev)
    rc3, d = runner.run_implicit(c, None, dev=dev)
    assert rc1 == rc2 == rc3 == 0
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(a.view(np.uint32), d.view(np.uint32))


def test_implicit_rejects_bad_descriptor(runner):
    from conftest import load_package
    vx = load_package().vxfa
    c = cases.decode_case(64, seed=49)
    rc, _ = runner.run_implicit(c, vx.mask_desc(7, 0, 0), check=False)
    assert rc == vx.INVALID_ARG


# --- f16 KV cache append: vxfa_kv_append / vxfa_flash_attn_ext_append ---------
# New K/V rows arrive as F32 (the projections of build_decoder_layer) and are
# rounded to f16 into the cache (the ggml_cpy of src/voxtral.cpp:1758-1770).
# The cache bytes after the call must equal numpy's float16 (round to nearest
# even) of the rows, every other cache byte untouched; the attention output is
# checked against the oracle run on that appended cache.

def _append_rows(rng, bk, n_new, row, special=False):
    k = rng.standard_normal((bk, n_new, row)).astype(np.float32)
    v = rng.standard_normal((bk, n_new, row)).astype(np.float32)
    if special:   # overflow to inf, subnormals, an exact tie, negative zero
        k[0, 0, :6] = [70000.0, -1e6, 3e-6, -6e-8, np.float32(1.0 + 2.0 ** -11), -0.0]
    return k, v


def _expected_cache(c, k_new, v_new):
    """The case with its cache rows n_kv - n_new .. n_kv - 1 set to f16(new)."""
    import copy
    e = copy.deepcopy(c)
    bk, n_new, row = k_new.shape
    for role, new in (("k", k_new), ("v", v_new)):
        b, t, ne, nb, off = e.views[role]
        D, nkv, hkv, _ = ne
        raw = e.bufs[b].view(np.uint8).reshape(-1).copy()
        with np.errstate(over="ignore"):
            bits = new.astype(np.float16).view(np.uint16)        # RNE, overflow -> inf
        for bb in range(bk):
            for tt in range(n_new):
                pos = nkv - n_new + tt
                for h in range(hkv):
                    at = off + pos * nb[1] + h * nb[2] + bb * nb[3]
                    raw[at:at + 2 * D] = bits[bb, tt, h * D:(h + 1) * D].view(np.uint8)
        e.bufs[b] = raw.view(e.bufs[b].dtype).reshape(e.bufs[b].shape)
    return e


def _check_append(runner, c, k_new, v_new, fused=True):
    import gpu_util
    e = _expected_cache(c, k_new, v_new)
    _say(f"[append] {c.name} n_new={k_new.shape[1]} bk={k_new.shape[0]} fused={fused}")
    rc, out, after = runner.run_append(c, k_new, v_new, fused=fused)
    assert rc == 0
    for role in ("k", "v"):
        b = c.views[role][0]
        assert np.array_equal(after[b], e.bufs[b].view(np.uint8).reshape(-1)), f"{role} cache bytes"
    exact = cases.oracle_f64(e)
    m, r, ok = gpu_util.parity(out, exact, ATOL, RTOL)
    _say(f"    vs f64 on the appended cache maxabs={m:.3e} rel={r:.3e}")
    assert np.isfinite(out).all() and ok, (m, r)
    return out


def test_kv_append_rows_bit_exact(runner):
    import torch
    import gpu_util
    from conftest import load_package
    vx = load_package().vxfa
    c = cases.decode_case(40, hq=16, hkv=8, hd=128, capacity=64, seed=61)
    k_new, v_new = _append_rows(np.random.default_rng(61), 1, 3, 8 * 128, special=True)
    e = _expected_cache(c, k_new, v_new)
    dev = gpu_util.to_device(c)
    d = gpu_util.descs(c, dev)
    kn = torch.from_numpy(k_new).to("cuda")
    vn = torch.from_numpy(v_new).to("cuda")
    ne, nb = (1024, 3, 1, 1), (4, 4096, 12288, 12288)
    rc = runner.ctx.kv_append(vx.desc(kn.data_ptr(), vx.F32, ne, nb), vx.desc(vn.data_ptr(), vx.F32, ne, nb),
                              d["k"], d["v"], stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0
    for role in ("k", "v"):
        b = c.views[role][0]
        assert np.array_equal(dev[b].cpu().numpy(), e.bufs[b].view(np.uint8).reshape(-1)), role


@pytest.mark.parametrize("n_kv", [1, 33, 1024, 8192])
def test_fused_decode_append(runner, n_kv):
    c = cases.decode_case(n_kv, capacity=n_kv + 16, seed=62 + n_kv)
    k_new, v_new = _append_rows(np.random.default_rng(n_kv), 1, 1, 8 * 128)
    fused = _check_append(runner, c, k_new, v_new, fused=True)
    separate = _check_append(runner, c, k_new, v_new, fused=False)
    assert np.abs(fused - separate).max() <= 1e-5


def test_fused_decode_append_groups_and_batch(runner):
    c = cases.decode_case(700, hq=16, hkv=8, hd=64, capacity=720, batch=3, seed=63)
    k_new, v_new = _append_rows(np.random.default_rng(63), 3, 1, 8 * 64)
    _check_append(runner, c, k_new, v_new, fused=True)


def test_fused_decode_append_masked(runner):
    """Streaming shape with an explicit window mask over the appended row."""
    c = cases.decode_case(5000, capacity=5008, window=1024, seed=64)
    k_new, v_new = _append_rows(np.random.default_rng(64), 1, 1, 8 * 128)
    _check_append(runner, c, k_new, v_new, fused=True)


def test_prefill_append_matches_separate(runner):
    c = cases.prefill_case(64, seed=65, kv_offset=448)
    k_new, v_new = _append_rows(np.random.default_rng(65), 1, 64, 8 * 128)
    a = _check_append(runner, c, k_new, v_new, fused=True)
    b = _check_append(runner, c, k_new, v_new, fused=False)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_append_rejects_bad_rows(runner):
    from conftest import load_package
    vx = load_package().vxfa
    c = cases.decode_case(64, seed=66)
    k_new, v_new = _append_rows(np.random.default_rng(66), 1, 1, 8 * 128 + 8)   # wrong row length
    rc, _, _ = runner.run_append(c, k_new, v_new, fused=True, check=False)
    assert rc == vx.INVALID_ARG


# --- ring-buffer KV cache: vxfa_flash_attn_ext_ring -----------------------------
# Logical row p lives in cache row (start + p) % capacity. The kernel walks the
# logical rows in the same tiles as for a linear cache, so the output must be
# bit-identical to vxfa_flash_attn_ext on the linear cache with the same rows.

@pytest.mark.parametrize("n_kv,capacity,start", [(1000, 1024, 0), (1000, 1024, 500), (2048, 2048, 2047),
                                                 (8192, 8192, 77), (1, 64, 63), (33, 40, 20)])
def test_ring_equals_linear(runner, n_kv, capacity, start):
    from conftest import load_package
    vx = load_package().vxfa
    lin = cases.decode_case(n_kv, seed=71 + n_kv)
    _say(f"[ring] n_kv={n_kv} capacity={capacity} start={start}")
    rc, ref = runner.run(lin)
    assert rc == 0
    rg = cases.ring_case(lin, capacity, start, seed=72)
    rc, out, _ = runner.run_ring(rg, vx.ring(start, n_kv))
    assert rc == 0
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    _ring_vs_oracle(out, lin)


def _ring_vs_oracle(out, lin):
    """The ring output against the oracle run on the linear cache holding
    the same rows in logical order (kv_cache_shift_left's result,
    src/voxtral.cpp:1237-1266)."""
    import gpu_util
    for name, ref in (("ggml-fp32", cases.oracle_ggml(lin)), ("f64", cases.oracle_f64(lin))):
        m, r, ok = gpu_util.parity(out, ref, ATOL, RTOL)
        _say(f"    ring vs {name} maxabs={m:.3e} rel={r:.3e}")
        assert ok, (name, m, r)


@pytest.mark.parametrize("n_kv,capacity,start", [(512, 512, 300), (100, 128, 100), (4096, 8192, 6000)])
def test_ring_fused_append(runner, n_kv, capacity, start):
    """The step's new row lands in cache row (start + n_kv - 1) % capacity,
    nothing else is written, and the output equals the linear fused append."""
    from conftest import load_package
    vx = load_package().vxfa
    lin = cases.decode_case(n_kv, hq=32, hkv=8, hd=128, seed=73 + n_kv)
    k_new, v_new = _append_rows(np.random.default_rng(74), 1, 1, 8 * 128)
    rc, ref, _ = runner.run_append(lin, k_new, v_new, fused=True)
    assert rc == 0
    rg = cases.ring_case(lin, capacity, start, seed=75)
    rc, out, after = runner.run_ring(rg, vx.ring(start, n_kv), k_new, v_new)
    assert rc == 0
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    _ring_vs_oracle(out, _expected_cache(lin, k_new, v_new))
    row = (start + n_kv - 1) % capacity
    for role, new in (("k", k_new), ("v", v_new)):
        b = rg.views[role][0]
        expect = rg.bufs[b].copy()
        expect[0, row] = new[0, 0].astype(np.float16).view(np.uint16).reshape(8, 128)
        assert np.array_equal(after[b], expect.view(np.uint8).reshape(-1)), role


def test_ring_as_sliding_window(runner):
    """A 2048-row ring holding the window equals the explicit window mask over a 16K cache."""
    import gpu_util
    from conftest import load_package
    vx = load_package().vxfa
    big = cases.decode_case(16285, capacity=16384, window=2048, seed=76)
    rc, ref = runner.run(big)
    assert rc == 0
    win = cases.decode_case(2048, seed=76)
    win.bufs["q"] = big.bufs["q"]
    for role in ("k", "v"):
        b = big.views[role][0]
        win.bufs[b] = big.bufs[b][:, 16285 - 2048:16285].copy()
    rg = cases.ring_case(win, 2048, 1234, seed=77)
    rc, out, _ = runner.run_ring(rg, vx.ring(1234, 2048))
    assert rc == 0
    m, r, ok = gpu_util.parity(out, ref, 1e-5, 1e-5)
    _say(f"    ring vs 16K windowed decode maxabs={m:.3e} rel={r:.3e}")
    assert ok


def test_ring_rejects_bad_descriptors(runner):
    from conftest import load_package
    vx = load_package().vxfa
    c = cases.ring_case(cases.decode_case(100, seed=78), 128, 0)
    assert runner.run_ring(c, vx.ring(128, 100), check=False)[0] == vx.INVALID_ARG
    assert runner.run_ring(c, vx.ring(0, 129), check=False)[0] == vx.INVALID_ARG
    p = cases.ring_case(cases.decode_case(100, seed=79), 128, 5)
    p.views["q"] = cases.prefill_case(4, seed=79, causal=False).views["q"]
    p.bufs["q"] = cases.prefill_case(4, seed=79, causal=False).bufs["q"]
    assert runner.run_ring(p, vx.ring(5, 100), check=False)[0] == vx.UNSUPPORTED


# --- rotary embedding fused into the op: vxfa_flash_attn_ext_rope -------------
# The same call with q and the new K rows rotated on the host by the ggml
# restatement (cases.rope_ggml) and passed through vxfa_flash_attn_ext_append
# is the reference; cos / sin may differ in the last bit between the device
# and the host, so outputs are compared at 2e-4 and cache bytes to within one
# f16 step (and mostly equal), besides the oracle bar.

def _rope_check(runner, c, k_new, v_new, positions, n_dims, base):
    import copy
    import gpu_util
    B, Nq, Hq, D = c.out_shape
    qb, qt, qne, qnb, qoff = c.views["q"]
    q = c.bufs[qb]
    # q buffers are [B][tokens][heads][D] (the mul_mat output's view); rotate per token
    q4 = q.reshape(B, -1, Hq, D)
    pos_b = np.asarray(positions, dtype=np.int32).reshape(B, Nq)
    qr = np.stack([cases.rope_ggml(q4[b], pos_b[b], n_dims, base) for b in range(B)]).reshape(q.shape)
    hkv = k_new.shape[2] // D
    kr = np.stack([cases.rope_ggml(k_new[b].reshape(Nq, hkv, D), pos_b[b], n_dims, base).reshape(Nq, -1)
                   for b in range(k_new.shape[0])])
    host = copy.deepcopy(c)
    host.bufs[qb] = qr.astype(np.float32)
    _say(f"[rope] {c.name} n_dims={n_dims} base={base} positions {positions[0]}..{positions[-1]}")
    rc, ref, _ = runner.run_append(host, kr, v_new, fused=True)
    assert rc == 0
    rc, out, after = runner.run_rope(c, k_new, v_new, positions, n_dims, base)
    assert rc == 0
    m, r, ok = gpu_util.parity(out, ref, 2e-4, 2e-4)
    _say(f"    vs host-rotated maxabs={m:.3e} rel={r:.3e}")
    assert ok, (m, r)
    e = _expected_cache(host, kr, v_new)
    for role in ("k", "v"):
        b = c.views[role][0]
        got = after[b].view(np.uint16).astype(np.int32)
        want = e.bufs[b].view(np.uint16).reshape(-1).astype(np.int32)
        diff = np.abs(got - want)
        _say(f"    {role} cache: {int((diff > 0).sum())} of {diff.size} halves differ, max {int(diff.max())} steps")
        assert diff.max() <= 1 and (diff > 0).mean() < 1e-3
    exact = cases.oracle_f64(e)
    m, r, ok = gpu_util.parity(out, exact, ATOL, RTOL)
    assert ok, (m, r)


def test_rope_decode_step(runner):
    """Decoder step at position 8191 (theta 1e6, hd 128): q and the new row rotated."""
    c = cases.decode_case(8192, capacity=8192, seed=81)
    k_new, v_new = _append_rows(np.random.default_rng(81), 1, 1, 8 * 128)
    _rope_check(runner, c, k_new, v_new, [8191], 128, 1.0e6)


def test_rope_prefill_after_cache(runner):
    c = cases.prefill_case(64, seed=82, kv_offset=448)
    k_new, v_new = _append_rows(np.random.default_rng(82), 1, 64, 8 * 128)
    _rope_check(runner, c, k_new, v_new, list(range(448, 512)), 128, 1.0e6)


def test_rope_partial_dims_and_small_base(runner):
    c = cases.prefill_case(40, hq=8, hkv=2, hd=64, seed=83, kv_offset=10)
    k_new, v_new = _append_rows(np.random.default_rng(83), 1, 40, 2 * 64)
    _rope_check(runner, c, k_new, v_new, list(range(1000, 1040)), 48, 10000.0)


def test_rope_rejects_unsupported(runner):
    from conftest import load_package
    vx = load_package().vxfa
    c = cases.decode_case(64, seed=84)
    k_new, v_new = _append_rows(np.random.default_rng(84), 1, 1, 8 * 128)
    assert runner.run_rope(c, k_new, v_new, [63], 128, 1e6, mode=2, check=False)[0] == vx.UNSUPPORTED
    assert runner.run_rope(c, k_new, v_new, [63], 127, 1e6, check=False)[0] == vx.INVALID_ARG
    k2, v2 = _append_rows(np.random.default_rng(84), 1, 2, 8 * 128)
    assert runner.run_rope(c, k2, v2, [62, 63], 128, 1e6, check=False)[0] == vx.INVALID_ARG


def test_ring_wrapped_with_appended_row_wrapping(runner):
    """The appended row itself wraps to cache row 0 (start + n_kv - 1 ==
    capacity), checked against the oracle on the appended linear cache."""
    from conftest import load_package
    vx = load_package().vxfa
    n_kv, capacity = 300, 512
    start = capacity - n_kv + 1
    lin = cases.decode_case(n_kv, seed=79)
    k_new, v_new = _append_rows(np.random.default_rng(79), 1, 1, 8 * 128)
    rg = cases.ring_case(lin, capacity, start, seed=80)
    rc, out, after = runner.run_ring(rg, vx.ring(start, n_kv), k_new, v_new)
    assert rc == 0
    assert (start + n_kv - 1) % capacity == 0
    _ring_vs_oracle(out, _expected_cache(lin, k_new, v_new))
    b = rg.views["k"][0]
    assert np.array_equal(after[b].view(np.uint16).reshape(capacity, 8, 128)[0],
                          k_new[0, 0].astype(np.float16).view(np.uint16).reshape(8, 128))


# --- the workspace: fixed at context creation, graph-safe ------------------------

def test_graph_capture_then_larger_eager_calls(runner):
    """A decode step captured into a HIP graph at n_kv 1024 (8 splits: its
    partial records live in the context's workspace) replays to the eager
    bits after eager calls that use more splits and records (n_kv 8192, 32
    ragged streams), with eager work between the replays: no call resizes,
    moves or leaves dirty the context's workspace. (Captures of F32 staging
    and of the no-alloc scratch are in test_gpu_decode_layout.py and
    test_zz_no_alloc.py.)"""
    import torch
    import gpu_util
    small = cases.decode_case(1024, seed=91)
    dev = gpu_util.to_device(small)
    rc, ref = runner.run(small, dev=dev)
    assert rc == 0
    d = gpu_util.descs(small, dev)
    B, Nq, Hq, D = small.out_shape
    out = torch.zeros(B * Nq * Hq * D, device="cuda", dtype=torch.float32)
    ne, nb = small.dst_ne_nb()
    dst = gpu_util.vxfa.desc(out.data_ptr(), gpu_util.vxfa.F32, ne, nb)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        runner.ctx.flash_attn_ext(d["q"], d["k"], d["v"], None, dst, small.scale, stream=stream.cuda_stream)
    torch.cuda.synchronize()
    big = cases.decode_case(8192, seed=92)
    batch = cases.batched_case(32, capacity=4096, lo=512, hi=4096, seed=93)
    check_case(runner, big)
    check_case(runner, batch)
    for rep in range(3):
        out.fill_(float("nan"))
        with torch.cuda.stream(stream):
            g.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(small.out_shape)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), rep
        runner.run(big, verify_inputs=False)   # eager work between replays


# --- F32 K/V: the reference's own cache and encoder K/V --------------------------
# voxtral.cpp's KV cache is F32 (src/voxtral.cpp:1126-1136) and its encoder's
# K/V are F32 mul_mat outputs (:1581-1605). ggml keeps Q in F32 for an F32 K.
# Decode does the same (F32 QK^T and P.V); prefill rounds K, V and Q to f16
# (its tiles reach LDS through direct copies of an f16 staging copy). Every
# case is held to the bar against the restatement (F32 dot products) and the
# exact reference; decode also to a bar 100 times tighter.

# F32 decode: both products in F32, so the output agrees with the exact
# reference and with ggml's F32 restatement to F32 rounding, far inside the
# bar (f16-rounded Q and K leave errors near 1e-3 on these inputs).
F32_ATOL, F32_RTOL = 2e-5, 1e-4


@pytest.mark.parametrize("n_kv,hd,groups,q_f16", [(1024, 128, 4, False), (8192, 128, 4, False), (3000, 64, 2, False),
                                                  (700, 128, 1, False), (1024, 128, 4, True), (2048, 64, 4, False),
                                                  (517, 128, 2, False), (33, 64, 1, True), (1, 128, 4, False)])
def test_f32_cache_decode_keeps_f32_products(runner, n_kv, hd, groups, q_f16):
    import gpu_util
    c = cases.decode_case(n_kv, hq=8 * groups, hkv=8, hd=hd, seed=1300 + n_kv + hd, kv_f32=True, q_f16=q_f16)
    rc, out = runner.run(c)
    assert rc == 0
    for tag, ref in (("ggml-fp32", cases.oracle_ggml(c)), ("f64", cases.oracle_f64(c))):
        m, r, ok = gpu_util.parity(out, ref, F32_ATOL, F32_RTOL, elem_rtol=F32_RTOL)
        _say(f"    F32 decode n_kv {n_kv} hd {hd} G {groups} vs {tag}: maxabs={m:.3e} rel={r:.3e} "
             f"elem={gpu_util.elem_rel(out, ref):.3e}")
        assert ok, (tag, m, r)

@pytest.mark.parametrize("n_kv", [1, 100, 1024, 8192])
def test_f32_cache_decode(runner, n_kv):
    check_case(runner, cases.decode_case(n_kv, capacity=n_kv + 3, seed=1100 + n_kv, kv_f32=True))


def test_f32_cache_decode_window_groups_batch(runner):
    check_case(runner, cases.decode_case(3000, seed=1201, window=700, kv_f32=True))
    check_case(runner, cases.decode_case(900, hq=16, hkv=8, hd=64, batch=3, seed=1202, kv_f32=True))
    check_case(runner, cases.batched_case(8, capacity=2048, lo=100, hi=2048, seed=1203, kv_f32=True))


def test_f32_cache_decode_implicit_window(runner):
    c = cases.decode_case(5000, seed=1204, kv_f32=True)
    _implicit(runner, c, offset=4999, window=2048, bitwise=False)


def test_f32_encoder_prefill_1500x20(runner):
    check_case(runner, cases.encoder_case(1500, 20, 64, seed=1205, kv_f32=True))


def test_f32_realtime_encoder_window(runner):
    check_case(runner, cases.encoder_case(1000, 4, 64, seed=1206, window=750, kv_f32=True))


def test_f32_decoder_prefill_439_causal(runner):
    check_case(runner, cases.prefill_case(439, seed=1207, kv_f32=True))


def _runner_with_env(**kw):
    """A second context created with tuning variables set (a context reads
    them once, at creation)."""
    import os
    import gpu_util
    old = {k: os.environ.get(k) for k in kw}
    os.environ.update({k: str(v) for k, v in kw.items()})
    try:
        return gpu_util.Runner()
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


# F32 K/V with a mask tensor on the short masked prefill (voxtral's decoder
# prefill as the unchanged application calls it): the staging launch also
# finds each mask row's live interval and the kernel takes its block classes
# from them instead of reading the mask first; mixed blocks still read their
# words from the tensor.

@pytest.mark.parametrize("n,nkv", [(339, 439), (439, 439), (64, 65), (129, 511), (2, 130)])
def test_f32_prefill_interval_classes_bitwise(runner, n, nkv):
    """Causal masks (rows are intervals): the same bits as classifying from
    the mask (VXFA_PAIR_INTERVALS=0 on a second context), within the bar of
    the oracle."""
    c = cases.prefill_case(n, seed=1400 + n + nkv, kv_offset=nkv - n, kv_f32=True)
    out = check_case(runner, c)
    other = _runner_with_env(VXFA_PAIR_INTERVALS=0)
    try:
        rc, out2 = other.run(c)
        assert rc == 0
    finally:
        other.close()
    assert np.array_equal(out.view(np.uint32), out2.view(np.uint32))


def test_f32_prefill_intervals_with_f16_q(runner):
    """F16 Q on the interval route (the pair kernel's F16-Q instantiation):
    a causal prefill after 100 cached rows with F32 K/V, the same bits as
    classifying from the mask, within the bar of the oracle."""
    n, off = 139, 100
    c = cases.prefill_case(n, seed=1600, kv_offset=off, kv_f32=True)
    q = c.bufs["q"].reshape(n, 32, 128).astype(np.float32)
    c.bufs["q"] = cases.f16_bits(q)
    c.views["q"] = ("q", oracle.F16, *cases.views.decoder_q(n, 32, 128, 2), 0)
    out = check_case(runner, c)
    other = _runner_with_env(VXFA_PAIR_INTERVALS=0)
    try:
        rc, out2 = other.run(c)
        assert rc == 0
    finally:
        other.close()
    assert np.array_equal(out.view(np.uint32), out2.view(np.uint32))


@pytest.mark.parametrize("kind", ["sparse", "bias", "empty_rows", "window"])
def test_f32_prefill_masks_through_intervals(runner, kind):
    """Masks whose rows are not all intervals take the fallback (every block
    of such a row's tile computed with its words from the tensor): isolated
    live entries at chunk and tile edges, finite additive values, fully masked
    rows, and a sliding window as a tensor; F32 K/V, against the oracle."""
    rng = np.random.default_rng(1500 + len(kind))
    if kind == "sparse":
        n, nkv = 71, 133
        c = cases.prefill_case(n, causal=False, kv_offset=nkv - n, seed=1501, kv_f32=True)
        c = cases.with_mask(c, _sparse_mask(rng, n, nkv))
    elif kind == "bias":
        c = cases.prefill_case(90, hq=8, hkv=2, seed=1502, kv_f32=True)
        m = c.bufs["mask"].reshape(90, 90)
        bias = cases.f16_bits(rng.uniform(-3, 3, size=m.shape).astype(np.float32))
        c.bufs["mask"] = np.where(m == cases.NEG_INF_F16, m, bias).astype(np.uint16)
    elif kind == "empty_rows":
        c = cases.prefill_case(70, hq=4, hkv=2, seed=1503, kv_f32=True)
        m = c.bufs["mask"].reshape(70, 70)
        m[5, :] = cases.NEG_INF_F16
        m[69, :] = cases.NEG_INF_F16
    else:
        n, nkv = 200, 437
        c = cases.prefill_case(n, causal=False, kv_offset=nkv - n, seed=1504, kv_f32=True)
        c = cases.with_mask(c, cases.implicit_mask(n, nkv, nkv - n, 50))
    if kind == "sparse":
        # A few live entries per row: each output follows a handful of V rows,
        # and the f16 rounding of Q that prefill applies against F32 K (ggml
        # keeps Q in F32 there) shows at up to ~1.3x the max-abs bar on this
        # mask. Held to the bar against the exact reference with Q rounded as
        # the kernel does, and to twice the bar against ggml's F32 semantics.
        import gpu_util
        rc, out = runner.run(c)
        assert rc == 0
        m1, r1, ok1 = gpu_util.parity(out, cases.oracle_f64(c, q_f16=True), ATOL, RTOL)
        m2, r2, ok2 = gpu_util.parity(out, cases.oracle_f64(c), 2 * ATOL, RTOL)
        _say(f"    sparse F32 prefill: vs exact with Q rounded maxabs={m1:.3e} rel={r1:.3e}; "
             f"vs exact F32 Q maxabs={m2:.3e} rel={r2:.3e}")
        assert ok1, (m1, r1)
        assert ok2, (m2, r2)
        return
    out = check_case(runner, c)
    if kind == "empty_rows":
        assert (out[0, 5] == 0).all() and (out[0, 69] == 0).all()


def test_f32_prefill_beyond_staging_reports_no_workspace(runner):
    """K and V of 16384 rows x 8 x 128 need 64 MiB of f16 staging; the context
    holds 32 MiB, so the call returns VXFA_NO_WORKSPACE and launches nothing."""
    from conftest import load_package
    vx = load_package().vxfa
    c = cases.prefill_case(2, seed=1208, causal=False, kv_offset=16382, kv_f32=True)
    rc, _ = runner.run(c, check=False)
    assert rc == vx.NO_WORKSPACE
    assert "staging" in runner.ctx.last_error()


def test_f32_cache_append_and_ring_are_unsupported(runner):
    from conftest import load_package
    vx = load_package().vxfa
    c = cases.decode_case(64, seed=1209, kv_f32=True)
    k_new, v_new = _append_rows(np.random.default_rng(1209), 1, 1, 8 * 128)
    assert runner.run_append(c, k_new, v_new, fused=True, check=False)[0] == vx.UNSUPPORTED
    assert runner.run_ring(c, vx.ring(0, 64), check=False)[0] == vx.UNSUPPORTED
