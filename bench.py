#!/usr/bin/env python3
"""Benchmark of the gfx950 GGML_OP_FLASH_ATTN_EXT path on one MI355X.

Headline workload (the `value`): audio-encoder self-attention prefill,
1500 frames x 20 heads, hd 64, no mask, scale 1/8, 32 layers with distinct
synthetic N(0,1) tensors. One step = the 32 layer calls. value = algorithmic
TFLOP/s (4*D*Hq per (q, kv) pair). It is measured after every other
configuration, so the GPU has left its idle clocks by then (a few ms of
work after idle ran ~6 % slower than the steady state).

Every configured shape is also measured and reported under "configs":
decode at n_kv 1024 and 8192, decoder prefill 439 causal, the 100-step
sliding-window decode and the 32-stream ragged batch; besides them the
shapes the unchanged application passes: the offline encoder with F32 K/V
(mul_mat outputs), the realtime encoder (1500 frames x 32 heads, hd 64,
sliding-causal window 750, as a mask tensor and as an implicit mask, f16 and
F32 K/V) and decoder prefill against the reference's F32 cache. HBM-bound
shapes rotate over per-layer buffers larger than the 256 MB MALL, so their
bytes come from HBM; the sliding window is also reported warm (one cache).

--stream-sweep adds a sweep of the read-only streaming probe
(bench_stream.hip) over grid sizes and loads in flight, at 30 x 32 MiB and
1 GiB.

The CPU baseline is ggml's one-row algorithm with its AVX2/F16C vector
kernels (oracle/fa_cpu_simd.c, bit-identical to the scalar oracle in
f16-accumulator mode), timed on every configuration at min(hw threads, 16)
threads, voxtral's default, and at every hardware thread.
"""
from __future__ import annotations

import argparse
import ctypes
import importlib.util
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))

MFMA_PEAK_TFLOPS = 2516.6   # MI355X dense f16/bf16: 256 CU x 2.4 GHz x 4096 FLOP/clk
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
HEADLINE_KERNEL = "fa_prefill64_pp"
METRIC = "attn µs/layer; prefill TFLOP/s % MFMA peak; decode HBM GB/s % peak @1 GPU"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def load_package():
    pkg_dir = os.path.join(ROOT, "voxtral.cpp_amd")
    spec = importlib.util.spec_from_file_location(
        "voxtral_cpp_amd", os.path.join(pkg_dir, "__init__.py"), submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["voxtral_cpp_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


PKG = load_package()
vxfa, views = PKG.vxfa, PKG.views


# ---------------------------------------------------------------------------
# synthetic inputs on the device

def randn(torch, shape, seed, sigma=1.0, dtype=None):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn(shape, generator=g, device="cuda", dtype=torch.float32)
    if sigma != 1.0:
        x.mul_(sigma)
    return x.to(dtype) if dtype is not None else x


class Layer:
    """Descriptors of one flash_attn_ext call plus the tensors behind them."""

    def __init__(self, q, k, v, mask, dst, scale, keep, md=None, kn=None, vn=None, fused=True, ring=None,
                 rope=None):
        self.q, self.k, self.v, self.mask, self.dst = q, k, v, mask, dst
        self.scale = scale
        self.keep = keep
        self.md = md   # vxfa_mask_desc for the implicit-mask entry point, else None
        self.kn, self.vn, self.fused = kn, vn, fused   # new K/V rows (F32) to append first, else None
        self.ring = ring   # vxfa_ring: k/v are a ring-buffer cache
        self.rope = rope   # vxfa_rope: rotate q and the appended K rows first


def f32s(x):
    import numpy as np
    return float(np.float32(x))


def encoder_layers(torch, n_layers, seq=1500, heads=20, hd=64, seed=1000, kv_f32=False, mask=None, md=None):
    """Encoder attention layers: q/k/v [seq][heads][hd] viewed as [hd, seq,
    heads] (src/voxtral.cpp:1591-1605); K/V f16, or F32 as the unchanged
    application's mul_mat outputs are; mask: an F16 [seq, seq] tensor (the
    realtime encoder's window), md: an implicit mask descriptor instead."""
    kvt, kty, elt = (torch.float32, vxfa.F32, 4) if kv_f32 else (torch.float16, vxfa.F16, 2)
    out = []
    for i in range(n_layers):
        q = randn(torch, (seq, heads, hd), seed + 3 * i).half().float()  # f16-valued F32, as after mul_mat
        k = randn(torch, (seq, heads, hd), seed + 3 * i + 1, dtype=kvt)
        v = randn(torch, (seq, heads, hd), seed + 3 * i + 2, dtype=kvt)
        dst = torch.empty(seq * heads * hd, device="cuda", dtype=torch.float32)
        mdesc = vxfa.desc(mask.data_ptr(), vxfa.F16, *views.mask(seq, seq)) if mask is not None else None
        out.append(Layer(vxfa.desc(q.data_ptr(), vxfa.F32, *views.encoder_qkv(seq, heads, hd, 4)),
                         vxfa.desc(k.data_ptr(), kty, *views.encoder_qkv(seq, heads, hd, elt)),
                         vxfa.desc(v.data_ptr(), kty, *views.encoder_qkv(seq, heads, hd, elt)),
                         mdesc,
                         vxfa.desc(dst.data_ptr(), vxfa.F32, *views.dst(hd, heads, seq)),
                         f32s(1.0 / math.sqrt(hd)), (q, k, v, dst, mask), md))
    return out


def window_mask(torch, n, window):
    """voxtral's realtime-encoder mask (src/voxtral.cpp:2179-2190, cast to
    F16 at :1564): row q attends kv iff q - window < kv <= q"""
    i_q = torch.arange(n, device="cuda")[:, None]
    i_k = torch.arange(n, device="cuda")[None, :]
    allow = (i_k <= i_q) & (i_k >= i_q - (window - 1))
    return torch.where(allow, 0.0, float("-inf")).to(torch.float16).contiguous()


def window_pairs(n, window):
    """(q, kv) pairs a sliding-causal window leaves: sum over rows of min(q + 1, window)"""
    w = min(n, window)
    return w * (w + 1) // 2 + (n - w) * window


def decode_layers(torch, n_layers, n_kv, hq=32, hkv=8, hd=128, capacity=None, seed=2000, batch=1,
                  kv_sigma=1.0, masks=None, kv_f32=False):
    cap = capacity or n_kv
    kvt = torch.float32 if kv_f32 else torch.float16
    out = []
    for i in range(n_layers):
        q = randn(torch, (batch, 1, hq, hd), seed + 3 * i)
        k = randn(torch, (batch, cap, hkv, hd), seed + 3 * i + 1, kv_sigma, kvt)
        v = randn(torch, (batch, cap, hkv, hd), seed + 3 * i + 2, kv_sigma, kvt)
        dst = torch.empty(batch * hq * hd, device="cuda", dtype=torch.float32)
        qne, qnb = views.decoder_q(1, hq, hd)
        qne = (qne[0], qne[1], qne[2], batch)
        qnb = (qnb[0], qnb[1], qnb[2], hq * hd * 4)
        kne, knb = views.kv_cache(n_kv, hkv, hd, cap, elt=4 if kv_f32 else 2, batch=batch)
        kty = vxfa.F32 if kv_f32 else vxfa.F16
        md = None
        if masks is not None:
            m = masks
            md = vxfa.desc(m.data_ptr(), vxfa.F16, *views.mask(n_kv, 1, 1, batch))
        out.append(Layer(vxfa.desc(q.data_ptr(), vxfa.F32, qne, qnb),
                         vxfa.desc(k.data_ptr(), kty, kne, knb),
                         vxfa.desc(v.data_ptr(), kty, kne, knb),
                         md,
                         vxfa.desc(dst.data_ptr(), vxfa.F32, *views.dst(hd, hq, 1, batch)),
                         f32s(1.0 / math.sqrt(hd)), (q, k, v, dst, masks)))
    return out


def prefill_layers(torch, n_layers, n=439, hq=32, hkv=8, hd=128, seed=3000, kv_f32=False):
    i_q = torch.arange(n, device="cuda")[:, None]
    i_k = torch.arange(n, device="cuda")[None, :]
    mask = torch.where(i_k <= i_q, 0.0, float("-inf")).to(torch.float16).contiguous()
    kvt, kty, elt = (torch.float32, vxfa.F32, 4) if kv_f32 else (torch.float16, vxfa.F16, 2)
    out = []
    for i in range(n_layers):
        q = randn(torch, (n, hq, hd), seed + 3 * i)
        k = randn(torch, (n, hkv, hd), seed + 3 * i + 1, dtype=kvt)
        v = randn(torch, (n, hkv, hd), seed + 3 * i + 2, dtype=kvt)
        dst = torch.empty(n * hq * hd, device="cuda", dtype=torch.float32)
        kne, knb = views.kv_cache(n, hkv, hd, n, elt=elt)
        out.append(Layer(vxfa.desc(q.data_ptr(), vxfa.F32, *views.decoder_q(n, hq, hd)),
                         vxfa.desc(k.data_ptr(), kty, kne, knb),
                         vxfa.desc(v.data_ptr(), kty, kne, knb),
                         vxfa.desc(mask.data_ptr(), vxfa.F16, *views.mask(n, n)),
                         vxfa.desc(dst.data_ptr(), vxfa.F32, *views.dst(hd, hq, n)),
                         f32s(1.0 / math.sqrt(hd)), (q, k, v, dst, mask)))
    return out


# ---------------------------------------------------------------------------
# timing

def time_calls(torch, ctx, calls, steps, warmup, graph=True):
    """Time `steps` passes over `calls` (one step = every call once).

    The step is captured once into a HIP graph (torch.cuda.CUDAGraph records
    the library's launches on the capture stream) and replayed, so the timed
    region measures the kernels rather than the Python ctypes call per layer.
    Events are recorded on the stream the kernels run on. Returns
    (ms per step, µs per call)."""
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()

    def one_step(sh):
        for L in calls:
            if L.rope is not None:   # rotary embedding + append + attention
                ctx.flash_attn_ext_rope(L.q, L.k, L.v, L.kn, L.vn, L.rope, L.mask, L.dst, L.scale, stream=sh)
                continue
            if L.ring is not None:   # decode step over a ring-buffer cache (+ its new row)
                ctx.flash_attn_ext_ring(L.q, L.k, L.v, L.ring, L.kn, L.vn, L.dst, L.scale, stream=sh)
                continue
            if L.kn is not None and L.fused:   # append fused into the attention call
                ctx.flash_attn_ext_append(L.q, L.k, L.v, L.kn, L.vn, L.mask, L.dst, L.scale, stream=sh)
                continue
            if L.kn is not None:   # append, then attention: two calls
                ctx.kv_append(L.kn, L.vn, L.k, L.v, stream=sh)
            if L.md is not None:   # implicit causal / window mask
                ctx.flash_attn_ext_implicit(L.q, L.k, L.v, L.md, L.dst, L.scale, stream=sh)
            else:
                ctx.flash_attn_ext(L.q, L.k, L.v, L.mask, L.dst, L.scale, stream=sh)

    with torch.cuda.stream(stream):   # one eager step loads the kernels before capture
        one_step(stream.cuda_stream)
    torch.cuda.synchronize()
    g = None
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            one_step(stream.cuda_stream)
        torch.cuda.synchronize()
    # untimed warm-up steps, replayed like the timed ones: a few milliseconds
    # of work leave the GPU short of its steady state (the first 20 steps of
    # the encoder after 2 ms of work ran ~6 % slower than the next 20)
    with torch.cuda.stream(stream):
        for _ in range(max(1, warmup)):
            if g is not None:
                g.replay()
            else:
                one_step(stream.cuda_stream)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):   # replay() launches on the current stream
        start.record(stream)
        for _ in range(steps):
            if g is not None:
                g.replay()
            else:
                one_step(stream.cuda_stream)
        end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end)
    return ms / steps, 1000.0 * ms / (steps * len(calls))


def decode_bytes(n_live, hq=32, hkv=8, hd=128, mask_bytes=0, elt=2):
    return n_live * hkv * hd * elt * 2 + hq * hd * 4 * 2 + mask_bytes


# ---------------------------------------------------------------------------
# CPU baseline: ggml's one-row flash_attn_ext with its AVX2/F16C vector
# kernels (oracle/fa_cpu_simd.c), bounded samples of every configuration, at
# voxtral's default thread count min(hw, 16) and at every hardware thread

def _cpu_inputs(kind, seed):
    """Host tensors (oracle Views) of one call of configuration `kind`."""
    import numpy as np
    sys.path.insert(0, ROOT)
    from oracle import oracle
    rng = np.random.default_rng(seed)
    f16 = lambda shape, sigma=1.0: (rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma)).astype(
        np.float16).view(np.uint16)
    V = oracle.View
    if kind in ("encoder", "realtime"):
        seq, heads, hd = 1500, (20 if kind == "encoder" else 32), 64
        q = rng.standard_normal((seq, heads, hd), dtype=np.float32).astype(np.float16).astype(np.float32)
        m = None
        if kind == "realtime":   # sliding-causal window 750 (src/voxtral.cpp:2179-2190)
            iq, ik = np.arange(seq)[:, None], np.arange(seq)[None, :]
            allow = (ik <= iq) & (ik >= iq - 749)
            m = V(np.where(allow, 0, 0xFC00).astype(np.uint16), oracle.F16, *views.mask(seq, seq))
        return (V(q, oracle.F32, *views.encoder_qkv(seq, heads, hd, 4)),
                V(f16((seq, heads, hd)), oracle.F16, *views.encoder_qkv(seq, heads, hd, 2)),
                V(f16((seq, heads, hd)), oracle.F16, *views.encoder_qkv(seq, heads, hd, 2)), m, 0.125)
    scale = f32s(1 / math.sqrt(128))
    if kind in ("decode1024", "decode8192"):
        n_kv = 1024 if kind == "decode1024" else 8192
        kne, knb = views.kv_cache(n_kv, 8, 128, n_kv)
        return (V(rng.standard_normal((1, 32, 128), dtype=np.float32), oracle.F32, *views.decoder_q(1, 32, 128)),
                V(f16((n_kv, 8, 128)), oracle.F16, kne, knb), V(f16((n_kv, 8, 128)), oracle.F16, kne, knb), None, scale)
    if kind == "prefill439":
        n = 439
        kne, knb = views.kv_cache(n, 8, 128, n)
        mask = np.where(np.arange(n)[None, :] <= np.arange(n)[:, None], 0, 0xFC00).astype(np.uint16)
        return (V(rng.standard_normal((n, 32, 128), dtype=np.float32), oracle.F32, *views.decoder_q(n, 32, 128)),
                V(f16((n, 8, 128)), oracle.F16, kne, knb), V(f16((n, 8, 128)), oracle.F16, kne, knb),
                V(mask, oracle.F16, *views.mask(n, n)), scale)
    if kind == "sliding":
        # one step of the streaming decode: cache of 16384 rows, n_kv 16335
        # (the middle of the 100 steps), 2048-row window in the mask
        cap, n_kv, window = 16384, 16335, 2048
        kne, knb = views.kv_cache(n_kv, 8, 128, cap)
        mask = np.zeros(n_kv, dtype=np.uint16)
        mask[: n_kv - window] = 0xFC00
        return (V(rng.standard_normal((1, 32, 128), dtype=np.float32), oracle.F32, *views.decoder_q(1, 32, 128)),
                V(f16((cap, 8, 128)), oracle.F16, kne, knb), V(f16((cap, 8, 128)), oracle.F16, kne, knb),
                V(mask, oracle.F16, *views.mask(n_kv, 1)), scale)
    if kind == "batched":
        # 32 streams of ragged length (the GPU leg's lengths), cache rows past
        # a stream's length are never read (their mask entries are -inf)
        B, cap = 32, 8192
        import torch
        g = torch.Generator(device="cpu")
        g.manual_seed(5)
        lens = torch.randint(512, 8193, (B,), generator=g).numpy()
        k = np.zeros((B, cap, 8, 128), dtype=np.uint16)
        v = np.zeros((B, cap, 8, 128), dtype=np.uint16)
        mask = np.full((B, cap), 0xFC00, dtype=np.uint16)
        for b in range(B):
            k[b, : lens[b]] = f16((int(lens[b]), 8, 128), 0.5)
            v[b, : lens[b]] = f16((int(lens[b]), 8, 128), 0.5)
            mask[b, : lens[b]] = 0
        qne, qnb = views.decoder_q(1, 32, 128)
        qne, qnb = (qne[0], qne[1], qne[2], B), (qnb[0], qnb[1], qnb[2], 32 * 128 * 4)
        kne, knb = views.kv_cache(cap, 8, 128, cap, batch=B)
        return (V(rng.standard_normal((B, 1, 32, 128), dtype=np.float32), oracle.F32, qne, qnb),
                V(k, oracle.F16, kne, knb), V(v, oracle.F16, kne, knb),
                V(mask, oracle.F16, *views.mask(cap, 1, 1, B)), scale)
    raise ValueError(kind)


# configuration -> (input kind, calls timed per repetition, repetitions);
# about 10-11 s of CPU work in all at 16 threads (both thread counts)
CPU_SAMPLES = {
    "encoder_prefill_1500x20_hd64": ("encoder", 1, 61),
    "realtime_encoder_1500x32_hd64_w750": ("realtime", 1, 41),
    "decode_nkv1024": ("decode1024", 50, 41),
    "decode_nkv8192": ("decode8192", 5, 61),
    "decoder_prefill_439_causal": ("prefill439", 1, 61),
    "sliding_window_decode_16k_w2048": ("sliding", 20, 41),
    "batched_ragged_32_streams": ("batched", 1, 61),
}


def cpu_baselines():
    """Median µs per call of every configuration through the vectorised CPU
    restatement, at min(hw, 16) threads (voxtral's default,
    src/voxtral.cpp:1046-1051) and at every hardware thread of this process."""
    import numpy as np
    sys.path.insert(0, ROOT)
    from oracle import oracle
    t_def, t_all = oracle.default_threads(), oracle.host_threads()
    res = {}
    total = 0.0
    for name, (kind, calls, reps) in CPU_SAMPLES.items():
        q, k, v, m, scale = _cpu_inputs(kind, seed=11 + len(res))
        out = None
        row = {}
        for label, thr in (("default", t_def), ("all", t_all)):
            out = oracle.fa_cpu_simd(q, k, v, m, scale, threads=thr, out=out)   # warm-up
            times = []
            for _ in range(reps):
                t0 = time.perf_counter()
                for _ in range(calls):
                    oracle.fa_cpu_simd(q, k, v, m, scale, threads=thr, out=out)
                times.append((time.perf_counter() - t0) / calls)
                total += times[-1] * calls
            row[f"us_per_call_{label}"] = float(np.median(times)) * 1e6
            row[f"threads_{label}"] = thr
        row["sample"] = f"{calls} call(s) x {reps} repetitions per thread count, median"
        res[name] = row
        log(f"[cpu] {name}: {row['us_per_call_default']:.0f} us ({t_def} threads), "
            f"{row['us_per_call_all']:.0f} us ({t_all} threads)")
    return res, t_def, t_all, total


def stream_read_ceiling(torch, steps, warmup):
    """Reference rate for the decode kernels: a plain read-only stream
    (bench_stream.hip: 16-byte loads, eight in flight per thread, 512
    workgroups) over 30 distinct 32 MiB buffers (a decode layer's K/V bytes
    at n_kv 8192; 1 GB in all, past the 256 MB MALL), one launch per buffer,
    replayed from a HIP graph like the decode layers, so it pays the same
    per-launch ramp and tail. Reported as GB/s of buffer bytes."""
    lib = ctypes.CDLL(os.path.join(ROOT, "bench_stream.so"))
    lib.bench_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    n, nbytes = 30, 32 << 20
    bufs = [torch.ones(nbytes // 4, device="cuda", dtype=torch.float32) for _ in range(n)]
    out = torch.zeros(4, device="cuda", dtype=torch.int32)
    stream = torch.cuda.Stream()

    def step():
        for b in bufs:
            if lib.bench_stream_read(b.data_ptr(), nbytes, out.data_ptr(), stream.cuda_stream):
                raise RuntimeError("bench_stream_read launch failed")

    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for _ in range(max(1, warmup)):
            step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        g.replay()
        start.record(stream)
        for _ in range(steps):
            g.replay()
        end.record(stream)
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1000.0 / (steps * n)
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"[hbm read ceiling] 32 MiB read-only stream: {us:.2f} us, {gbs:.0f} GB/s")
    del g, bufs
    torch.cuda.empty_cache()
    return {"us_per_32MiB": us, "gbs": gbs, "frac_hbm_peak": gbs / HBM_PEAK_GBS,
            "method": "bench_stream.hip read-only stream over 30 distinct 32 MiB buffers, HIP-graph replay, "
                      "one launch per buffer"}


def stream_sweep(torch):
    """Read-only streaming probe (bench_stream.hip) over grid sizes and loads
    in flight per thread: 30 distinct 32 MiB buffers (one launch each, a
    decode layer's K/V bytes at n_kv 8192) and one 1 GiB buffer, HIP-graph
    replays. Rows: (bytes per launch, launches, grid, loads, us per launch,
    GB/s)."""
    lib = ctypes.CDLL(os.path.join(ROOT, "bench_stream.so"))
    lib.bench_stream_sweep.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                       ctypes.c_void_p]
    big = torch.ones((1 << 30) // 4, device="cuda", dtype=torch.float32)
    out = torch.zeros(4, device="cuda", dtype=torch.int32)
    stream = torch.cuda.Stream()
    rows = []

    def one(nbytes, nbuf, grid, loads, reps=10):
        def step():
            for i in range(nbuf):
                if lib.bench_stream_sweep(big.data_ptr() + i * nbytes, nbytes, grid, loads, out.data_ptr(),
                                          stream.cuda_stream):
                    raise RuntimeError("bench_stream_sweep launch failed")
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            step()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            for _ in range(3):
                g.replay()
            start.record(stream)
            for _ in range(reps):
                g.replay()
            end.record(stream)
        torch.cuda.synchronize()
        us = start.elapsed_time(end) * 1000.0 / (reps * nbuf)
        rows.append({"bytes": nbytes, "launches": nbuf, "grid": grid, "loads": loads, "us_per_launch": us,
                     "gbs": nbytes / (us * 1e-6) / 1e9})
        log(f"[stream sweep] {nbytes / 2**20:7.0f} MiB x{nbuf:2d} grid {grid:5d} loads {loads:2d}: "
            f"{us:8.2f} us  {rows[-1]['gbs']:6.0f} GB/s")
        del g

    for grid in (256, 512, 1024, 2048, 4096):
        for loads in (4, 8, 16):
            one(32 << 20, 30, grid, loads)
    for grid in (1024, 2048, 4096, 8192, 16384):
        for loads in (8, 16):
            one(1 << 30, 1, grid, loads)
    del big
    torch.cuda.empty_cache()
    best32 = max((r for r in rows if r["launches"] == 30), key=lambda r: r["gbs"])
    best1g = max((r for r in rows if r["launches"] == 1), key=lambda r: r["gbs"])
    return {"rows": rows, "best_32MiB": best32, "best_1GiB": best1g}


def load_traffic(kernel_prefix):
    """HBM bytes per launch of the headline kernel, from the committed PMC
    profile (profiles/encoder_prefill_traffic.json): FETCH_SIZE + WRITE_SIZE
    per dispatch, each scaled by the same counter's reading for a copy kernel
    of known size. None when the profile is absent or names another kernel."""
    path = os.path.join(ROOT, "profiles", "encoder_prefill_traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if not str(t.get("kernel", "")).startswith(kernel_prefix):
        return None
    return t.get("hbm_bytes_per_launch")


def calib_copy(torch, mib=256, reps=3):
    """A plain copy of known size, for scaling the FETCH_SIZE / WRITE_SIZE
    counters in a PMC run (each copy reads and writes `mib` MiB)."""
    n = mib * (1 << 20) // 4
    a = torch.ones(n, device="cuda", dtype=torch.float32)
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    log(f"[calib] copied {mib} MiB x {reps}")


# ---------------------------------------------------------------------------

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", default="", help="comma list of configs to run (debug)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a 256 MiB copy kernel (counter calibration for PMC runs)")
    ap.add_argument("--stream-sweep", action="store_true",
                    help="also sweep the read-only streaming probe over grids and loads in flight")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(attention shards by kv head or stream with no exchange; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    vxfa.load()
    ctx = vxfa.Context(0)
    only = set(args.only.split(",")) if args.only else None
    want = lambda name: only is None or name in only
    K, W = args.steps, args.warmup
    configs = {}

    # --only decode_plain: just the plain decode layers (n_kv 1024 and 8192),
    # for counter runs that must tell those kernels apart
    plain_only = only is not None and "decode_plain" in only
    if want("decode") or want("ceiling") or plain_only:
        configs["hbm_read_ceiling"] = stream_read_ceiling(torch, K, W)

    if want("decode") or plain_only:
        # cold: enough distinct layer caches that one step's reads exceed the
        # 256 MB MALL (n_kv 1024: 80 x 4.2 MB; n_kv 8192: 30 x 33.6 MB)
        for n_kv, layers in ((1024, 80), (8192, 30)):
            dl = decode_layers(torch, layers, n_kv, seed=2000 + n_kv)
            _, us = time_calls(torch, ctx, dl, K, W)
            by = decode_bytes(n_kv)
            gbs = by / (us * 1e-6) / 1e9
            log(f"[decode n_kv={n_kv}] {us:.2f} us/layer  {gbs:.0f} GB/s")
            ceil = configs.get("hbm_read_ceiling", {}).get("gbs")
            configs[f"decode_nkv{n_kv}"] = {"us_per_layer": us, "gbs": gbs, "frac_hbm_peak": gbs / HBM_PEAK_GBS,
                                            "frac_read_ceiling": gbs / ceil if ceil else None,
                                            "bytes_per_layer": by, "layers": layers,
                                            "cache": f"cold ({layers} layer caches, {layers * by / 1e6:.0f} MB "
                                                     "per step > 256 MB MALL)"}
            if n_kv == 8192 and not plain_only:
                # the new token's K/V (F32, one 1024-float row each) appended to the f16 cache:
                # fused into the attention launch, and as a separate append launch
                news = [(randn(torch, (1024,), 7000 + 2 * i), randn(torch, (1024,), 7001 + 2 * i))
                        for i in range(layers)]
                row = lambda t: vxfa.desc(t.data_ptr(), vxfa.F32, (1024, 1, 1, 1), (4, 4096, 4096, 4096))
                res_app = {}
                for fused in (True, False):
                    calls = [Layer(L.q, L.k, L.v, None, L.dst, L.scale, L.keep, None, row(kn), row(vn), fused)
                             for L, (kn, vn) in zip(dl, news)]
                    _, res_app[fused] = time_calls(torch, ctx, calls, K, W)
                # and with the rotary embedding of q and the new K row fused in (position 8191, theta 1e6)
                pos = torch.full((1,), 8191, dtype=torch.int32, device="cuda")
                rp = vxfa.rope(pos.data_ptr(), 128, 1.0e6)
                calls = [Layer(L.q, L.k, L.v, None, L.dst, L.scale, L.keep, None, row(kn), row(vn), True, None, rp)
                         for L, (kn, vn) in zip(dl, news)]
                _, us_rope = time_calls(torch, ctx, calls, K, W)
                log(f"[decode n_kv=8192 + append] fused {res_app[True]:.2f} us/layer; "
                    f"append launch + attention {res_app[False]:.2f} us/layer; "
                    f"rope + append + attention fused {us_rope:.2f} us/layer")
                configs["decode_nkv8192"].update({"append_fused_us_per_layer": res_app[True],
                                                  "append_separate_us_per_layer": res_app[False],
                                                  "rope_append_fused_us_per_layer": us_rope})
                del pos
                del news
            del dl
            torch.cuda.empty_cache()
    if want("decode"):
        # the reference's own F32 cache (src/voxtral.cpp:1126-1136), read in place
        dl = decode_layers(torch, 30, 8192, seed=2500, kv_f32=True)
        _, us = time_calls(torch, ctx, dl, K, W)
        by = decode_bytes(8192, elt=4)
        gbs = by / (us * 1e-6) / 1e9
        log(f"[decode n_kv=8192, F32 cache] {us:.2f} us/layer  {gbs:.0f} GB/s")
        configs["decode_nkv8192_f32_cache"] = {"us_per_layer": us, "gbs": gbs, "frac_hbm_peak": gbs / HBM_PEAK_GBS,
                                               "bytes_per_layer": by, "layers": 30, "cache": "cold (30 layers)"}
        del dl
        torch.cuda.empty_cache()

    if want("prefill"):
        pl = prefill_layers(torch, 30)
        _, us = time_calls(torch, ctx, pl, K, W)
        fl = 4.0 * 128 * 32 * (439 * 440 // 2)
        tf = fl / (us * 1e-6) / 1e12
        log(f"[decoder prefill 439 causal] {us:.2f} us/layer  {tf:.1f} TFLOP/s")
        configs["decoder_prefill_439_causal"] = {"us_per_layer": us, "tflops": tf,
                                                 "frac_mfma_peak": tf / MFMA_PEAK_TFLOPS,
                                                 "flops_per_layer": fl, "layers": 30}
        # the same layers with the causal mask as a descriptor (no mask tensor)
        md = vxfa.mask_desc(vxfa.MASK_CAUSAL, 0, 0)
        impl = [Layer(L.q, L.k, L.v, None, L.dst, L.scale, L.keep, md) for L in pl]
        _, us_i = time_calls(torch, ctx, impl, K, W)
        tf_i = fl / (us_i * 1e-6) / 1e12
        log(f"[decoder prefill 439 causal, implicit mask] {us_i:.2f} us/layer  {tf_i:.1f} TFLOP/s")
        configs["decoder_prefill_439_causal"].update({"implicit_mask_us_per_layer": us_i, "implicit_mask_tflops": tf_i})
        del impl
        del pl
        torch.cuda.empty_cache()

    if want("sliding"):
        cap, n0, window, steps = 16384, 16284, 2048, 100
        res = {}
        # cold: 40 caches, so the 100 steps' windows (40 x 8.4 MB) exceed the 256 MB MALL;
        # warm: one cache, whose window stays MALL-resident from step to step
        for mode, ncache, implicit in (("cold", 40, False), ("warm", 1, False), ("implicit", 40, True)):
            caches = decode_layers(torch, ncache, cap, capacity=cap, seed=4000)
            masks = []
            calls = []
            for t in range(steps):
                n_kv = n0 + t + 1
                m = torch.zeros(n_kv, device="cuda", dtype=torch.float16)
                m[: n_kv - window] = float("-inf")
                masks.append(m)
                L = caches[t % ncache]
                kne, knb = views.kv_cache(n_kv, 8, 128, cap)
                md = vxfa.mask_desc(vxfa.MASK_CAUSAL, window, n_kv - 1) if implicit else None
                mdesc = None if implicit else vxfa.desc(m.data_ptr(), vxfa.F16, *views.mask(n_kv, 1))
                calls.append(Layer(L.q, vxfa.desc(L.k.data, vxfa.F16, kne, knb),
                                   vxfa.desc(L.v.data, vxfa.F16, kne, knb), mdesc, L.dst, L.scale, None, md))
            _, us = time_calls(torch, ctx, calls, max(1, K // 4), 1)
            by = decode_bytes(window, mask_bytes=0 if implicit else 2 * (n0 + steps // 2))
            res[mode] = (us, by / (us * 1e-6) / 1e9)
            del caches, calls, masks
            torch.cuda.empty_cache()
        # the same window kept as a 2048-row ring (logical row p at cache row
        # (start + p) % 2048): each step drops the oldest row and appends its
        # new one in the same launch; 40 rings (336 MB) keep the reads cold
        nr = 40
        rings = decode_layers(torch, nr, window, capacity=window, seed=4100)
        news = [(randn(torch, (1024,), 8000 + 2 * t), randn(torch, (1024,), 8001 + 2 * t)) for t in range(steps)]
        row = lambda t: vxfa.desc(t.data_ptr(), vxfa.F32, (1024, 1, 1, 1), (4, 4096, 4096, 4096))
        calls = []
        for t in range(steps):
            L = rings[t % nr]
            calls.append(Layer(L.q, L.k, L.v, None, L.dst, L.scale, None, None, row(news[t][0]), row(news[t][1]),
                               True, vxfa.ring(t % window, window)))
        _, us_ring = time_calls(torch, ctx, calls, max(1, K // 4), 1)
        res["ring"] = (us_ring, decode_bytes(window) / (us_ring * 1e-6) / 1e9)
        del rings, news, calls
        torch.cuda.empty_cache()
        log(f"[sliding window as a ring + append] {us_ring:.2f} us/step {res['ring'][1]:.0f} GB/s")
        log(f"[sliding window] cold {res['cold'][0]:.2f} us/step {res['cold'][1]:.0f} GB/s; "
            f"warm {res['warm'][0]:.2f} us/step; implicit mask (cold) {res['implicit'][0]:.2f} us/step")
        configs["sliding_window_decode_16k_w2048"] = {
            "us_per_step_cold": res["cold"][0], "gbs_cold": res["cold"][1],
            "frac_hbm_peak_cold": res["cold"][1] / HBM_PEAK_GBS,
            "us_per_step_warm": res["warm"][0], "gbs_warm": res["warm"][1], "steps": steps,
            "implicit_mask_us_per_step_cold": res["implicit"][0], "implicit_mask_gbs_cold": res["implicit"][1],
            "ring_append_us_per_step_cold": res["ring"][0], "ring_append_gbs_cold": res["ring"][1],
            "bytes_per_step": decode_bytes(window, mask_bytes=2 * (n0 + steps // 2))}

    if want("batched"):
        B, cap = 32, 8192
        g = torch.Generator(device="cpu")
        g.manual_seed(5)
        lens = torch.randint(512, 8193, (B,), generator=g)
        mask = torch.zeros(B, cap, dtype=torch.float16)
        for b in range(B):
            mask[b, lens[b]:] = float("-inf")
        mask = mask.cuda()
        bl = decode_layers(torch, 1, cap, batch=B, seed=5000, kv_sigma=0.5, masks=mask)
        _, us = time_calls(torch, ctx, bl, K, W)
        by = int(lens.sum()) * 8 * 128 * 2 * 2 + B * cap * 2 + B * 32 * 128 * 4 * 2
        gbs = by / (us * 1e-6) / 1e9
        log(f"[batched 32 streams] {us:.2f} us/call {gbs:.0f} GB/s")
        configs["batched_ragged_32_streams"] = {"us_per_call": us, "gbs": gbs, "frac_hbm_peak": gbs / HBM_PEAK_GBS,
                                                "bytes_per_call": by, "sum_len": int(lens.sum())}
        del bl
        torch.cuda.empty_cache()

    if want("prefill"):
        # the reference's own F32 cache (src/voxtral.cpp:1126-1136): prefill
        # stages an f16 copy of K and V in the context's workspace first
        pl = prefill_layers(torch, 30, seed=3100, kv_f32=True)
        _, us = time_calls(torch, ctx, pl, K, W)
        fl = 4.0 * 128 * 32 * (439 * 440 // 2)
        log(f"[decoder prefill 439 causal, F32 cache] {us:.2f} us/layer  {fl / (us * 1e-6) / 1e12:.1f} TFLOP/s")
        configs["decoder_prefill_439_causal"].update({"f32_cache_us_per_layer": us,
                                                      "f32_cache_tflops": fl / (us * 1e-6) / 1e12})
        del pl
        torch.cuda.empty_cache()

    if want("realtime"):
        # realtime encoder attention: 1500 frames x 32 heads, hd 64, sliding-
        # causal window 750 (src/voxtral.cpp:2179-2190, cast at :1564, FA at
        # :1611), 32 layers; the mask tensor, the implicit mask, and F32 K/V
        # as the application passes them
        seq, heads, window = 1500, 32, 750
        fl = 4.0 * 64 * heads * window_pairs(seq, window)
        m = window_mask(torch, seq, window)
        res = {}
        for tag, kw in (("mask", dict(mask=m)), ("implicit", dict(md=vxfa.mask_desc(vxfa.MASK_CAUSAL, window, 0))),
                        ("mask_f32_kv", dict(mask=m, kv_f32=True))):
            rl = encoder_layers(torch, 32, seq, heads, 64, seed=6000, **kw)
            _, us = time_calls(torch, ctx, rl, K, W)
            res[tag] = us
            log(f"[realtime encoder 1500x32 w750, {tag}] {us:.2f} us/layer  {fl / (us * 1e-6) / 1e12:.1f} TFLOP/s")
            del rl
            torch.cuda.empty_cache()
        configs["realtime_encoder_1500x32_hd64_w750"] = {
            "us_per_layer": res["mask"], "tflops": fl / (res["mask"] * 1e-6) / 1e12,
            "frac_mfma_peak": fl / (res["mask"] * 1e-6) / 1e12 / MFMA_PEAK_TFLOPS, "flops_per_layer": fl,
            "implicit_mask_us_per_layer": res["implicit"],
            "implicit_mask_tflops": fl / (res["implicit"] * 1e-6) / 1e12,
            "f32_kv_us_per_layer": res["mask_f32_kv"], "layers": 32,
            "note": "q F32 (f16-valued), k/v f16 unless stated; FLOPs count the window's live (q, kv) pairs only"}
        del m

    if want("encoder_f32"):
        # the offline encoder as the unchanged application calls it: K/V are
        # F32 mul_mat outputs (src/voxtral.cpp:1581-1605), staged as f16 first
        el = encoder_layers(torch, 32, seed=1500, kv_f32=True)
        _, us = time_calls(torch, ctx, el, K, W)
        flops_enc = 4.0 * 1500 * 1500 * 64 * 20
        log(f"[encoder, F32 K/V] {us:.2f} us/layer  {flops_enc / (us * 1e-6) / 1e12:.1f} TFLOP/s")
        configs["encoder_prefill_1500x20_hd64_f32_kv"] = {"us_per_layer": us,
                                                           "tflops": flops_enc / (us * 1e-6) / 1e12, "layers": 32}
        del el
        torch.cuda.empty_cache()

    if args.stream_sweep:
        configs["hbm_stream_sweep"] = stream_sweep(torch)

    # --- headline: encoder prefill, 32 layers (after the other configurations: warm GPU) ---
    enc = encoder_layers(torch, 32)
    flops_enc = 4.0 * 1500 * 1500 * 64 * 20
    ms_step, us_layer = time_calls(torch, ctx, enc, K, W)
    tflops = flops_enc / (us_layer * 1e-6) / 1e12
    log(f"[encoder] {us_layer:.2f} us/layer  {tflops:.1f} TFLOP/s")
    configs["encoder_prefill_1500x20_hd64"] = {
        "us_per_layer": us_layer, "tflops": tflops, "frac_mfma_peak": tflops / MFMA_PEAK_TFLOPS,
        "flops_per_layer": flops_enc, "layers": 32, "measured": "last of the GPU configurations"}
    headline = (ms_step, us_layer, tflops)
    del enc
    torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        log("[cpu baseline] every configuration on the host cores ...")
        rows, t_def, t_all, total = cpu_baselines()
        for name, row in rows.items():
            c = configs.setdefault(name, {})
            c["cpu_us_per_call"] = row["us_per_call_default"]
            c["cpu_us_per_call_all_threads"] = row["us_per_call_all"]
            gpu_us = c.get("us_per_layer", c.get("us_per_step_cold", c.get("us_per_call")))
            if gpu_us:
                c["speedup_vs_cpu"] = row["us_per_call_default"] / gpu_us
        enc_us = rows["encoder_prefill_1500x20_hd64"]["us_per_call_default"]
        cpu = {"value": flops_enc / (enc_us * 1e-6) / 1e12, "unit": "TFLOP/s", "cores": t_def, "kind": "port",
               "sample": "every configuration: encoder 1500x20 hd64 (one layer), realtime encoder 1500x32 hd64 "
                         "window 750, decode n_kv 1024 and 8192, decoder prefill 439 causal, one sliding-window "
                         "step (n_kv 16335, window 2048), the 32-stream ragged batch; median of 41-61 repetitions "
                         "per configuration and thread count through oracle/fa_cpu_simd.c (ggml's one-row "
                         "algorithm with AVX2/F16C vector kernels, f16 V accumulation), "
                         f"{total:.1f} s of CPU work",
               "threads_default": t_def, "threads_all": t_all,
               "value_all_threads": flops_enc / (rows["encoder_prefill_1500x20_hd64"]["us_per_call_all"] * 1e-6)
               / 1e12,
               "configs": rows}
        log(f"[cpu baseline] encoder {cpu['value']*1e3:.1f} GFLOP/s at {t_def} threads, "
            f"{cpu['value_all_threads']*1e3:.1f} GFLOP/s at {t_all} threads")

    ms_step, us_layer, tflops = headline
    line = {
        "metric": METRIC,
        "value": tflops,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic, seeded N(0,1) (torch generator on device)",
        "config": {"workload": "audio-encoder self-attention prefill: q/k/v [64, 1500, 20] (q f16-valued F32, "
                               "k/v f16), no mask, scale 1/8, 32 layers per step",
                   "global_batch": 1, "seq_len": 1500, "heads": 20, "head_dim": 64, "layers": 32},
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": tflops / MFMA_PEAK_TFLOPS, "traffic": load_traffic(HEADLINE_KERNEL),
                     "kernel": "fa_prefill64_pp<false, true>", "us_per_launch": us_layer,
                     "traffic_unit": "bytes per launch (FETCH_SIZE + WRITE_SIZE, copy-calibrated)",
                     "algorithmic_bytes": 2 * 1500 * 20 * 64 * 2 + 2 * 1500 * 20 * 64 * 4},
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)
    if args.calib_copy:
        calib_copy(torch)
    ctx.close()


if __name__ == "__main__":
    main()
