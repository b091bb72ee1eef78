"""Device side of the parity tests: copy a Case's host bytes to the GPU, call
the C ABI through ctypes, read the output back. Inputs on the device are
byte-identical to what the oracle reads.

Every device buffer sits inside guard bands: dst between CANARY floats of a
NaN payload the kernels never write, each input buffer (q, k, v, mask, new
rows) between GUARD bytes of a fixed pattern. After each call the guards
must be intact, and the inputs the op only reads (q, k, v, mask) must still
hold their host bytes."""
from __future__ import annotations

import numpy as np
import torch

from conftest import load_package

vxfa = load_package().vxfa

CANARY = 4096  # floats of guard band on each side of dst
CANARY_BITS = np.uint32(0x7FC0DEAD)  # a NaN payload the kernels never write
GUARD = 4096   # bytes of guard band on each side of an input buffer (keeps 16-byte alignment)
GUARD_BYTE = 0xA5


def guarded(host: np.ndarray) -> torch.Tensor:
    """A device copy of host's bytes inside guard bands; the returned tensor
    (uint8) is a view of the inner bytes."""
    raw = np.ascontiguousarray(host).view(np.uint8).reshape(-1)
    outer = torch.full((raw.size + 2 * GUARD,), GUARD_BYTE, dtype=torch.uint8, device="cuda")
    inner = outer[GUARD:GUARD + raw.size]
    inner.copy_(torch.from_numpy(raw))
    return inner


def guards_intact(t: torch.Tensor) -> bool:
    """True when t was made by guarded() and its bands still hold the pattern
    (tensors made otherwise have no bands and pass)."""
    st = t.untyped_storage()
    off = t.storage_offset() * t.element_size()
    n = t.numel() * t.element_size()
    if off != GUARD or st.nbytes() != n + 2 * GUARD:
        return True
    full = torch.empty(0, dtype=torch.uint8, device=t.device).set_(st)
    lo, hi = full[:GUARD], full[GUARD + n:]
    return bool((lo == GUARD_BYTE).all().item()) and bool((hi == GUARD_BYTE).all().item())


def to_device(case):
    return {n: guarded(a) for n, a in case.bufs.items()}


def descs(case, dev):
    out = {}
    for role, (b, t, ne, nb, off) in case.views.items():
        out[role] = vxfa.desc(dev[b].data_ptr() + off, t, ne, nb)
    return out


def new_rows(rows):
    """Device copy (guarded) and descriptor of F32 new K/V rows [Bk, n_new, row]."""
    t = guarded(np.ascontiguousarray(rows, dtype=np.float32))
    bk, n_new, row = rows.shape
    ne, nb = (row, n_new, 1, bk), (4, 4 * row, 4 * row * n_new, 4 * row * n_new)
    return t, vxfa.desc(t.data_ptr(), vxfa.F32, ne, nb)


class Runner:
    """Owns one vxfa context on the current torch stream."""

    def __init__(self):
        self.ctx = vxfa.Context(0)

    def _dst(self, case):
        B, Nq, Hq, D = case.out_shape
        n = B * Nq * Hq * D
        buf = torch.from_numpy(np.full(n + 2 * CANARY, CANARY_BITS, dtype=np.uint32)).to("cuda")
        ne, nb = case.dst_ne_nb()
        return buf, vxfa.desc(buf.data_ptr() + 4 * CANARY, vxfa.F32, ne, nb)

    def _finish(self, case, buf, dev, read_only, extra=()):
        """Synchronise, check guards, dst canaries and untouched inputs; return dst."""
        torch.cuda.synchronize()
        B, Nq, Hq, D = case.out_shape
        n = B * Nq * Hq * D
        host = buf.cpu().numpy()
        assert (host[:CANARY] == CANARY_BITS).all(), "write before dst"
        assert (host[CANARY + n:] == CANARY_BITS).all(), "write after dst"
        for name, t in list(dev.items()) + [(f"extra{i}", t) for i, t in enumerate(extra)]:
            assert guards_intact(t), f"write outside buffer {name}"
        for name in read_only:
            if name in dev and name in case.bufs:
                got = dev[name].cpu().numpy()
                want = np.ascontiguousarray(case.bufs[name]).view(np.uint8).reshape(-1)
                assert np.array_equal(got, want), f"input buffer {name} was modified"
        return host[CANARY:CANARY + n].view(np.float32).reshape(B, Nq, Hq, D).copy()

    def _inputs(self, case):
        return [case.views[r][0] for r in ("q", "k", "v", "mask") if r in case.views]

    def run(self, case, dev=None, check=True, verify_inputs=True):
        dev = dev if dev is not None else to_device(case)
        d = descs(case, dev)
        buf, dst = self._dst(case)
        stream = torch.cuda.current_stream().cuda_stream
        rc = self.ctx.flash_attn_ext(d["q"], d["k"], d["v"], d.get("mask"), dst, case.scale,
                                     stream=stream, check=check)
        out = self._finish(case, buf, dev, self._inputs(case) if verify_inputs else ())
        return rc, out

    def run_noalloc(self, case, dev=None, check=True):
        """The case through vxfa_flash_attn_ext_noalloc (no context; the
        library's static scratch) on the current device and stream."""
        dev = dev if dev is not None else to_device(case)
        d = descs(case, dev)
        buf, dst = self._dst(case)
        stream = torch.cuda.current_stream().cuda_stream
        rc = vxfa.flash_attn_ext_noalloc(d["q"], d["k"], d["v"], d.get("mask"), dst, case.scale, stream=stream,
                                         check=check)
        return rc, self._finish(case, buf, dev, self._inputs(case))

    def run_implicit(self, case, mask_desc, dev=None, check=True):
        """The case's q/k/v through vxfa_flash_attn_ext_implicit (its mask
        tensor, if any, is not passed)."""
        dev = dev if dev is not None else to_device(case)
        d = descs(case, dev)
        buf, dst = self._dst(case)
        stream = torch.cuda.current_stream().cuda_stream
        rc = self.ctx.flash_attn_ext_implicit(d["q"], d["k"], d["v"], mask_desc, dst, case.scale,
                                              stream=stream, check=check)
        return rc, self._finish(case, buf, dev, self._inputs(case))

    def run_append(self, case, k_new, v_new, fused=True, check=True):
        """Append the F32 rows k_new / v_new ([Bk, n_new, Hkv * D]) to the last
        rows of the case's k/v cache views and attend: one
        vxfa_flash_attn_ext_append call (fused=True) or vxfa_kv_append then
        vxfa_flash_attn_ext. Returns (rc, out, device buffers after the call)."""
        dev = to_device(case)
        d = descs(case, dev)
        kn, dkn = new_rows(k_new)
        vn, dvn = new_rows(v_new)
        buf, dst = self._dst(case)
        stream = torch.cuda.current_stream().cuda_stream
        if fused:
            rc = self.ctx.flash_attn_ext_append(d["q"], d["k"], d["v"], dkn, dvn, d.get("mask"), dst, case.scale,
                                                stream=stream, check=check)
        else:
            rc = self.ctx.kv_append(dkn, dvn, d["k"], d["v"], stream=stream, check=check)
            if rc == 0:
                rc = self.ctx.flash_attn_ext(d["q"], d["k"], d["v"], d.get("mask"), dst, case.scale,
                                             stream=stream, check=check)
        ro = [case.views[r][0] for r in ("q", "mask") if r in case.views]
        out = self._finish(case, buf, dev, ro, extra=(kn, vn))
        after = {name: t.cpu().numpy() for name, t in dev.items()}
        return rc, out, after

    def run_ring(self, case, ring_desc, k_new=None, v_new=None, check=True):
        """vxfa_flash_attn_ext_ring over the case's k/v views (the whole ring),
        optionally appending the F32 rows k_new / v_new ([Bk, 1, Hkv * D]).
        Returns (rc, out, device buffers after the call)."""
        dev = to_device(case)
        d = descs(case, dev)
        dkn = dvn = None
        extra = ()
        if k_new is not None:
            kn, dkn = new_rows(k_new)
            vn, dvn = new_rows(v_new)
            extra = (kn, vn)
        buf, dst = self._dst(case)
        stream = torch.cuda.current_stream().cuda_stream
        rc = self.ctx.flash_attn_ext_ring(d["q"], d["k"], d["v"], ring_desc, dkn, dvn, dst, case.scale,
                                          stream=stream, check=check)
        ro = [case.views["q"][0]] if k_new is not None else self._inputs(case)
        out = self._finish(case, buf, dev, ro, extra=extra)
        after = {name: t.cpu().numpy() for name, t in dev.items()}
        return rc, out, after

    def run_rope(self, case, k_new, v_new, positions, n_dims, freq_base, mode=0, check=True):
        """vxfa_flash_attn_ext_rope: rotate the case's q and k_new (F32
        [Bk, n_new, Hkv * D]) at `positions` (int32 [B * Nq]), append, attend.
        Returns (rc, out, device buffers after the call)."""
        dev = to_device(case)
        d = descs(case, dev)
        kn, dkn = new_rows(k_new)
        vn, dvn = new_rows(v_new)
        pos = guarded(np.ascontiguousarray(positions, dtype=np.int32))
        rp = vxfa.rope(pos.data_ptr(), n_dims, freq_base, mode)
        buf, dst = self._dst(case)
        stream = torch.cuda.current_stream().cuda_stream
        rc = self.ctx.flash_attn_ext_rope(d["q"], d["k"], d["v"], dkn, dvn, rp, d.get("mask"), dst, case.scale,
                                          stream=stream, check=check)
        ro = [case.views[r][0] for r in ("q", "mask") if r in case.views]
        out = self._finish(case, buf, dev, ro, extra=(kn, vn, pos))
        after = {name: t.cpu().numpy() for name, t in dev.items()}
        return rc, out, after

    def close(self):
        self.ctx.close()


def parity(gpu, ref, atol=2e-3, rtol=1e-2, elem_rtol=1e-2):
    """(max-abs, relative Frobenius error, ok) of gpu against ref; ok also
    requires elem_rel(gpu, ref) <= elem_rtol (the bar's relative tolerance,
    also where atol / rtol are tighter than the bar)."""
    ref = ref.astype(np.float64)
    diff = gpu.astype(np.float64) - ref
    maxabs = float(np.abs(diff).max()) if diff.size else 0.0
    den = float(np.linalg.norm(ref))
    rel = float(np.linalg.norm(diff) / den) if den > 0 else float(np.linalg.norm(diff))
    return maxabs, rel, (maxabs <= atol and rel <= rtol and elem_rel(gpu, ref) <= elem_rtol)


def elem_rel(gpu, ref, floor=0.05):
    """Element-wise relative error max |gpu - ref| / |ref| over the elements
    whose magnitude is at least `floor` of the largest one (outputs near zero
    are held by the max-abs bound instead)."""
    ref = np.asarray(ref, dtype=np.float64)
    top = float(np.abs(ref).max()) if ref.size else 0.0
    if top == 0.0:
        return 0.0
    big = np.abs(ref) >= floor * top
    if not big.any():
        return 0.0
    return float((np.abs(np.asarray(gpu, dtype=np.float64) - ref)[big] / np.abs(ref)[big]).max())
