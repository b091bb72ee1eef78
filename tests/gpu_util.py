"""Device side of the parity tests: copy a Case's host bytes to the GPU, call
the C ABI through ctypes, read the output back. Inputs on the device are
byte-identical to what the oracle reads."""
from __future__ import annotations

import numpy as np
import torch

from conftest import load_package

vxfa = load_package().vxfa

CANARY = 4096  # floats of guard band on each side of dst
CANARY_BITS = np.uint32(0x7FC0DEAD)  # a NaN payload the kernels never write


def to_device(case):
    return {n: torch.from_numpy(a.view(np.uint8).reshape(-1)).to("cuda") for n, a in case.bufs.items()}


def descs(case, dev):
    out = {}
    for role, (b, t, ne, nb, off) in case.views.items():
        out[role] = vxfa.desc(dev[b].data_ptr() + off, t, ne, nb)
    return out


class Runner:
    """Owns one vxfa context on the current torch stream."""

    def __init__(self):
        self.ctx = vxfa.Context(0)

    def run(self, case, dev=None, check=True):
        dev = dev if dev is not None else to_device(case)
        d = descs(case, dev)
        B, Nq, Hq, D = case.out_shape
        n = B * Nq * Hq * D
        buf = torch.from_numpy(np.full(n + 2 * CANARY, CANARY_BITS, dtype=np.uint32)).to("cuda")
        ne, nb = case.dst_ne_nb()
        dst = vxfa.desc(buf.data_ptr() + 4 * CANARY, vxfa.F32, ne, nb)
        stream = torch.cuda.current_stream().cuda_stream
        rc = self.ctx.flash_attn_ext(d["q"], d["k"], d["v"], d.get("mask"), dst, case.scale,
                                     stream=stream, check=check)
        torch.cuda.synchronize()
        host = buf.cpu().numpy()
        assert (host[:CANARY] == CANARY_BITS).all(), "write before dst"
        assert (host[CANARY + n:] == CANARY_BITS).all(), "write after dst"
        return rc, host[CANARY:CANARY + n].view(np.float32).reshape(B, Nq, Hq, D).copy()

    def run_implicit(self, case, mask_desc, dev=None, check=True):
        """The case's q/k/v through vxfa_flash_attn_ext_implicit (its mask
        tensor, if any, is not passed)."""
        dev = dev if dev is not None else to_device(case)
        d = descs(case, dev)
        B, Nq, Hq, D = case.out_shape
        n = B * Nq * Hq * D
        buf = torch.from_numpy(np.full(n + 2 * CANARY, CANARY_BITS, dtype=np.uint32)).to("cuda")
        ne, nb = case.dst_ne_nb()
        dst = vxfa.desc(buf.data_ptr() + 4 * CANARY, vxfa.F32, ne, nb)
        stream = torch.cuda.current_stream().cuda_stream
        rc = self.ctx.flash_attn_ext_implicit(d["q"], d["k"], d["v"], mask_desc, dst, case.scale,
                                              stream=stream, check=check)
        torch.cuda.synchronize()
        host = buf.cpu().numpy()
        assert (host[:CANARY] == CANARY_BITS).all(), "write before dst"
        assert (host[CANARY + n:] == CANARY_BITS).all(), "write after dst"
        return rc, host[CANARY:CANARY + n].view(np.float32).reshape(B, Nq, Hq, D).copy()

    def run_append(self, case, k_new, v_new, fused=True, check=True):
        """Append the F32 rows k_new / v_new ([Bk, n_new, Hkv * D]) to the last
        rows of the case's k/v cache views and attend: one
        vxfa_flash_attn_ext_append call (fused=True) or vxfa_kv_append then
        vxfa_flash_attn_ext. Returns (rc, out, device buffers after the call)."""
        dev = to_device(case)
        d = descs(case, dev)
        kn = torch.from_numpy(np.ascontiguousarray(k_new, dtype=np.float32)).to("cuda")
        vn = torch.from_numpy(np.ascontiguousarray(v_new, dtype=np.float32)).to("cuda")
        bk, n_new, row = k_new.shape
        ne = (row, n_new, 1, bk)
        nb = (4, 4 * row, 4 * row * n_new, 4 * row * n_new)
        dkn = vxfa.desc(kn.data_ptr(), vxfa.F32, ne, nb)
        dvn = vxfa.desc(vn.data_ptr(), vxfa.F32, ne, nb)
        B, Nq, Hq, D = case.out_shape
        n = B * Nq * Hq * D
        buf = torch.from_numpy(np.full(n + 2 * CANARY, CANARY_BITS, dtype=np.uint32)).to("cuda")
        dne, dnb = case.dst_ne_nb()
        dst = vxfa.desc(buf.data_ptr() + 4 * CANARY, vxfa.F32, dne, dnb)
        stream = torch.cuda.current_stream().cuda_stream
        if fused:
            rc = self.ctx.flash_attn_ext_append(d["q"], d["k"], d["v"], dkn, dvn, d.get("mask"), dst, case.scale,
                                                stream=stream, check=check)
        else:
            rc = self.ctx.kv_append(dkn, dvn, d["k"], d["v"], stream=stream, check=check)
            if rc == 0:
                rc = self.ctx.flash_attn_ext(d["q"], d["k"], d["v"], d.get("mask"), dst, case.scale,
                                             stream=stream, check=check)
        torch.cuda.synchronize()
        host = buf.cpu().numpy()
        assert (host[:CANARY] == CANARY_BITS).all(), "write before dst"
        assert (host[CANARY + n:] == CANARY_BITS).all(), "write after dst"
        after = {name: t.cpu().numpy() for name, t in dev.items()}
        return rc, host[CANARY:CANARY + n].view(np.float32).reshape(B, Nq, Hq, D).copy(), after

    def run_ring(self, case, ring_desc, k_new=None, v_new=None, check=True):
        """vxfa_flash_attn_ext_ring over the case's k/v views (the whole ring),
        optionally appending the F32 rows k_new / v_new ([Bk, 1, Hkv * D]).
        Returns (rc, out, device buffers after the call)."""
        dev = to_device(case)
        d = descs(case, dev)
        dkn = dvn = None
        keep = []
        if k_new is not None:
            kn = torch.from_numpy(np.ascontiguousarray(k_new, dtype=np.float32)).to("cuda")
            vn = torch.from_numpy(np.ascontiguousarray(v_new, dtype=np.float32)).to("cuda")
            keep += [kn, vn]
            bk, n_new, row = k_new.shape
            ne, nb = (row, n_new, 1, bk), (4, 4 * row, 4 * row * n_new, 4 * row * n_new)
            dkn = vxfa.desc(kn.data_ptr(), vxfa.F32, ne, nb)
            dvn = vxfa.desc(vn.data_ptr(), vxfa.F32, ne, nb)
        B, Nq, Hq, D = case.out_shape
        n = B * Nq * Hq * D
        buf = torch.from_numpy(np.full(n + 2 * CANARY, CANARY_BITS, dtype=np.uint32)).to("cuda")
        dne, dnb = case.dst_ne_nb()
        dst = vxfa.desc(buf.data_ptr() + 4 * CANARY, vxfa.F32, dne, dnb)
        stream = torch.cuda.current_stream().cuda_stream
        rc = self.ctx.flash_attn_ext_ring(d["q"], d["k"], d["v"], ring_desc, dkn, dvn, dst, case.scale,
                                          stream=stream, check=check)
        torch.cuda.synchronize()
        host = buf.cpu().numpy()
        assert (host[:CANARY] == CANARY_BITS).all(), "write before dst"
        assert (host[CANARY + n:] == CANARY_BITS).all(), "write after dst"
        after = {name: t.cpu().numpy() for name, t in dev.items()}
        return rc, host[CANARY:CANARY + n].view(np.float32).reshape(B, Nq, Hq, D).copy(), after

    def run_rope(self, case, k_new, v_new, positions, n_dims, freq_base, mode=0, check=True):
        """vxfa_flash_attn_ext_rope: rotate the case's q and k_new (F32
        [Bk, n_new, Hkv * D]) at `positions` (int32 [B * Nq]), append, attend.
        Returns (rc, out, device buffers after the call)."""
        dev = to_device(case)
        d = descs(case, dev)
        kn = torch.from_numpy(np.ascontiguousarray(k_new, dtype=np.float32)).to("cuda")
        vn = torch.from_numpy(np.ascontiguousarray(v_new, dtype=np.float32)).to("cuda")
        pos = torch.from_numpy(np.ascontiguousarray(positions, dtype=np.int32)).to("cuda")
        bk, n_new, row = k_new.shape
        ne, nb = (row, n_new, 1, bk), (4, 4 * row, 4 * row * n_new, 4 * row * n_new)
        dkn = vxfa.desc(kn.data_ptr(), vxfa.F32, ne, nb)
        dvn = vxfa.desc(vn.data_ptr(), vxfa.F32, ne, nb)
        rp = vxfa.rope(pos.data_ptr(), n_dims, freq_base, mode)
        B, Nq, Hq, D = case.out_shape
        n = B * Nq * Hq * D
        buf = torch.from_numpy(np.full(n + 2 * CANARY, CANARY_BITS, dtype=np.uint32)).to("cuda")
        dne, dnb = case.dst_ne_nb()
        dst = vxfa.desc(buf.data_ptr() + 4 * CANARY, vxfa.F32, dne, dnb)
        stream = torch.cuda.current_stream().cuda_stream
        rc = self.ctx.flash_attn_ext_rope(d["q"], d["k"], d["v"], dkn, dvn, rp, d.get("mask"), dst, case.scale,
                                          stream=stream, check=check)
        torch.cuda.synchronize()
        host = buf.cpu().numpy()
        assert (host[:CANARY] == CANARY_BITS).all(), "write before dst"
        assert (host[CANARY + n:] == CANARY_BITS).all(), "write after dst"
        after = {name: t.cpu().numpy() for name, t in dev.items()}
        return rc, host[CANARY:CANARY + n].view(np.float32).reshape(B, Nq, Hq, D).copy(), after

    def close(self):
        self.ctx.close()


def parity(gpu, ref, atol=2e-3, rtol=1e-2):
    """max-abs and relative (Frobenius) error of gpu against ref."""
    ref = ref.astype(np.float64)
    diff = gpu.astype(np.float64) - ref
    maxabs = float(np.abs(diff).max()) if diff.size else 0.0
    den = float(np.linalg.norm(ref))
    rel = float(np.linalg.norm(diff) / den) if den > 0 else float(np.linalg.norm(diff))
    return maxabs, rel, (maxabs <= atol and rel <= rtol)
