"""A MoE layer's routed experts on the device, mirroring moe.zig: the Routed tables (a trellis slab a matrix with
every expert 256-byte aligned, int64 pointer and int32 width tables, stacked suh / svh), the Scratch and `routed`."""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import device
from ._lib import MoeScratch, Routed as _Routed, check, lib
from .synth import HostLayer


def _align(n: int) -> int:
    return (n + 255) & ~255


class Routed:
    """moe.zig Routed (moe.zig:19-37) built from a HostLayer. Experts the host layer did not generate point at a
    shared placeholder of the right size (never read unless picked)."""

    def __init__(self, host: HostLayer):
        self.host = host
        E, D, I = host.count, host.dims, host.width
        self.count, self.dims, self.width, self.cb = E, D, I, host.cb
        self.slabs, self.ptr, self.k2 = [], [], []
        for m in range(3):
            sizes = [int(t.nbytes) if t is not None else 0 for t in host.trellis[m]]
            need = max(sizes)
            offs, total = [], 0
            for s in sizes:
                offs.append(total)
                total += _align(s)
            placeholder_at = total
            total += _align(need)
            buf = np.zeros(total, np.uint8)
            for e, t in enumerate(host.trellis[m]):
                if t is not None:
                    buf[offs[e]: offs[e] + t.nbytes] = t.view(np.uint8)
            slab = device.upload(buf)
            base = slab.data_ptr()
            ptrs = np.array([base + (offs[e] if host.trellis[m][e] is not None else placeholder_at) for e in range(E)],
                            np.int64)
            self.slabs.append(slab)
            self.ptr.append(device.upload(ptrs))
            self.k2.append(device.upload(host.k2[m]))
        self.suh_g, self.suh_u, self.svh_g, self.svh_u, self.suh_d, self.svh_d = (
            device.upload(a) for a in (host.suh_g, host.suh_u, host.svh_g, host.svh_u, host.suh_d, host.svh_d))
        k2gu = np.concatenate([host.k2[0], host.k2[1]])
        self.k2_gu = (int(k2gu.min()), int(k2gu.max()))
        self.k2_d = (int(host.k2[2].min()), int(host.k2[2].max()))
        self.c = self.struct()

    def struct(self) -> _Routed:
        r = _Routed()
        for m in range(3):
            r.ptr[m] = self.ptr[m].data_ptr()
            r.k2[m] = self.k2[m].data_ptr()
        r.suh_g, r.suh_u, r.svh_g, r.svh_u, r.suh_d, r.svh_d = (
            t.data_ptr() for t in (self.suh_g, self.suh_u, self.svh_g, self.svh_u, self.suh_d, self.svh_d))
        r.count, r.dims, r.width, r.cb = self.count, self.dims, self.width, self.cb
        r.k2_gu[0], r.k2_gu[1] = self.k2_gu
        r.k2_d[0], r.k2_d[1] = self.k2_d
        return r


class Scratch:
    """moe.zig Scratch (moe.zig:242-275): one device buffer carved by ea_moe_scratch_init."""

    def __init__(self, ex: Routed, rows: int, slots: int, stream: int | None = None):
        n = lib().ea_moe_scratch_bytes(C.byref(ex.c), rows, slots)
        self.buf = torch.empty(n + 256, dtype=torch.uint8, device="cuda")
        base = (self.buf.data_ptr() + 255) & ~255
        self.c = MoeScratch()
        check(lib().ea_moe_scratch_init(device.stream() if stream is None else stream, C.byref(self.c), base, n,
                                        C.byref(ex.c), rows, slots), "Scratch.init")
        self.rows, self.slots = rows, slots


def routed(stream: int, x: int, x_stride: int, pick: int, wts: int, ex: Routed, s: Scratch, out: int, R: int,
           x_dtype: int = 1) -> None:
    """moe.routed (moe.zig:279-293): out fp32 [R, D] = the routed experts of R rows weighted by wts."""
    check(lib().ea_moe_routed(stream, x, x_dtype, x_stride, pick, wts, C.byref(ex.c), C.byref(s.c), out, R),
          "routed")


def ffn_decode(stream: int, x: int, x_stride: int, logits: int, bias: int, scale: float, pick: int, wts: int,
               ex: Routed, shared, s: Scratch, out: int, R: int, x_dtype: int = 1) -> None:
    """ffnMain's expert part in one call (forward.zig:2361-2403; one launch at one row, five above): top-8 of logits
    into pick / wts, then out fp32 [R, D] = moe.routed(x) + the shared expert's mlp(x). shared: (gate, up, down)
    ctypes ea_linear structs, or None for the routed part alone."""
    arr = None
    if shared is not None:
        from ._lib import Linear as _Linear

        arr = (C.POINTER(_Linear) * 3)(*[C.pointer(l) for l in shared])
    check(lib().ea_ffn_moe_decode(stream, x, x_dtype, x_stride, logits, bias, scale, pick, wts, C.byref(ex.c),
                                  C.addressof(arr) if arr is not None else None,
                                  C.byref(s.c), out, R), "ffn_decode")


def ffn_decode_router(stream: int, x: int, x_stride: int, router_w: int, logits: int, bias: int, scale: float,
                      pick: int, wts: int, ex: Routed, shared, s: Scratch, out: int, R: int, x_dtype: int = 1) -> None:
    """ffn_decode from the normed activations (forward.zig:2350-2403): logits fp32 [R, 256] = x @ router_w^T (bf16
    router weight [256, D], ops.router's eight ordered slices) into `logits`, then ffn_decode on them."""
    arr = None
    if shared is not None:
        from ._lib import Linear as _Linear

        arr = (C.POINTER(_Linear) * 3)(*[C.pointer(l) for l in shared])
    check(lib().ea_ffn_moe_decode_router(stream, x, x_dtype, x_stride, router_w, logits, bias, scale, pick, wts,
                                         C.byref(ex.c), C.addressof(arr) if arr is not None else None, C.byref(s.c),
                                         out, R), "ffn_decode_router")


def ffn_decode_static(stream: int, x: int, x_stride: int, logits: int, bias: int, scale: float, pick: int, wts: int,
                      ex: Routed, shared, out: int, R: int, x_dtype: int = 1) -> None:
    """ffn_decode with no scratch argument (ea_ffn_moe_decode_static): the library's per-device scratch array, for
    callers that cannot allocate; R <= 16; calls overlapping on one device race."""
    arr = None
    if shared is not None:
        from ._lib import Linear as _Linear

        arr = (C.POINTER(_Linear) * 3)(*[C.pointer(l) for l in shared])
    check(lib().ea_ffn_moe_decode_static(stream, x, x_dtype, x_stride, logits, bias, scale, pick, wts, C.byref(ex.c),
                                         C.addressof(arr) if arr is not None else None, out, R), "ffn_decode_static")
