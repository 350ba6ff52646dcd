"""Whole layers generated straight into device memory (seeded torch generator on the GPU): the bench's resident
expert shards, too large to build on the host. Any bit stream is a valid EXL3 tile, so random words are honest
weights for timing; the layout is exactly moe.zig's (one 256-byte-aligned slab per matrix, int64 pointer and int32
width tables, stacked fp16 scales) and linear.zig's strips for the shared expert."""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import device
from ._lib import Linear as _Linear, Routed as _Routed
from .linear import plan


def _words(gen: torch.Generator, n: int) -> torch.Tensor:
    return torch.randint(-(2**31), 2**31 - 1, (n,), dtype=torch.int32, device="cuda", generator=gen)


def _scales(gen: torch.Generator, n: int, magnitude: float) -> torch.Tensor:
    sign = torch.randint(0, 2, (n,), device="cuda", generator=gen).to(torch.float32) * 2 - 1
    mag = torch.rand(n, device="cuda", generator=gen) + 0.5
    return (sign * mag * magnitude).to(torch.float16)


class DeviceRouted:
    """One layer's routed experts (gate, up, down of E experts) resident on the device."""

    def __init__(self, seed: int, experts: int = 256, dims: int = 6144, width: int = 256, k2=8, cb: int = 1):
        gen = torch.Generator(device="cuda")
        gen.manual_seed(seed)
        E, D, I = experts, dims, width
        k2s = np.full(E, k2, np.int32) if np.isscalar(k2) else np.asarray(k2, np.int32)
        self.k2_host = k2s
        self.count, self.dims, self.width, self.cb = E, D, I, cb
        shapes = [(D, I), (D, I), (I, D)]
        self.slabs, self.ptr, self.k2, self.bytes, self.offs = [], [], [], [], []
        for (K, N) in shapes:
            sizes = [(K // 16) * (N // 16) * 4 * int(w) * 4 for w in k2s]
            offs = np.concatenate([[0], np.cumsum([(s + 255) & ~255 for s in sizes])]).astype(np.int64)
            slab = _words(gen, int(offs[-1]) // 4)
            self.slabs.append(slab)
            self.offs.append(offs)
            self.ptr.append(device.upload(offs[:-1] + slab.data_ptr()))
            self.k2.append(device.upload(k2s))
            self.bytes.append(np.array(sizes, np.int64))
        self.suh_g, self.suh_u = _scales(gen, E * D, 1.0), _scales(gen, E * D, 1.0)
        self.svh_g, self.svh_u = _scales(gen, E * I, 0.02), _scales(gen, E * I, 0.02)
        self.suh_d, self.svh_d = _scales(gen, E * I, 1.0), _scales(gen, E * D, 0.02)
        self.c = _Routed()
        for m in range(3):
            self.c.ptr[m] = self.ptr[m].data_ptr()
            self.c.k2[m] = self.k2[m].data_ptr()
        (self.c.suh_g, self.c.suh_u, self.c.svh_g, self.c.svh_u, self.c.suh_d, self.c.svh_d) = (
            t.data_ptr() for t in (self.suh_g, self.suh_u, self.svh_g, self.svh_u, self.suh_d, self.svh_d))
        self.c.count, self.c.dims, self.c.width, self.c.cb = E, D, I, cb
        self.c.k2_gu[0], self.c.k2_gu[1] = int(k2s.min()), int(k2s.max())
        self.c.k2_d[0], self.c.k2_d[1] = int(k2s.min()), int(k2s.max())

    def expert_bytes(self, e: int) -> int:
        """Trellis + scale bytes one expert's three matrices occupy (what a layer reads for it once)."""
        D, I = self.dims, self.width
        return int(sum(b[e] for b in self.bytes)) + 2 * (2 * D + 2 * I + I + D)

    def total_bytes(self) -> int:
        return int(sum(s.numel() * 4 for s in self.slabs))

    def host_copy(self, experts) -> dict:
        """The named experts' trellis words (per matrix: {expert: uint32 array}), the width table and every stacked
        scale, copied to host memory (synchronous): what a host-side check of this layer reads."""
        out = {"trellis": [{}, {}, {}], "k2": self.k2_host.copy(), "dims": self.dims, "width": self.width,
               "cb": self.cb, "count": self.count}
        for m in range(3):
            for e in sorted(set(int(e) for e in experts)):
                a, b = int(self.offs[m][e]) // 4, int(self.offs[m][e] + self.bytes[m][e]) // 4
                out["trellis"][m][e] = self.slabs[m][a:b].cpu().numpy().view(np.uint32).copy()
        for name in ("suh_g", "suh_u", "svh_g", "svh_u", "suh_d", "svh_d"):
            out[name] = getattr(self, name).view(torch.int16).cpu().numpy().view(np.uint16).copy()
        return out


class DeviceLinear:
    """One EXL3 linear (strips layout) resident on the device, (sk, wk) from plan()."""

    def __init__(self, gen: torch.Generator, k: int, n: int, k2: int = 8, cb: int = 1):
        self.k, self.n, self.k2, self.cb = k, n, k2, cb
        self.sk, self.wk = plan(k, n)
        self.words = _words(gen, (k // 16) * (n // 16) * 4 * k2)
        self.suh = _scales(gen, k, 1.0)
        self.svh = _scales(gen, n, 0.02)
        self.counters = torch.zeros(8 * (n // 128), dtype=torch.int32, device="cuda")
        self.c = _Linear(self.words.data_ptr(), self.suh.data_ptr(), self.svh.data_ptr(), self.counters.data_ptr(),
                         k, n, k2, cb, self.sk, self.wk)

    def bytes(self) -> int:
        return self.words.numel() * 4 + 2 * (self.k + self.n)

    def host_copy(self) -> dict:
        """Words (strips layout), suh, svh and the plan, copied to host memory (synchronous)."""
        return {"words": self.words.cpu().numpy().view(np.uint32).copy(),
                "suh": self.suh.view(torch.int16).cpu().numpy().view(np.uint16).copy(),
                "svh": self.svh.view(torch.int16).cpu().numpy().view(np.uint16).copy(),
                "k": self.k, "n": self.n, "k2": self.k2, "cb": self.cb, "sk": self.sk, "wk": self.wk}


class DeviceShared:
    """The shared expert of a TP=8 rank: gate and up (D -> I) and down (I -> D)."""

    def __init__(self, seed: int, dims: int = 6144, width: int = 256, k2: int = 8, cb: int = 1):
        gen = torch.Generator(device="cuda")
        gen.manual_seed(seed)
        self.gate = DeviceLinear(gen, dims, width, k2, cb)
        self.up = DeviceLinear(gen, dims, width, k2, cb)
        self.down = DeviceLinear(gen, width, dims, k2, cb)

    def bytes(self) -> int:
        return self.gate.bytes() + self.up.bytes() + self.down.bytes()

    def host_copy(self) -> list:
        return [self.gate.host_copy(), self.up.host_copy(), self.down.host_copy()]


def linear_ptrs(ls):
    return (C.POINTER(_Linear) * len(ls))(*[C.pointer(l.c) for l in ls])
