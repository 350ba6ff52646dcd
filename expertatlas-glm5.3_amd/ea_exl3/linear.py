"""EXL3 linears mirroring exl3.zig (Kernels.rotIn / linear / unpackW) and linear.zig (Linear, plan, call,
callRotated) over the C ABI."""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import device
from ._lib import MAX_JOBS, Jobs, Linear as _Linear, LinearScratch, RotJobs, U32, U64, check, lib

F16, BF16, F32 = 0, 1, 2


def plan(k: int, n: int) -> tuple[int, int]:
    """linear.zig:61-79 (plan): (K splits, warps) from the shape alone."""
    sk, wk = U32(), U32()
    lib().ea_linear_plan(k, n, C.byref(sk), C.byref(wk))
    return sk.value, wk.value


def strips(T: np.ndarray, K: int, N: int, k2: int) -> np.ndarray:
    """[K/16, N/16, TW] -> [N/128, K/16, 8, TW] (linear.zig:99-107)."""
    tw = 4 * k2
    return np.ascontiguousarray(T.reshape(K // 16, N // 128, 8, tw).transpose(1, 0, 2, 3)).reshape(-1)


class Linear:
    """linear.zig Linear: words in the strips layout, fp16 suh / svh, counters, (sk, wk) from plan()."""

    def __init__(self, trellis_expert_layout: np.ndarray, suh: np.ndarray, svh: np.ndarray, k: int, n: int, k2: int,
                 cb: int):
        self.k, self.n, self.k2, self.cb = k, n, k2, cb
        self.sk, self.wk = plan(k, n)
        self.words = device.upload(strips(trellis_expert_layout, k, n, k2))
        self.suh = device.upload(suh)
        self.svh = device.upload(svh)
        self.counters = device.zeros(8 * (n // 128), torch.int32)
        self.c = _Linear(self.words.data_ptr(), self.suh.data_ptr(), self.svh.data_ptr(), self.counters.data_ptr(),
                         k, n, k2, cb, self.sk, self.wk)

    def strides(self) -> tuple[int, int]:
        tw = 4 * self.k2
        return 8 * tw, (self.k // 16) * 8 * tw


class Scratch:
    """linear.zig Scratch: xh fp16 [M, K] a layer and Z fp32 [SK, M, N] a layer with SK > 1. Z starts zero, as the
    counters do: the small-row kernel's tagged hand-off leaves every slot it used zero again."""

    def __init__(self, max_rows: int, max_k: int, max_zn: int):
        self.xh = [device.empty(max_rows * max_k, torch.float16) for _ in range(MAX_JOBS)]
        self.z = [device.zeros(max(max_zn, 1), torch.float32) for _ in range(MAX_JOBS)]
        self.c = LinearScratch()
        for i in range(MAX_JOBS):
            self.c.xh[i] = self.xh[i].data_ptr()
            self.c.z[i] = self.z[i].data_ptr()


def _arrays(ls, outs, dtypes):
    arr = (C.POINTER(_Linear) * len(ls))(*[C.pointer(l.c) for l in ls])
    o = (U64 * len(outs))(*outs)
    d = (C.c_int * len(dtypes))(*dtypes)
    return arr, o, d


def call(stream: int, s: Scratch, ls, x: int, x_dtype: int, m: int, outs, out_dtypes) -> None:
    """linear.call (linear.zig:164-178): outs[j] = x @ W_j for 1..3 groupable layers, one rot_in + one linear."""
    arr, o, d = _arrays(ls, outs, out_dtypes)
    check(lib().ea_linear_call(stream, C.byref(s.c), arr, len(ls), x, x_dtype, m, o, d), "linear.call")


def call_rotated(stream: int, s: Scratch, ls, m: int, outs, out_dtypes) -> None:
    arr, o, d = _arrays(ls, outs, out_dtypes)
    check(lib().ea_linear_call_rotated(stream, C.byref(s.c), arr, len(ls), m, o, d), "linear.callRotated")


class Kernels:
    """exl3.Kernels (exl3.zig:57-137)."""

    def __init__(self, dev: int = 0):
        device.init(dev)

    def rot_in(self, stream: int, x: int, x_dtype: int, suh, xh, m: int, kdim: int) -> None:
        j = RotJobs()
        for i, (a, b) in enumerate(zip(suh, xh)):
            j.suh[i], j.xh[i] = a, b
        check(lib().ea_exl3_rot_in(stream, x, x_dtype, C.byref(j), len(suh), m, kdim), "rotIn")

    def linear(self, stream: int, jobs: Jobs, m: int, kdim: int, k2: int, cb: int, wk: int, loads: int = 3) -> None:
        check(lib().ea_exl3_linear(stream, C.byref(jobs), m, kdim, k2, cb, wk, loads), "linear")

    def unpack_w(self, stream: int, t: int, w: int, kdim: int, n: int, k2: int, cb: int, stride_k: int,
                 stride_nb: int) -> None:
        check(lib().ea_exl3_unpack(stream, t, w, kdim, n, k2, cb, stride_k, stride_nb), "unpackW")
