"""Routed-expert kernels of the decode path, mirroring experts.zig's Kernels (experts.zig:73-211): the same calls,
argument meaning and error names, over the C ABI. Addresses are device pointers (ints)."""
from __future__ import annotations

import ctypes as C

from . import device
from ._lib import GroupedArgs, check, lib

F16, BF16, F32 = 0, 1, 2


class Kernels:
    """experts.Kernels: `load` once per device, then the five launches."""

    def __init__(self, dev: int = 0):
        device.init(dev)

    @classmethod
    def load(cls, dev: int = 0) -> "Kernels":
        return cls(dev)

    def group(self, stream: int, pick: int, uids: int, ucount: int, members: int, rows: int, slots: int, experts: int,
              maxm: int) -> None:
        check(lib().ea_experts_group(stream, pick, uids, ucount, members, rows, slots, experts, maxm), "group")

    def rot_in(self, stream: int, x: int, x_stride: int, pick: int, suh0: int, suh1: int, out0: int, out1: int,
               rows: int, kdim: int, slots: int, experts: int, x_dtype: int = BF16) -> None:
        check(lib().ea_experts_rot_in(stream, x, x_dtype, x_stride, pick, suh0, suh1, out0, out1, rows, kdim, slots,
                                      experts), "rotIn")

    def grouped(self, stream: int, a: GroupedArgs) -> None:
        check(lib().ea_experts_grouped(stream, C.byref(a)), "grouped")

    def gateup_epilogue(self, stream: int, z: int, pick: int, svh_g: int, svh_u: int, suh_d: int, xd: int, rows: int,
                        p: int, n: int, sk: int, slots: int, experts: int, limit: float, act_mode: int) -> None:
        check(lib().ea_experts_gateup_epilogue(stream, z, pick, svh_g, svh_u, suh_d, xd, rows, p, n, sk, slots,
                                               experts, limit, act_mode), "gateupEpilogue")

    def down_combine(self, stream: int, z: int, pick: int, svh_d: int, y: int, wts: int, out: int, rows: int, p: int,
                     d: int, sk: int, slots: int, experts: int) -> None:
        check(lib().ea_experts_down_combine(stream, z, pick, svh_d, y, wts, out, rows, p, d, sk, slots, experts),
              "downCombine")


def grouped_args(**kw) -> GroupedArgs:
    """GroupedArgs with the reference's defaults (experts.zig:41-67: ns 0)."""
    a = GroupedArgs()
    for k, v in kw.items():
        setattr(a, k, v)
    return a
