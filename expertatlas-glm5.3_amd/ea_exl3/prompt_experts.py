"""Routed experts of prompt chunks, mirroring prompt_experts.zig (supported, Scratch, run) over the C ABI."""
from __future__ import annotations

import ctypes as C

import torch

from ._lib import I32, PromptScratch, check, lib
from .moe import Routed


def supported(ex: Routed) -> bool:
    ok = I32(0)
    check(lib().ea_prompt_experts_supported(C.byref(ex.c), C.byref(ok)), "supported")
    return bool(ok.value)


class Scratch:
    """prompt_experts.zig Scratch: passes of at most 4096 rows; one device buffer carved by the library."""

    def __init__(self, ex: Routed, rows: int, slots: int, planes: bool = True, stream: int = 0):
        n = lib().ea_prompt_scratch_bytes(C.byref(ex.c), rows, slots, int(planes))
        self.buf = torch.empty(n + 256, dtype=torch.uint8, device="cuda")
        base = (self.buf.data_ptr() + 255) & ~255
        self.c = PromptScratch()
        check(lib().ea_prompt_scratch_init(stream or torch.cuda.current_stream().cuda_stream, C.byref(self.c), base, n,
                                           C.byref(ex.c), rows, slots, int(planes)), "Scratch.init")


def run(stream: int, x: int, xstride: int, pick: int, wts: int, ex: Routed, sc: Scratch, out: int, R: int,
        do_round: bool = True, half_sums: bool = False, x_dtype: int = 1) -> None:
    """prompt_experts.run (prompt_experts.zig:146-248): out [R, D] = sum over slots of wts * expert(x)."""
    check(lib().ea_prompt_experts_run(stream, x, x_dtype, xstride, pick, wts, C.byref(ex.c), C.byref(sc.c), out, R,
                                      int(do_round), int(half_sums)), "prompt_experts.run")
