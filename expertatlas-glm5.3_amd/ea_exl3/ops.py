"""The routing input and the shared expert's activation: ops.topk (ops.zig:187-191) and swiglu2 (native_ops.cu)."""
from __future__ import annotations

from ._lib import check, lib


def topk(stream: int, logits: int, bias: int, pick: int, wts: int, rows: int, scale: float = 2.5, log: int = 0) -> None:
    """pick int32 / wts fp32 [rows, 8]: sigmoid + bias, top 8 (lower id on ties), wts normalised * scale."""
    check(lib().ea_topk8(stream, logits, bias, pick, wts, rows, scale, log), "topk")


def swiglu2(stream: int, g: int, u: int, out: int, rows: int, width: int) -> None:
    """out = bf16(bf16(silu(g)) * u), bf16 rows of `width`."""
    check(lib().ea_swiglu2(stream, g, u, out, rows, width), "swiglu2")


def add_f32(stream: int, a: int, b: int, n: int) -> None:
    """a += b over n fp32 values (glue.addF32)."""
    check(lib().ea_add_f32(stream, a, b, n), "addF32")
