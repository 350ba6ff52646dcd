"""The routing input and the shared expert's activation: ops.router (ops.zig:131-136), ops.topk (ops.zig:187-191)
and swiglu2 (native_ops.cu)."""
from __future__ import annotations

from ._lib import check, lib


def router(stream: int, x: int, x_stride: int, w: int, part: int, out: int, m: int, d: int, ne: int,
           x_dtype: int = 1) -> None:
    """out fp32 [m, ne] = x [m, d] @ w^T (w bf16 [ne, d]), the reduction in eight slices of d / 8 added in order
    (written to part fp32 [8, m, ne] too when part != 0). x bf16 as the reference's, or fp16 (x_dtype 0)."""
    check(lib().ea_router(stream, x, x_dtype, x_stride, w, part, out, m, d, ne), "router")


def topk(stream: int, logits: int, bias: int, pick: int, wts: int, rows: int, scale: float = 2.5, log: int = 0) -> None:
    """pick int32 / wts fp32 [rows, 8]: sigmoid + bias, top 8 (lower id on ties), wts normalised * scale."""
    check(lib().ea_topk8(stream, logits, bias, pick, wts, rows, scale, log), "topk")


def swiglu2(stream: int, g: int, u: int, out: int, rows: int, width: int) -> None:
    """out = bf16(bf16(silu(g)) * u), bf16 rows of `width`."""
    check(lib().ea_swiglu2(stream, g, u, out, rows, width), "swiglu2")


def add_f32(stream: int, a: int, b: int, n: int) -> None:
    """a += b over n fp32 values (glue.addF32)."""
    check(lib().ea_add_f32(stream, a, b, n), "addF32")
