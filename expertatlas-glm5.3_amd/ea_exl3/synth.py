"""Seeded synthetic data for the EXL3 expert path: trellis words, scales, activations, router logits.

Counter-based (SplitMix64 of seed + index), so any host produces the same bytes for the same seed. Any bit stream is
a valid EXL3 tile, so random words are honest weights for timing and parity; the scales give W = diag(suh) H W_q H
diag(svh) / 128 entries of about the BASELINE's N(0, 0.02) size.
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)


def mix64(x):
    """SplitMix64's finaliser (Steele, Lea & Flood 2014) on a uint64 array (or scalar)."""
    with np.errstate(over="ignore"):
        x = np.asarray(x, dtype=np.uint64) + GOLDEN
        x = (x ^ (x >> np.uint64(30))) * M1
        x = (x ^ (x >> np.uint64(27))) * M2
        return x ^ (x >> np.uint64(31))


def seed_of(*parts: int) -> int:
    """One 64-bit seed from several integers."""
    h = np.uint64(0)
    for p in parts:
        h = mix64(h ^ np.uint64(p & 0xFFFFFFFFFFFFFFFF))
    return int(h)


def words(seed: int, n: int) -> np.ndarray:
    """n uint32 words: word i = half (i & 1) of mix64(mix64(seed) + i // 2), the low half first."""
    base = mix64(np.uint64(seed))
    with np.errstate(over="ignore"):
        v = mix64(base + np.arange((n + 1) // 2, dtype=np.uint64))
    return v.view(np.uint32)[:n].copy()


def tile_words(k2: int) -> int:
    return 4 * k2


def matrix_words(K: int, N: int, k2: int) -> int:
    return (K // 16) * (N // 16) * tile_words(k2)


def trellis(seed: int, layer: int, mat: int, expert: int, K: int, N: int, k2: int) -> np.ndarray:
    """One expert matrix's trellis in the expert layout [K/16][N/16][4 K2] (uint32)."""
    return words(seed_of(seed, layer, mat, expert, k2), matrix_words(K, N, k2))


def f16_bits(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float16).view(np.uint16)


def bf16_bits(a) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even."""
    u = np.asarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return u.astype(np.uint16)


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def scales(seed: int, n: int, magnitude: float) -> np.ndarray:
    """fp16 bits of random-sign scales: sign * magnitude * U(0.5, 1.5)."""
    rng = np.random.default_rng(seed_of(seed, 0x5CA1E))
    v = rng.choice([-1.0, 1.0], n) * magnitude * rng.uniform(0.5, 1.5, n)
    return f16_bits(v)


def activations(seed: int, rows: int, dims: int, dtype: str = "f16") -> np.ndarray:
    """x ~ N(0, 1) as fp16 bits (dtype 'f16'), bf16 bits ('bf16') or float32 ('f32')."""
    x = np.random.default_rng(seed_of(seed, 0xAC7)).standard_normal((rows, dims)).astype(np.float32)
    if dtype == "f16":
        return f16_bits(x)
    if dtype == "bf16":
        return bf16_bits(x)
    return x


def logits(seed: int, rows: int, experts: int = 256) -> tuple[np.ndarray, np.ndarray]:
    """Router logits N(0, 1) [rows, experts] and bias N(0, 0.1) [experts], float32."""
    rng = np.random.default_rng(seed_of(seed, 0x106))
    return rng.standard_normal((rows, experts)).astype(np.float32), (0.1 * rng.standard_normal(experts)).astype(np.float32)


def picks_uniform(seed: int, rows: int, experts: int = 256, slots: int = 8) -> np.ndarray:
    """Uniform top-`slots` picks without replacement per row (int32 [rows, slots])."""
    rng = np.random.default_rng(seed_of(seed, 0x71C))
    return np.stack([rng.choice(experts, slots, replace=False) for _ in range(rows)]).astype(np.int32)


def picks_zipf(seed: int, rows: int, s: float = 1.1, experts: int = 256, slots: int = 8) -> np.ndarray:
    """Zipf(s)-skewed top-`slots` picks without replacement per row over a seeded expert ranking."""
    rng = np.random.default_rng(seed_of(seed, 0x21F))
    p = 1.0 / np.arange(1, experts + 1) ** s
    p /= p.sum()
    perm = rng.permutation(experts)
    return np.stack([perm[rng.choice(experts, slots, replace=False, p=p)] for _ in range(rows)]).astype(np.int32)


def routing_weights(seed: int, rows: int, slots: int = 8, scale: float = 2.5) -> np.ndarray:
    """Positive weights summing to `scale` per row (float32 [rows, slots])."""
    w = np.random.default_rng(seed_of(seed, 0x3E7)).uniform(0.05, 1.0, (rows, slots)).astype(np.float32)
    return (w / w.sum(axis=1, keepdims=True) * scale).astype(np.float32)


def mixed_widths(seed: int, experts: int, frac3: float = 0.7) -> np.ndarray:
    """Per-expert K2: frac3 of the experts at 3 bits (K2 6), the rest at 4 bits (K2 8)."""
    rng = np.random.default_rng(seed_of(seed, 0x3B17))
    k2 = np.full(experts, 8, np.int32)
    k2[rng.permutation(experts)[: int(round(frac3 * experts))]] = 6
    return k2


class HostLayer:
    """One layer's routed experts on the host (the moe.zig Routed layout before upload): per matrix (gate, up, down)
    one trellis array per expert; per-expert K2 per matrix (gate and up share it); stacked fp16 suh / svh."""

    def __init__(self, seed: int, experts: int = 256, dims: int = 6144, width: int = 256, k2=8, cb: int = 1,
                 layer: int = 0, only=None):
        self.seed, self.layer, self.count, self.dims, self.width, self.cb = seed, layer, experts, dims, width, cb
        k2 = np.full(experts, k2, np.int32) if np.isscalar(k2) else np.asarray(k2, np.int32)
        self.k2 = [k2.copy(), k2.copy(), k2.copy()]
        D, I = dims, width
        shapes = [(D, I), (D, I), (I, D)]
        keep = set(range(experts)) if only is None else set(int(e) for e in only)
        self.trellis = []
        for m, (K, N) in enumerate(shapes):
            mats = []
            for e in range(experts):
                if e in keep:
                    mats.append(trellis(seed, layer, m, e, K, N, int(self.k2[m][e])))
                else:
                    mats.append(None)
            self.trellis.append(mats)
        self.suh_g = scales(seed_of(seed, layer, 1), experts * D, 1.0)
        self.suh_u = scales(seed_of(seed, layer, 2), experts * D, 1.0)
        self.svh_g = scales(seed_of(seed, layer, 3), experts * I, 0.02)
        self.svh_u = scales(seed_of(seed, layer, 4), experts * I, 0.02)
        self.suh_d = scales(seed_of(seed, layer, 5), experts * I, 1.0)
        self.svh_d = scales(seed_of(seed, layer, 6), experts * D, 0.02)

    def matrix(self, mat: int, e: int) -> np.ndarray:
        t = self.trellis[mat][e]
        if t is None:
            raise KeyError(f"expert {e} matrix {mat} was not generated")
        return t
