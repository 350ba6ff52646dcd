"""An EXL3 encoder for synthetic weights: a matrix W [K, N] becomes the format's trellis tiles and input / output
scales, so that the decode path's dense form diag(suh) (H / sqrt 128) W_q (H / sqrt 128) diag(svh) approximates W.
BASELINE's configs draw W ~ N(0, 0.02) in bf16 and quantize it to 16x16 trellis tiles with 128-block random-sign
Hadamard rotations; the reference does this offline with ExLlamaV3 (glm53/weights/convert.sh:75-90), which is not in
this image, so this module is this build's own encoder of the same format:

  - rotation: suh = random signs (the input side), svh = random signs x one scale a column, chosen so that the
    rotated matrix W_q = (H / sqrt 128) diag(suh) W diag(svh)^-1 (H / sqrt 128) has the codebook's RMS;
  - the trellis: each 16x16 tile of W_q is a circular bit stream of 256 values; value p's state is the 16 stream bits
    ending at its last bit (K2 / 2 new bits a value at even K2), its weight the codebook's value of that state. A beam
    search over the stream (width `beam`, the states of the candidate streams, cumulative squared error) picks the
    bits; the stream's wrap-around (the first values' states start with the last values' bits) is closed by a second
    pass that starts from the first pass's tail and is held to write that same tail.

The greedy / beam search is not ExLlamaV3's Viterbi search, so its error is somewhat larger; every bit stream is a
valid tile, and the decode is the format's whatever search produced it. Host-side numpy; sized for test matrices."""
from __future__ import annotations

import numpy as np

from .synth import f16_bits, seed_of


def codebook(cb: int) -> np.ndarray:
    """The codebook's value of every 16-bit state as float32 (decode.cuh:86-120): mcg (1) and 3inst (0) sum the two
    fp16 halves of (x & 0x8FFF8FFF) ^ 0x3B603B60 in fp16; mul1 (2) is fma16(0x6400 + byte sum, 0x1eee, 0xc931)."""
    s = np.arange(65536, dtype=np.uint64)
    if cb == 2:
        x = (s * 0x83DCD12D) & 0xFFFFFFFF
        tot = (x & 255) + ((x >> 8) & 255) + ((x >> 16) & 255) + (x >> 24)
        h = (0x6400 + tot).astype(np.uint16).view(np.float16).astype(np.float64)
        a = np.float64(np.uint16(0x1EEE).view(np.float16))
        c = np.float64(np.uint16(0xC931).view(np.float16))
        return (h * a + c).astype(np.float16).astype(np.float32)
    x = ((s * 0xCBAC1FED) if cb == 1 else (s * 89226354 + 64248484)) & 0xFFFFFFFF
    x = (x & 0x8FFF8FFF) ^ 0x3B603B60
    lo = (x & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float32)
    hi = (x >> 16).astype(np.uint16).view(np.float16).astype(np.float32)
    return (lo + hi).astype(np.float16).astype(np.float32)


def value_place() -> tuple[np.ndarray, np.ndarray]:
    """Value p = 8 L + j of a tile sits at row 2 (L & 3) + (j & 1) + 8 ((j >> 1) & 1), column (L >> 2) + 8 (j >> 2)
    (decode.cuh:134-136)."""
    p = np.arange(256)
    L, j = p >> 3, p & 7
    return 2 * (L & 3) + (j & 1) + 8 * ((j >> 1) & 1), (L >> 2) + 8 * (j >> 2)


def hadamard128() -> np.ndarray:
    i = np.arange(128)
    return np.where(np.bitwise_count(i[:, None] & i[None, :]) % 2 == 1, -1.0, 1.0)


def _rot(a: np.ndarray, axis: int) -> np.ndarray:
    """(H / sqrt 128) applied in 128-blocks along `axis` (H is symmetric and H H = 128 I)."""
    H = hadamard128() / np.sqrt(128.0)
    a = np.moveaxis(a, axis, -1)
    sh = a.shape
    out = (a.reshape(-1, 128) @ H).reshape(sh)
    return np.moveaxis(out, -1, axis)


def encode_tiles(target: np.ndarray, k2: int, lut: np.ndarray, beam: int = 8) -> np.ndarray:
    """Trellis words [T, 4 K2] u32 for T tiles of 256 target values each, in stream order (value p's target at [:, p]).
    Even K2 only (K2 / 2 bits a value)."""
    if k2 % 2:
        raise ValueError("the encoder takes even widths (K2 / 2 whole bits a value)")
    bits = k2 // 2
    T = target.shape[0]
    nsym = 1 << bits
    syms = np.arange(nsym, dtype=np.uint32)
    tail_bits = 16 - bits
    nb = 256 * bits
    tail = np.zeros(T, np.uint32)
    for final in (False, True):
        reg = tail[:, None].copy()  # [T, 1]: the stream's last 16 - bits bits precede value 0
        err = np.zeros((T, 1), np.float64)
        parents = np.zeros((256, T, beam), np.int32)
        chosen = np.zeros((256, T, beam), np.uint8)
        for p in range(256):
            cand = ((reg[:, :, None] << bits) | syms[None, None, :]) & 0xFFFF  # [T, B, nsym]
            ce = err[:, :, None] + (lut[cand] - target[:, p, None, None]) ** 2
            if final and (p + 1) * bits > nb - tail_bits:
                # the last symbols must write the tail this pass started from, so the stream closes on itself
                ok = np.ones((T, nsym), bool)
                for i in range(bits):
                    q = p * bits + i
                    if q >= nb - tail_bits:
                        tb = (tail >> (tail_bits - 1 - (q - (nb - tail_bits)))) & 1
                        ok &= ((syms[None, :] >> (bits - 1 - i)) & 1) == tb[:, None]
                ce = np.where(ok[:, None, :], ce, np.inf)
            flat = ce.reshape(T, -1)
            B = min(beam, flat.shape[1])
            idx = np.argpartition(flat, B - 1, axis=1)[:, :B] if flat.shape[1] > B else np.tile(np.arange(B), (T, 1))
            parent, sym = idx // nsym, idx % nsym
            rows = np.arange(T)[:, None]
            reg = cand.reshape(T, -1)[rows, idx]
            err = flat[rows, idx]
            parents[p, :, :B] = parent
            chosen[p, :, :B] = sym
        best = np.argmin(err, axis=1)
        stream = np.zeros((T, 256), np.uint32)
        b = best
        rows = np.arange(T)
        for p in range(255, -1, -1):
            stream[:, p] = chosen[p, rows, b]
            b = parents[p, rows, b]
        # the tail the next pass starts from: the last 16 - bits stream bits
        acc = np.zeros(T, np.uint32)
        for p in range(256 - (tail_bits + bits - 1) // bits, 256):
            acc = ((acc << bits) | stream[:, p]) & 0xFFFF
        tail = acc & ((1 << tail_bits) - 1)
    # pack: symbols in order, each `bits` wide, most significant first; word w holds stream bits [32 w, 32 w + 32)
    nbits = 256 * bits
    bitarr = np.zeros((T, nbits), np.uint8)
    for i in range(bits):
        bitarr[:, i::bits] = (stream >> (bits - 1 - i)) & 1
    words = np.zeros((T, nbits // 32), np.uint64)
    for i in range(32):
        words = (words << 1) | bitarr[:, i::32].astype(np.uint64)
    return words.astype(np.uint32)


def decode_tiles(words: np.ndarray, k2: int, lut: np.ndarray) -> np.ndarray:
    """The values [T, 256] (stream order) of tiles [T, 4 K2] u32: the encoder's own check of its streams."""
    bits = k2 // 2
    T, nw = words.shape
    nbits = nw * 32
    bitarr = np.zeros((T, nbits), np.uint8)
    for i in range(32):
        bitarr[:, i::32] = (words >> (31 - i)) & 1
    ends = (np.arange(256) + 1) * bits
    out = np.zeros((T, 256), np.float32)
    for p in range(256):
        q = (ends[p] - 16 + np.arange(16)) % nbits
        s = np.zeros(T, np.uint32)
        for b in bitarr[:, q].T:
            s = (s << 1) | b
        out[:, p] = lut[s]
    return out


def quantize(W: np.ndarray, k2: int, cb: int = 1, seed: int = 0, beam: int = 8):
    """W [K, N] (float) -> (trellis words of the expert layout [K/16 * N/16 * 4 K2] u32, suh fp16 bits [K], svh fp16
    bits [N]): tile (kt, nt) at ((kt N/16) + nt) 4 K2 words."""
    K, N = W.shape
    rng = np.random.default_rng(seed_of(seed, 0xE4C))
    lut = codebook(cb)
    su = rng.choice([-1.0, 1.0], K)
    sv = rng.choice([-1.0, 1.0], N)
    # (H / sqrt 128) diag(su) W diag(sv) (H / sqrt 128)
    Wq = _rot(_rot(W.astype(np.float64) * su[:, None] * sv[None, :], 0), 1)
    scale = np.sqrt(np.mean(Wq ** 2)) / np.sqrt(np.mean(lut.astype(np.float64) ** 2))
    Wq = Wq / scale
    rows, cols = value_place()
    tiles = Wq.reshape(K // 16, 16, N // 16, 16).transpose(0, 2, 1, 3).reshape(-1, 16, 16)
    target = tiles[:, rows, cols]  # [T, 256] in stream order
    words = encode_tiles(target.astype(np.float32), k2, lut, beam)
    suh = f16_bits(su)
    svh = f16_bits(sv * scale)
    return words.reshape(-1), suh, svh


def dense(words: np.ndarray, suh: np.ndarray, svh: np.ndarray, K: int, N: int, k2: int, cb: int = 1) -> np.ndarray:
    """The dense matrix diag(suh) (H / sqrt 128) W_q (H / sqrt 128) diag(svh) of encoded tiles (float64)."""
    lut = codebook(cb)
    vals = decode_tiles(words.reshape(-1, 4 * k2), k2, lut)
    rows, cols = value_place()
    tiles = np.zeros((vals.shape[0], 16, 16))
    tiles[:, rows, cols] = vals
    Wq = tiles.reshape(K // 16, N // 16, 16, 16).transpose(0, 2, 1, 3).reshape(K, N)
    su = np.asarray(suh, np.uint16).view(np.float16).astype(np.float64)
    sv = np.asarray(svh, np.uint16).view(np.float16).astype(np.float64)
    return su[:, None] * _rot(_rot(Wq, 0), 1) * sv[None, :]
