"""The EXL3 encoder of synthetic weights (ea_exl3/encode.py), pinned to the oracle's decode (CPU only):

  - its codebook tables are the oracle's (exhaustive over the 65,536 states, all three codebooks);
  - its stream decode is the oracle's tile decode (random tiles, every even width);
  - a quantized N(0, 0.02) matrix decodes (through the oracle's dequant and the dense identity) to the encoder's own
    dense form bit for bit, and lies within the expected distance of the original: the format round-trips
    realistic weights;
  - the wrap-around of the circular stream is closed: the first values of a tile are no worse than the rest."""
import numpy as np
import pytest

import oracle as orc
from ea_exl3 import encode


@pytest.mark.parametrize("cb", [0, 1, 2])
def test_codebook_is_the_oracles(cb):
    np.testing.assert_array_equal(encode.codebook(cb).astype(np.float16).view(np.uint16), orc.codebook_lut(cb))


@pytest.mark.parametrize("k2", [2, 4, 6, 8, 10, 12, 16])
def test_stream_decode_is_the_oracles(k2):
    rng = np.random.default_rng(k2)
    words = rng.integers(0, 2**32, (6, 4 * k2), dtype=np.uint64).astype(np.uint32)
    got = encode.decode_tiles(words, k2, encode.codebook(1))
    rows, cols = encode.value_place()
    for t in range(6):
        w = orc.decode_tile(words[t], k2, 1).reshape(16, 16)  # fp16 bits [row, col]
        want = w.view(np.float16).astype(np.float32)[rows, cols]
        np.testing.assert_array_equal(got[t], want)


@pytest.mark.parametrize("k2,bound", [(8, 0.2), (6, 0.3), (4, 0.5)])
def test_quantized_matrix_round_trips(k2, bound):
    K, N = 256, 384
    rng = np.random.default_rng(10 + k2)
    W = (0.02 * rng.standard_normal((K, N))).astype(np.float32)
    words, suh, svh = encode.quantize(W, k2, 1, seed=k2, beam=8)
    Wd = encode.dense(words, suh, svh, K, N, k2, 1)
    # the oracle's view of the same tiles: W_q from its dequant, then diag(suh) (H/sqrt128) W_q (H/sqrt128) diag(svh)
    Wq = orc.dequant_expert(words, K, N, k2, 1).view(np.float16).astype(np.float64)
    H = encode.hadamard128() / np.sqrt(128.0)
    blk = np.kron(np.eye(K // 128), H), np.kron(np.eye(N // 128), H)
    su = suh.view(np.float16).astype(np.float64)
    sv = svh.view(np.float16).astype(np.float64)
    W_or = su[:, None] * (blk[0] @ Wq @ blk[1]) * sv[None, :]
    np.testing.assert_allclose(Wd, W_or, rtol=0, atol=1e-12)
    rel = np.sqrt(np.mean((Wd - W) ** 2)) / np.sqrt(np.mean(W.astype(np.float64) ** 2))
    assert rel < bound, rel
    # a wrong scale or a transposed placement would not come close
    assert rel < 0.6 * np.sqrt(np.mean((W.T[:K, :K] if K <= N else W) ** 2)) / np.sqrt(np.mean(W ** 2)) + bound


def test_stream_wrap_is_closed():
    rng = np.random.default_rng(3)
    lut = encode.codebook(1)
    target = rng.choice(lut, (64, 256)).astype(np.float32)  # targets the codebook can hit exactly
    words = encode.encode_tiles(target, 8, lut, beam=8)
    got = encode.decode_tiles(words, 8, lut)
    err = (got - target) ** 2
    assert np.mean(err[:, :3]) <= 4 * np.mean(err[:, 3:]) + 1e-6
