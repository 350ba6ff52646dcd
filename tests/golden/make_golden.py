"""Writes the golden fixtures of this directory from the CPU oracle (oracle/liboracle.so) and the seeded input
generator (ea_exl3.synth):

    python tests/golden/make_golden.py

golden.npz holds, for each case, the generator's parameters, a SHA-256 of the generated inputs (so a change in the
generator is caught, not silently re-fixtured) and the oracle's outputs:
  - cb_lut_sha256[cb]: the 65,536-entry fp16 codebook tables (decode.cuh:86-120) of mcg, mul1 and 3inst;
  - tile_<k2>_<cb>: one 16x16 trellis tile (words) and its decoded fp16 bits, K2 in 2..16, every codebook;
  - topk: router logits / bias of 6 rows (with exact ties) and the top-8 picks and weights;
  - layer_r1 / layer_r16: a reduced-width MoE layer (E 16, D 512, I 128, 3- and 4-bit experts) through moe.routed,
    fp32 outputs of R = 1 and R = 16 rows.
The reference ships no golden vectors for this path; these pin this build's oracle and HIP path against regressions,
while the oracle itself is pinned by the independent checks in tests/test_oracle_*.py.
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "expertatlas-glm5.3_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import oracle as orc  # noqa: E402
from ea_exl3 import synth  # noqa: E402

OUT = os.path.join(HERE, "golden.npz")
TILE_WIDTHS = list(range(2, 17))
LAYER = dict(E=16, D=512, I=128, seed=901)


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def tile_case(k2: int, cb: int):
    T = synth.words(synth.seed_of(77, k2, cb), 4 * k2)
    return T, orc.decode_tile(T, k2, cb).astype(np.uint16)


def topk_case():
    logits, bias = synth.logits(55, 6)
    logits[2, :] = 0.5         # all sigmoids tied: the picks follow the bias, then the id
    logits[3, 7] = logits[3, 9] = 4.0
    bias = bias.copy()
    bias[9] = bias[7]          # an exact tie between two strong experts: the lower id first
    pick, wts = orc.topk8(logits, bias)
    return logits, bias, pick, wts


def layer_case(R: int):
    E, D, I, seed = LAYER["E"], LAYER["D"], LAYER["I"], LAYER["seed"]
    k2 = synth.mixed_widths(seed, E)
    pick = synth.picks_uniform(seed + R, R, E, 8)
    wts = synth.routing_weights(seed + 2 * R, R, 8)
    host = synth.HostLayer(seed, experts=E, dims=D, width=I, k2=k2, only=np.unique(pick))
    x = synth.activations(seed + 3 * R, R, D, "f16")
    mats = []
    for m in range(3):
        real = [t for t in host.trellis[m] if t is not None]
        mats.append([t if t is not None else np.zeros_like(real[0]) for t in host.trellis[m]])
    routed = orc.Routed(mats, host.k2, host.suh_g, host.suh_u, host.svh_g, host.svh_u, host.suh_d, host.svh_d, D, I,
                        host.cb)
    out = orc.moe_routed(x, pick, wts, routed, R, 8)
    digest = sha(x, pick, wts, host.k2[0], host.suh_g, host.suh_u, host.svh_g, host.svh_u, host.suh_d, host.svh_d,
                 *[t for m in range(3) for t in host.trellis[m] if t is not None])
    return host, x, pick, wts, out, digest


def main() -> None:
    data = {}
    data["cb_lut_sha256"] = np.array([sha(orc.codebook_lut(cb)) for cb in range(3)])
    for k2 in TILE_WIDTHS:
        for cb in range(3):
            T, W = tile_case(k2, cb)
            data[f"tile_{k2}_{cb}_words"] = T
            data[f"tile_{k2}_{cb}_w"] = W
    logits, bias, pick, wts = topk_case()
    data.update(topk_logits=logits, topk_bias=bias, topk_pick=pick, topk_wts=wts)
    for R in (1, 16):
        _, _, _, _, out, digest = layer_case(R)
        data[f"layer_r{R}_out"] = out
        data[f"layer_r{R}_inputs_sha256"] = np.array(digest)
    np.savez_compressed(OUT, **data)
    print(OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
