"""The tuned CPU baselines (oracle/cpu_layer.c, timed by bench.py's cpu_baseline leg) compute the oracle's functions:
moe.routed at the decode shapes within 2e-3 RMS (only the fp32 summation order differs: the oracle follows the
kernels' K splits, the baseline sums each column tile's k in order), for one row and sixteen, 3- and 4-bit experts,
fp16 and bf16 activations; and one EXL3 linear (rot_in, product, output rotation) within 1e-4 RMS, at config 1's
shape and two others. CPU only."""
import numpy as np
import pytest

import oracle as orc
from ea_exl3 import synth
from helpers import assert_close_rms, oracle_routed


@pytest.mark.parametrize("R,D,I,k2,bf16", [(1, 1024, 256, 8, False), (16, 512, 128, "mixed", True),
                                           (3, 2048, 256, 6, False)])
def test_cpu_baseline_matches_oracle(R, D, I, k2, bf16):
    E = 64
    k2v = synth.mixed_widths(3, E) if k2 == "mixed" else k2
    pick = synth.picks_uniform(40 + R, R, E, 8)
    wts = synth.routing_weights(41 + R, R, 8)
    host = synth.HostLayer(42 + R, experts=E, dims=D, width=I, k2=k2v, only=np.unique(pick))
    x = synth.activations(43 + R, R, D, "bf16" if bf16 else "f16")
    r = oracle_routed(host)
    want = orc.moe_routed(x, pick, wts, r, R, 8, bf16=bf16)
    got = orc.cpu_moe_routed(x, pick, wts, r, R, 8, bf16=bf16)
    assert_close_rms(got, want, 2e-3, "cpu baseline")
    assert np.max(np.abs(got - want)) > 0 or R == 1  # a different summation order, not the oracle itself


@pytest.mark.parametrize("M,K,N,k2,cb,bf16", [(1, 6144, 2048, 8, 1, False), (5, 1024, 512, 6, 0, False),
                                              (3, 2048, 256, 10, 2, True)])
def test_cpu_linear_matches_oracle(M, K, N, k2, cb, bf16):
    """The tuned CPU linear (config 1's baseline) against the oracle's rot_in then linear (one split, one warp: k in
    ascending order, as the baseline sums), within 1e-4 RMS: fp32 sums in a different grouping only."""
    from ea_exl3 import linear

    T = synth.trellis(1300 + k2, 0, 0, 0, K, N, k2)
    suh, svh = synth.scales(1301, K, 1.0), synth.scales(1302, N, 0.02)
    x = synth.activations(1303 + M, M, K, "bf16" if bf16 else "f16")
    S = linear.strips(T, K, N, k2)
    tw = 4 * k2
    xh = orc.exl3_rot_in(x, suh, M, K, bf16=bf16)
    want = orc.exl3_linear(xh, S, 8 * tw, (K // 16) * 8 * tw, svh, M, K, N, k2, cb, 1, 1, y_dtype=2)
    got = orc.cpu_exl3_linear(x, suh, S, svh, M, K, N, k2, cb, bf16=bf16)
    assert_close_rms(got, want, 1e-4, "cpu linear")
    # the RMS difference is at the fp32 rounding level of a reordered sum
    assert np.sqrt(np.mean((got - want) ** 2)) < 1e-5 * np.sqrt(np.mean(want ** 2))
