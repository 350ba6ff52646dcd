"""The tuned CPU baseline (oracle/cpu_layer.c, timed by bench.py's cpu_baseline leg) computes the oracle's moe.routed:
the same layer at the decode shapes, within 2e-3 RMS (only the fp32 summation order differs: the oracle follows the
kernels' K splits, the baseline sums each column tile's k in order), for one row and sixteen, 3- and 4-bit experts,
fp16 and bf16 activations. CPU only."""
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
