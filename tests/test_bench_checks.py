"""bench.py's parity checks (the oracle recomputing a timed leg's kept layer) on the CPU: fed the oracle's own output
they pass; fed an output with one planted mistake (a dropped slot, a wrong pick, one column off by 1 %) they fail.
The inputs are in the layout the bench copies off the GPU (DeviceRouted.host_copy / DeviceLinear.host_copy)."""
import numpy as np
import pytest

import bench
import oracle as orc
from ea_exl3 import linear, synth

D, I, E = 6144, 256, 256


def _layer_copy(host: synth.HostLayer, experts) -> dict:
    return {"trellis": [{int(e): host.trellis[m][int(e)] for e in experts} for m in range(3)], "k2": host.k2[0],
            "dims": host.dims, "width": host.width, "cb": host.cb, "count": host.count, "suh_g": host.suh_g,
            "suh_u": host.suh_u, "svh_g": host.svh_g, "svh_u": host.svh_u, "suh_d": host.suh_d, "svh_d": host.svh_d}


def _linear_copy(seed: int, K: int, N: int, k2: int = 8) -> dict:
    sk, wk = linear.plan(K, N)
    return {"words": linear.strips(synth.trellis(seed, 0, 0, 0, K, N, k2), K, N, k2),
            "suh": synth.scales(seed + 1, K, 1.0), "svh": synth.scales(seed + 2, N, 0.02), "k": K, "n": N, "k2": k2,
            "cb": 1, "sk": sk, "wk": wk}


@pytest.fixture(scope="module")
def decode_case():
    R = 2
    logits, bias = synth.logits(71, R)
    pick, wts = orc.topk8(logits, bias)
    host = synth.HostLayer(72, experts=E, dims=D, width=I, k2=synth.mixed_widths(73, E), only=np.unique(pick))
    shared = [_linear_copy(74, D, I), _linear_copy(75, D, I), _linear_copy(76, I, D)]
    x = synth.activations(77, R, D, "f16")
    d = {"j": 0, "rows": list(range(R)), "R": R, "x": x, "logits": logits, "bias": bias, "pick": pick.copy(),
         "wts": wts.copy(), "layer": _layer_copy(host, np.unique(pick)), "shared": shared, "sequence": False}
    want = orc.moe_routed(x, pick, wts, bench._host_routed(orc, d["layer"]), R, 8)
    d["out"] = want + bench._shared_oracle(orc, shared, x, R)
    return d


def test_decode_check_accepts_the_oracle(decode_case):
    res = bench.decode_check(orc, decode_case)
    assert res["ok"] and res["picks_bit_exact"] and res["max_diff_over_rms"] == 0.0


@pytest.mark.parametrize("mistake", ["dropped_slot", "wrong_pick", "column"])
def test_decode_check_rejects_a_planted_mistake(decode_case, mistake):
    d = dict(decode_case)
    if mistake == "dropped_slot":  # the output without slot 3's expert
        p, w = d["pick"].copy(), d["wts"].copy()
        w2 = w.copy()
        w2[:, 3] = 0.0
        routed = bench._host_routed(orc, d["layer"])
        d["out"] = orc.moe_routed(d["x"], p, w2, routed, 2, 8) + bench._shared_oracle(orc, d["shared"], d["x"], 2)
    elif mistake == "wrong_pick":
        p = d["pick"].copy()
        p[0, 0], p[0, 1] = p[0, 1], p[0, 0]
        d["pick"] = p
    else:
        o = d["out"].copy()
        o[1, 77] *= 1.01
        o[1, 77] += 0.5 * float(np.sqrt(np.mean(o.astype(np.float64) ** 2)))
        d["out"] = o
    assert not bench.decode_check(orc, d)["ok"]


def test_prefill_and_linear_checks():
    R = 3
    pick = synth.picks_zipf(81, R, 1.1, E, 8)
    wts = synth.routing_weights(82, R, 8)
    host = synth.HostLayer(83, experts=E, dims=D, width=I, k2=8, only=np.unique(pick))
    x = synth.activations(84, R, D, "f16")
    d = {"R": 512, "rows": [0, 1, 2], "x": x, "pick": pick, "wts": wts, "layer": _layer_copy(host, np.unique(pick))}
    d["out"] = orc.prompt_experts(x, pick, wts, bench._host_routed(orc, d["layer"]), R, 8)
    assert bench.prefill_check(orc, d)["ok"]
    d["out"] = d["out"].copy()
    d["out"][2, 5000] = np.nan
    assert not bench.prefill_check(orc, d)["ok"]

    lin = _linear_copy(85, D, 2048)
    xl = synth.activations(86, 1, D, "f16")
    tw = 32
    y = orc.exl3_linear(orc.exl3_rot_in(xl, lin["suh"], 1, D), lin["words"], 8 * tw, (D // 16) * 8 * tw, lin["svh"], 1,
                        D, 2048, 8, 1, lin["sk"], lin["wk"], y_dtype=2)
    dl = {"x": xl, "out": y, "lin": lin}
    assert bench.linear_check(orc, dl)["ok"]
    dl["out"] = y * np.float32(1.001)
    assert not bench.linear_check(orc, dl)["ok"]
