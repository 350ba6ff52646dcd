"""GPU parity at the workloads BASELINE.json names, at their real shapes, through the C ABI against the oracle:

  config 1: one 4-bit EXL3 linear K 6144 x N 2048 at one fp16 row, fp32 out (linear.call; exl3_linear.cu:231-484,
            linear.zig:190-204);
  config 4: the prefill path at 2048 rows (prompt_experts.zig:146-248): Zipf(1.1) routing over 256 4-bit experts,
            so the most picked experts span several items and both item lists are live;
  config 5: the decode layer at one row on full-shape layers with 70 % of the routed experts at 3 bits and the rest
            at 4, routed from logits, three distinct resident layers cycled on one scratch (moe.zig:279-293 and the
            shared expert of forward.zig:2328-2341).

Layer outputs meet the north star's bar, max|diff| <= 2e-3 * RMS(out); picks and weights are bit-exact."""
import numpy as np
import pytest

import oracle as orc
from helpers import assert_close_rms, oracle_routed

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ea():
    from ea_exl3 import device, linear, moe, prompt_experts, synth

    device.init(0)
    return device, linear, moe, prompt_experts, synth


def test_config1_linear_6144x2048_one_row(ea):
    device, linear, _, _, synth = ea
    M, K, N, k2, cb = 1, 6144, 2048, 8, 1
    T = synth.trellis(1001, 0, 0, 0, K, N, k2)
    suh, svh = synth.scales(1002, K, 1.0), synth.scales(1003, N, 0.02)
    x = synth.activations(1004, M, K, "f16")
    lin = linear.Linear(T, suh, svh, K, N, k2, cb)
    tw = 4 * k2
    xh = orc.exl3_rot_in(x, suh, M, K)
    want = orc.exl3_linear(xh, linear.strips(T, K, N, k2), 8 * tw, (K // 16) * 8 * tw, svh, M, K, N, k2, cb, lin.sk,
                           lin.wk, y_dtype=2)
    sc = linear.Scratch(M, K, lin.sk * M * N)
    dx = device.upload(x)
    y = device.zeros((M, N), torch.float32)
    for rep in range(3):  # the split-K counters are back at zero after each call
        linear.call(device.stream(), sc, [lin], dx.data_ptr(), 0, M, [y.data_ptr()], [2])
        np.testing.assert_array_equal(device.download(sc.xh[0][: M * K].view(torch.int16)).reshape(M, K), xh)
        assert_close_rms(device.download(y), want, 1e-4, f"config 1 linear rep {rep}")
        assert int(device.download(lin.counters).sum()) == 0
        # one row takes the tagged hand-off: every slot it used is zero again
        assert not np.any(device.download(sc.z[0]).view(np.uint32)), "tagged slots left behind"
    assert device.device_status() == 0


def test_config1_linear_flag_and_tagged_forms_share_z(ea):
    """16 rows take the flag form (fp32 partial sums left in Z), then 1 and 4 rows the tagged form on the same Z: the
    stale partial sums are never taken for tagged slots (the tag is a NaN pattern no fp32 result has)."""
    device, linear, _, _, synth = ea
    K, N, k2, cb = 6144, 2048, 8, 1
    T = synth.trellis(1011, 0, 0, 0, K, N, k2)
    suh, svh = synth.scales(1012, K, 1.0), synth.scales(1013, N, 0.02)
    lin = linear.Linear(T, suh, svh, K, N, k2, cb)
    tw = 4 * k2
    sc = linear.Scratch(16, K, lin.sk * 16 * N)
    for M in (16, 1, 4, 16, 1):
        x = synth.activations(1014 + M, M, K, "f16")
        want = orc.exl3_linear(orc.exl3_rot_in(x, suh, M, K), linear.strips(T, K, N, k2), 8 * tw, (K // 16) * 8 * tw,
                               svh, M, K, N, k2, cb, lin.sk, lin.wk, y_dtype=2)
        dx = device.upload(x)
        y = device.zeros((M, N), torch.float32)
        linear.call(device.stream(), sc, [lin], dx.data_ptr(), 0, M, [y.data_ptr()], [2])
        assert_close_rms(device.download(y), want, 1e-4, f"config 1 shape, {M} rows after other row counts")
        assert int(device.download(lin.counters).sum()) == 0
    assert device.device_status() == 0


@pytest.mark.parametrize("planes", [True, False])
def test_config4_prefill_2048_rows(ea, planes):
    """2048 rows x 6144 at the real shard shape. The GPU runs every row; the oracle checks every eighth row and the
    last (a row's output depends only on its own activations, picks and weights). With the pair plane all rows are
    bit-equal on a second run; without it (atomics in arrival order) a second run meets the same bar."""
    device, _, moe, pe, synth = ea
    R, E, D, I, slots = 2048, 256, 6144, 256, 8
    pick = synth.picks_zipf(1100, R, 1.1, E, slots)
    wts = synth.routing_weights(1101, R, slots)
    host = synth.HostLayer(1102, experts=E, dims=D, width=I, k2=8, only=np.unique(pick))
    x = synth.activations(1103, R, D, "f16")
    counts = np.bincount(pick.reshape(-1), minlength=E)
    assert counts.max() > 2 * 48  # the most picked expert spans three or more items
    ex = moe.Routed(host)
    assert pe.supported(ex)
    sc = pe.Scratch(ex, R, slots, planes=planes)
    assert (sc.c.plane != 0) == planes
    dx, dp, dw = device.upload(x), device.upload(pick), device.upload(wts)
    out = device.zeros((R, D), torch.float32)
    pe.run(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R,
           do_round=False, x_dtype=0)
    got = device.download(out)
    rows = np.unique(np.concatenate([np.arange(0, R, 8), [R - 1]]))
    want = orc.prompt_experts(np.ascontiguousarray(x[rows]), np.ascontiguousarray(pick[rows]),
                              np.ascontiguousarray(wts[rows]), oracle_routed(host), len(rows), slots)
    assert_close_rms(got[rows], want, 2e-3, f"config 4 prefill R=2048 (sampled rows), planes {planes}")
    assert np.all(np.isfinite(got))
    out2 = device.zeros((R, D), torch.float32)
    pe.run(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out2.data_ptr(), R,
           do_round=False, x_dtype=0)
    if planes:
        np.testing.assert_array_equal(device.download(out2), got)
    else:
        assert_close_rms(device.download(out2)[rows], want, 2e-3, "config 4 prefill R=2048, no plane, second run")
    assert device.device_status() == 0


def test_config5_mixed_width_layers_from_logits(ea):
    """Three distinct full-shape layers (70 % of the routed experts at 3 bits, the rest at 4; 4-bit shared expert)
    cycled twice on one scratch at one row, each routed from its own logits and checked against the oracle's
    topk -> moe.routed -> shared mlp -> add."""
    device, linear, moe, _, synth = ea
    from test_gpu_decode_layer import SharedHost

    E, D, I = 256, 6144, 256
    layers = []
    for l in range(3):
        logits, bias = synth.logits(1200 + l, 1)
        pick_w, wts_w = orc.topk8(logits, bias)
        k2 = synth.mixed_widths(1210 + l, E)
        host = synth.HostLayer(1220 + l, experts=E, dims=D, width=I, k2=k2, only=np.unique(pick_w))
        shared = SharedHost(linear, synth, 1230 + l, D, I, 8, 1)
        layers.append((logits, bias, pick_w, wts_w, host, moe.Routed(host), shared))
    widths = {int(l[4].k2[0][e]) for l in layers for e in l[2][0]}
    assert widths == {6, 8}  # both widths among the picked experts
    sc = moe.Scratch(layers[0][5], 1, 8)
    for call in range(6):
        logits, bias, pick_w, wts_w, host, ex, shared = layers[call % 3]
        x = synth.activations(1240 + call, 1, D, "f16")
        dx, dl, db = device.upload(x), device.upload(logits), device.upload(bias)
        dp, dw = device.zeros((1, 8), torch.int32), device.zeros((1, 8), torch.float32)
        out = device.zeros((1, D), torch.float32)
        moe.ffn_decode(device.stream(), dx.data_ptr(), D, dl.data_ptr(), db.data_ptr(), 2.5, dp.data_ptr(),
                       dw.data_ptr(), ex, [l.c for l in shared.lin], sc, out.data_ptr(), 1, x_dtype=0)
        np.testing.assert_array_equal(device.download(dp), pick_w)
        np.testing.assert_array_equal(device.download(dw), wts_w)
        want = orc.moe_routed(x, pick_w, wts_w, oracle_routed(host), 1, 8) + shared.oracle(x, 1, False)
        assert_close_rms(device.download(out), want, 2e-3, f"config 5 layer {call % 3} call {call}")
    assert device.device_status() == 0


@pytest.mark.parametrize("R", [64, 128])
def test_decode_window_rows_through_prefill(ea, R):
    """moe.routed on decode windows of 17..128 rows (forward.zig:21, moe.zig:279-293) at the full shard shape, config
    3's routing (uniform top-8) and widths (70 % of the experts at 3 bits): the scratch's prompt region runs the prefill
    path's item GEMMs. Every eighth row and the last against the oracle's moe.routed, and the same bits on a second
    run (the slots are added in order)."""
    device, _, moe, _, synth = ea
    E, D, I, slots = 256, 6144, 256, 8
    pick = synth.picks_uniform(1300 + R, R, E, slots)
    wts = synth.routing_weights(1301 + R, R, slots)
    host = synth.HostLayer(1302 + R, experts=E, dims=D, width=I, k2=synth.mixed_widths(1303, E), only=np.unique(pick))
    x = synth.activations(1304 + R, R, D, "f16")
    ex = moe.Routed(host)
    sc = moe.Scratch(ex, R, slots)
    assert sc.c.fused != 0  # the prompt region
    dx, dp, dw = device.upload(x), device.upload(pick), device.upload(wts)
    outs = []
    for _ in range(2):
        out = device.zeros((R, D), torch.float32)
        moe.routed(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R,
                   x_dtype=0)
        outs.append(device.download(out))
    rows = np.unique(np.concatenate([np.arange(0, R, 8), [R - 1]]))
    want = orc.moe_routed(np.ascontiguousarray(x[rows]), np.ascontiguousarray(pick[rows]),
                          np.ascontiguousarray(wts[rows]), oracle_routed(host), len(rows), slots)
    assert_close_rms(outs[0][rows], want, 2e-3, f"moe.routed, {R}-row window")
    np.testing.assert_array_equal(outs[1], outs[0])
    # a window smaller than the scratch: the first 40 rows alone give the same rows' bits
    out = device.zeros((40, D), torch.float32)
    moe.routed(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), 40, x_dtype=0)
    np.testing.assert_array_equal(device.download(out), outs[0][:40])
    assert device.device_status() == 0
