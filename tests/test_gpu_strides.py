"""Activation rows x_stride apart (wider than D, as rows inside a caller's larger buffer sit): every entry point that
takes x_stride gives the same bits as on the same rows packed. The gap between rows holds fp16 NaNs, so a read past a
row's D values would poison the outputs. Covered: moe.routed on a scratch of at most 16 rows (the decode layer), of
17..128 rows (the prefill path in the scratch's prompt region) and of more (the six-launch sequence);
ea_ffn_moe_decode with the shared expert (one row and four), and fed by the router GEMV; prompt_experts.run with and
without the pair plane."""
import numpy as np
import pytest

import oracle as orc

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

PAD = 96  # values between one row's end and the next row's start


@pytest.fixture(scope="module")
def ea():
    from ea_exl3 import device, linear, moe, prompt_experts, synth

    device.init(0)
    return device, linear, moe, prompt_experts, synth


def _strided(x, D):
    """x [R, D] fp16 / bf16 bits inside a [R, D + PAD] buffer whose gap holds NaN (0x7E00)."""
    R = x.shape[0]
    wide = np.full((R, D + PAD), 0x7E00, np.uint16)
    wide[:, :D] = x.view(np.uint16)
    return wide.view(x.dtype)


@pytest.mark.parametrize("R,cap", [(1, 16), (12, 16), (40, 64), (20, 200)])
def test_moe_routed_strided_rows(ea, R, cap):
    device, linear, moe, pe, synth = ea
    E, D, I, slots = 64, 1024, 256, 8
    pick = synth.picks_uniform(3000 + R, R, E, slots)
    wts = synth.routing_weights(3001 + R, R, slots)
    host = synth.HostLayer(3002 + R, experts=E, dims=D, width=I, k2=8, only=np.unique(pick))
    x = synth.activations(3003 + R, R, D, "f16")
    ex = moe.Routed(host)
    sc = moe.Scratch(ex, cap, slots)
    dp, dw = device.upload(pick), device.upload(wts)
    outs = []
    for xb, stride in ((x, D), (_strided(x, D), D + PAD)):
        dx = device.upload(np.ascontiguousarray(xb))
        out = device.zeros((R, D), torch.float32)
        moe.routed(device.stream(), dx.data_ptr(), stride, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R,
                   x_dtype=0)
        outs.append(device.download(out))
    assert np.isfinite(outs[0]).all()
    np.testing.assert_array_equal(outs[1], outs[0])
    assert device.device_status() == 0


@pytest.mark.parametrize("R", [1, 4])
def test_ffn_decode_strided_rows(ea, R):
    device, linear, moe, pe, synth = ea
    E, D, I = 256, 2048, 256
    logits, bias = synth.logits(3100 + R, R)
    picks = orc.topk8(logits, bias)[0]
    host = synth.HostLayer(3101 + R, experts=E, dims=D, width=I, k2=8, only=np.unique(picks))
    shapes = [(D, I), (D, I), (I, D)]
    lin = [linear.Linear(synth.trellis(3102, 0, m, 0, K, N, 8), synth.scales(3103 + m, K, 1.0),
                         synth.scales(3106 + m, N, 0.02), K, N, 8, 1) for m, (K, N) in enumerate(shapes)]
    x = synth.activations(3110 + R, R, D, "bf16")
    ex = moe.Routed(host)
    sc = moe.Scratch(ex, 16, 8)
    dl, db = device.upload(logits), device.upload(bias)
    outs = []
    for xb, stride in ((x, D), (_strided(x, D), D + PAD)):
        dx = device.upload(np.ascontiguousarray(xb))
        dp, dw = device.zeros((R, 8), torch.int32), device.zeros((R, 8), torch.float32)
        out = device.zeros((R, D), torch.float32)
        moe.ffn_decode(device.stream(), dx.data_ptr(), stride, dl.data_ptr(), db.data_ptr(), 2.5, dp.data_ptr(),
                       dw.data_ptr(), ex, [l.c for l in lin], sc, out.data_ptr(), R, x_dtype=1)
        outs.append(device.download(out))
    assert np.isfinite(outs[0]).all()
    np.testing.assert_array_equal(outs[1], outs[0])
    assert device.device_status() == 0


@pytest.mark.parametrize("planes", [True, False])
def test_prompt_experts_strided_rows(ea, planes):
    device, linear, moe, pe, synth = ea
    R, E, D, I = 96, 32, 512, 256
    pick = synth.picks_zipf(3200, R, 1.1, E, 8)
    wts = synth.routing_weights(3201, R, 8)
    host = synth.HostLayer(3202, experts=E, dims=D, width=I, k2=8, only=np.unique(pick))
    x = synth.activations(3203, R, D, "f16")
    ex = moe.Routed(host)
    sc = pe.Scratch(ex, R, 8, planes=planes)
    dp, dw = device.upload(pick), device.upload(wts)
    outs = []
    for xb, stride in ((x, D), (_strided(x, D), D + PAD)):
        dx = device.upload(np.ascontiguousarray(xb))
        out = device.zeros((R, D), torch.float32)
        pe.run(device.stream(), dx.data_ptr(), stride, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R,
               do_round=False, x_dtype=0)
        outs.append(device.download(out))
    assert np.isfinite(outs[0]).all()
    if planes:  # the slots added in order: the same bits
        np.testing.assert_array_equal(outs[1], outs[0])
    else:  # atomics in arrival order: the same values to fp32 rounding of the order
        np.testing.assert_allclose(outs[1], outs[0], rtol=0, atol=1e-5 * float(np.abs(outs[0]).max()))
    assert device.device_status() == 0


@pytest.mark.parametrize("R", [1, 3])
def test_ffn_decode_router_strided_rows(ea, R):
    """ea_ffn_moe_decode_router: the router GEMV reads the rows x_stride apart too; logits, picks and out the same
    bits as from packed rows."""
    device, linear, moe, pe, synth = ea
    E, D, I = 256, 2048, 256
    rng = np.random.default_rng(3300 + R)
    rw = synth.bf16_bits((0.02 * rng.standard_normal((E, D))).astype(np.float32))
    x = synth.activations(3301 + R, R, D, "f16")
    _, bias = synth.logits(3302, 1)
    picks = orc.topk8(orc.router(x, rw, 0), bias)[0]
    host = synth.HostLayer(3303 + R, experts=E, dims=D, width=I, k2=8, only=np.unique(picks))
    ex = moe.Routed(host)
    sc = moe.Scratch(ex, 16, 8)
    drw, db = device.upload(rw), device.upload(bias)
    got = []
    for xb, stride in ((x, D), (_strided(x, D), D + PAD)):
        dx = device.upload(np.ascontiguousarray(xb))
        dl = device.zeros((R, E), torch.float32)
        dp, dw = device.zeros((R, 8), torch.int32), device.zeros((R, 8), torch.float32)
        out = device.zeros((R, D), torch.float32)
        moe.ffn_decode_router(device.stream(), dx.data_ptr(), stride, drw.data_ptr(), dl.data_ptr(), db.data_ptr(), 2.5,
                              dp.data_ptr(), dw.data_ptr(), ex, None, sc, out.data_ptr(), R, x_dtype=0)
        got.append([device.download(t) for t in (dl, dp, dw, out)])
    for a, b in zip(got[0], got[1]):
        np.testing.assert_array_equal(b, a)
    np.testing.assert_array_equal(got[0][1], picks)
    assert device.device_status() == 0
