"""GPU parity of the EXL3 linear (the shared expert) and the prefill path through the C ABI against the CPU oracle:
unpack bit-exact, rot_in bit-exact, linear outputs within fp32-accumulation tolerance with the split-K counters
left at zero, the route exactly, and prompt_experts.run within 2e-3 * RMS(out) (also deterministic run to run)."""
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


def _case(synth, M, K, N, k2, seed):
    T = synth.trellis(seed, 0, 0, 0, K, N, k2)
    suh = synth.scales(seed + 1, K, 1.0)
    svh = synth.scales(seed + 2, N, 0.02)
    x = synth.activations(seed + 3, M, K, "bf16")
    return T, suh, svh, x


@pytest.mark.parametrize("k2,cb", [(8, 1), (10, 2), (12, 2), (6, 1)])
def test_unpack_bit_exact(ea, k2, cb):
    device, linear, _, _, synth = ea
    K, N = 256, 512
    T = synth.trellis(60, 0, 0, 0, K, N, k2)
    S = linear.strips(T, K, N, k2)
    tw = 4 * k2
    want = orc.dequant_expert(T, K, N, k2, cb)
    dS, dW = device.upload(S), device.zeros((K, N), torch.int16)
    linear.Kernels().unpack_w(device.stream(), dS.data_ptr(), dW.data_ptr(), K, N, k2, cb, 8 * tw, (K // 16) * 8 * tw)
    np.testing.assert_array_equal(device.download(dW), want)


@pytest.mark.parametrize("M,K,N,k2,cb,y_dtype", [
    (1, 6144, 256, 8, 1, 1),     # the shared expert's gate / up at batch 1 (plan: SK 8, WK 4), bf16 out
    (1, 256, 6144, 8, 1, 2),     # its down (SK 1), fp32 out
    (16, 6144, 256, 10, 2, 2),   # 5-bit mul1 (the real checkpoints' shared expert), 16 rows
    (40, 1024, 640, 8, 2, 0),    # three row passes, fp16 out
    (128, 512, 384, 6, 1, 2),    # the most rows a call takes
    (128, 6144, 256, 8, 1, 1),   # the shared expert's gate / up on a 128-row window: 8 row passes x 8 K splits at once
    (96, 256, 6144, 8, 1, 2),    # its down on a 96-row window
    (4, 6144, 2048, 8, 1, 2),    # config 1's shape at four rows (the small-row kernel: 32-column groups x 8 splits)
    (7, 2048, 512, 6, 1, 0),     # 3 bits, fp16 out, a ragged row count
    (2, 1024, 384, 4, 1, 2),     # 2 bits
    (3, 2048, 512, 12, 2, 2),    # 6-bit mul1 (widths above 10: the register-streaming kernel at any row count)
    (5, 1024, 384, 8, 2, 1),     # 4-bit mul1, bf16 out
    (1, 8192, 256, 8, 1, 2),     # SK 16: the tagged finisher polls eight splits
    (3, 8192, 512, 6, 1, 1),     # the same at three rows, 3 bits, bf16 out
])
def test_linear_call(ea, M, K, N, k2, cb, y_dtype):
    device, linear, _, _, synth = ea
    T, suh, svh, x = _case(synth, M, K, N, k2, 61 + M)
    lin = linear.Linear(T, suh, svh, K, N, k2, cb)
    xh_w = orc.exl3_rot_in(x, suh, M, K, bf16=True)
    tw = 4 * k2
    y_w = orc.exl3_linear(xh_w, linear.strips(T, K, N, k2), 8 * tw, (K // 16) * 8 * tw, svh, M, K, N, k2, cb, lin.sk,
                          lin.wk, y_dtype=2)
    sc = linear.Scratch(128, K, lin.sk * 128 * N)
    dx = device.upload(x)
    y = device.zeros((M, N), torch.float32 if y_dtype == 2 else torch.int16)
    for rep in range(2):  # twice: the counters must be back at zero after each call
        linear.call(device.stream(), sc, [lin], dx.data_ptr(), 1, M, [y.data_ptr()], [y_dtype])
        np.testing.assert_array_equal(device.download(sc.xh[0][: M * K].view(torch.int16)).reshape(M, K), xh_w)
        got = device.download(y)
        if y_dtype == 2:
            assert_close_rms(got, y_w, 1e-4, f"linear M={M} rep={rep}")
        else:  # one rounding to fp16 / bf16 of the fp32 result: half an ulp of the format, plus the fp32 slack
            got = got.view(np.float16).astype(np.float32) if y_dtype == 0 else synth.bf16_to_f32(got)
            eps = 2.0 ** -11 if y_dtype == 0 else 2.0 ** -8
            bound = eps * np.abs(y_w) + 1e-4 * np.sqrt(np.mean(y_w.astype(np.float64) ** 2))
            assert np.all(np.abs(got - y_w) <= bound), f"linear M={M}: rounded output off"
        assert int(device.download(lin.counters).sum()) == 0


def test_linear_call_rotated_matches_call(ea):
    """callRotated on the xh a call leaves in the scratch (the small-row kernel reads it instead of rotating) gives
    the call's result bit for bit; fp16 and bf16 inputs."""
    device, linear, _, _, synth = ea
    M, K, N, k2 = 3, 6144, 2048, 8
    T, suh, svh, x = _case(synth, M, K, N, k2, 90)
    lin = linear.Linear(T, suh, svh, K, N, k2, 1)
    sc = linear.Scratch(M, K, lin.sk * M * N)
    for x_dtype in (0, 1):
        xb = synth.activations(91 + x_dtype, M, K, ["f16", "bf16"][x_dtype])
        dx = device.upload(xb)
        y1, y2 = device.zeros((M, N), torch.float32), device.zeros((M, N), torch.float32)
        linear.call(device.stream(), sc, [lin], dx.data_ptr(), x_dtype, M, [y1.data_ptr()], [2])
        np.testing.assert_array_equal(device.download(sc.xh[0][: M * K].view(torch.int16)).reshape(M, K),
                                      orc.exl3_rot_in(xb, suh, M, K, bf16=x_dtype == 1))
        linear.call_rotated(device.stream(), sc, [lin], M, [y2.data_ptr()], [2])
        np.testing.assert_array_equal(device.download(y1), device.download(y2))
        assert int(device.download(lin.counters).sum()) == 0
    assert device.device_status() == 0


def test_linear_three_jobs_one_launch(ea):
    device, linear, _, _, synth = ea
    M, K = 3, 1024
    shapes = [(256, 8), (512, 8), (128, 8)]
    lins, wants, outs = [], [], []
    x = synth.activations(70, M, K, "f16")
    for i, (N, k2) in enumerate(shapes):
        T = synth.trellis(71 + i, 0, 0, 0, K, N, k2)
        suh, svh = synth.scales(72 + i, K, 1.0), synth.scales(73 + i, N, 0.02)
        lin = linear.Linear(T, suh, svh, K, N, k2, 1)
        lins.append(lin)
        xh = orc.exl3_rot_in(x, suh, M, K)
        tw = 4 * k2
        wants.append(orc.exl3_linear(xh, linear.strips(T, K, N, k2), 8 * tw, (K // 16) * 8 * tw, svh, M, K, N, k2,
                                     1, lin.sk, lin.wk))
        outs.append(device.zeros((M, N), torch.float32))
    sc = linear.Scratch(M, K, max(l.sk * M * l.n for l in lins))
    dx = device.upload(x)
    linear.call(device.stream(), sc, lins, dx.data_ptr(), 0, M, [o.data_ptr() for o in outs], [2, 2, 2])
    for o, w, l in zip(outs, wants, lins):
        assert_close_rms(device.download(o), w, 1e-4, "job")
        assert int(device.download(l.counters).sum()) == 0


def test_linear_errors(ea):
    device, linear, _, _, synth = ea
    from ea_exl3._lib import EaError

    T, suh, svh, x = _case(synth, 1, 256, 128, 8, 80)
    a = linear.Linear(T, suh, svh, 256, 128, 8, 1)
    T2 = synth.trellis(81, 0, 0, 0, 512, 128, 8)
    b = linear.Linear(T2, synth.scales(82, 512, 1.0), svh, 512, 128, 8, 1)
    sc = linear.Scratch(1, 512, 4096)
    y = device.zeros((1, 128), torch.float32)
    dx = device.upload(x)
    with pytest.raises(EaError) as e:  # different K: not groupable (linear.zig:133-138)
        linear.call(device.stream(), sc, [a, b], dx.data_ptr(), 1, 1, [y.data_ptr()] * 2, [2, 2])
    assert e.value.code == 14
    with pytest.raises(EaError) as e:  # 129 rows
        linear.call(device.stream(), sc, [a], dx.data_ptr(), 1, 129, [y.data_ptr()], [2])
    assert e.value.code == 14


# ---- prefill -------------------------------------------------------------------------------------------------------

def _prompt_case(ea, R, E, D, I, k2, seed, x_dtype=1, zipf=True, cb=1, planes=True):
    device, _, moe, pe, synth = ea
    slots = 8
    pick = synth.picks_zipf(seed, R, 1.1, E, slots) if zipf else synth.picks_uniform(seed, R, E, slots)
    wts = synth.routing_weights(seed + 1, R, slots)
    host = synth.HostLayer(seed + 2, experts=E, dims=D, width=I, k2=k2, cb=cb, only=np.unique(pick))
    x = synth.activations(seed + 3, R, D, ["f16", "bf16", "f32"][x_dtype])
    ex = moe.Routed(host)
    assert pe.supported(ex)
    sc = pe.Scratch(ex, R, slots, planes=planes)
    dx, dp, dw = device.upload(x), device.upload(pick), device.upload(wts)
    return host, ex, sc, x, pick, wts, dx, dp, dw


@pytest.mark.parametrize("R,E,D,I,k2", [(130, 64, 512, 256, 8), (300, 256, 1024, 256, "mixed"), (40, 32, 256, 128, 6),
                                        (120, 32, 256, 128, 12), (300, 32, 256, 128, 12), (300, 32, 256, 128, 8),
                                        # widths above 10 take the register-streaming GEMM with items of up to 112
                                        # pairs; Zipf over 32 experts gives the top experts ~300 pairs: three items
                                        (300, 32, 256, 128, 11), (300, 32, 256, 128, 14), (300, 32, 256, 128, 16),
                                        (260, 32, 512, 256, "wide-mixed")])
def test_prompt_experts_run(ea, R, E, D, I, k2):
    device, _, _, pe, synth = ea
    if k2 == "wide-mixed":  # every width class on the register-streaming path at once
        k2v = np.array([(12, 8, 6, 16, 10, 11, 4, 14)[e % 8] for e in range(E)], np.int32)
    else:
        k2v = synth.mixed_widths(5, E) if k2 == "mixed" else k2
    host, ex, sc, x, pick, wts, dx, dp, dw = _prompt_case(ea, R, E, D, I, k2v, 100 + R)
    want = orc.prompt_experts(x, pick, wts, oracle_routed(host), R, 8, bf16=True)
    out = device.zeros((R, D), torch.float32)
    pe.run(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R, do_round=False)
    got = device.download(out)
    assert_close_rms(got, want, 2e-3, "prompt experts")
    # the same bits on a second run (slots added in order, no atomics in the sums)
    out2 = device.zeros((R, D), torch.float32)
    pe.run(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out2.data_ptr(), R, do_round=False)
    np.testing.assert_array_equal(device.download(out2), got)
    # do_round: each value through bf16
    pe.run(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out2.data_ptr(), R, do_round=True)
    np.testing.assert_array_equal(device.download(out2), synth.bf16_to_f32(synth.bf16_bits(got)))
    assert device.device_status() == 0


@pytest.mark.parametrize("planes", [True, False])
def test_prompt_experts_full_shape_512(ea, planes):
    """BASELINE config 4 at its real shape: 512 rows, D 6144, I 256, 256 experts, Zipf(1.1), 4 bits, fp16 x; with the
    pair plane and without it."""
    device, _, _, pe, synth = ea
    R, D = 512, 6144
    host, ex, sc, x, pick, wts, dx, dp, dw = _prompt_case(ea, R, 256, D, 256, 8, 200, x_dtype=0, planes=planes)
    want = orc.prompt_experts(x, pick, wts, oracle_routed(host), R, 8)
    out = device.zeros((R, D), torch.float32)
    pe.run(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R,
           do_round=False, x_dtype=0)
    assert_close_rms(device.download(out), want, 2e-3, "prompt experts R=512")


@pytest.mark.parametrize("k2", [2, 3, 4, 5, 7, 9, 10])
def test_prompt_experts_every_staged_width(ea, k2):
    """The staged item GEMMs' widths the tests above leave out (K2 6 and 8 are theirs), through both item lists (Zipf
    over 32 experts at 160 rows gives items of both sizes), with the pair plane."""
    device, _, _, pe, synth = ea
    R, E, D, I = 160, 32, 512, 256
    host, ex, sc, x, pick, wts, dx, dp, dw = _prompt_case(ea, R, E, D, I, k2, 900 + k2)
    want = orc.prompt_experts(x, pick, wts, oracle_routed(host), R, 8, bf16=True)
    out = device.zeros((R, D), torch.float32)
    pe.run(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R, do_round=False)
    assert_close_rms(device.download(out), want, 2e-3, f"prompt experts, K2 {k2}")
    assert device.device_status() == 0


@pytest.mark.parametrize("planes", [True, False])
def test_prompt_experts_f32_activations(ea, planes):
    """fp32 activations (x_dtype 2: the rotation launch reads them and rounds the rotated rows to fp16 as for 16-bit
    ones), with the pair plane and without it, against the oracle on the same fp32 rows."""
    device, _, _, pe, synth = ea
    R, E, D, I = 96, 32, 512, 256
    host, ex, sc, x, pick, wts, dx, dp, dw = _prompt_case(ea, R, E, D, I, 8, 700 + int(planes), x_dtype=2,
                                                          planes=planes)
    assert x.dtype == np.float32
    want = orc.prompt_experts(x, pick, wts, oracle_routed(host), R, 8)
    out = device.zeros((R, D), torch.float32)
    pe.run(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R,
           do_round=False, x_dtype=2)
    assert_close_rms(device.download(out), want, 2e-3, f"prompt experts, fp32 x, planes={planes}")
    assert device.device_status() == 0


@pytest.mark.parametrize("cb,I", [(0, 256), (2, 256), (2, 128), (0, 128)])
def test_prompt_experts_codebooks(ea, cb, I):
    """3inst and mul1 through both item lists (the small items' ring kernel and the larger items' kernel), both
    ring widths (8 waves at I = 256, 4 at I = 128)."""
    device, _, _, pe, synth = ea
    R, E, D = 160, 48, 512
    host, ex, sc, x, pick, wts, dx, dp, dw = _prompt_case(ea, R, E, D, I, 8, 500 + cb + I, cb=cb)
    want = orc.prompt_experts(x, pick, wts, oracle_routed(host), R, 8, bf16=True)
    out = device.zeros((R, D), torch.float32)
    pe.run(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R, do_round=False)
    assert_close_rms(device.download(out), want, 2e-3, f"prompt experts cb={cb}")
    assert device.device_status() == 0


def test_prompt_unaligned_output_same_bits(ea):
    """An output 4 bytes off a 16-byte boundary takes the scalar combine: the same bits as the vector one."""
    device, _, _, pe, synth = ea
    R, D = 40, 512
    host, ex, sc, x, pick, wts, dx, dp, dw = _prompt_case(ea, R, 32, D, 128, 8, 400)
    a = device.zeros((R, D), torch.float32)
    pe.run(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, a.data_ptr(), R, do_round=False)
    b = device.zeros((R * D + 4,), torch.float32)
    pe.run(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, b.data_ptr() + 4, R,
           do_round=False)
    np.testing.assert_array_equal(device.download(b)[1:1 + R * D].reshape(R, D), device.download(a))
    assert device.device_status() == 0


def test_prompt_half_sums_and_invalid(ea):
    """half_sums is the reference's mode 1: no pair plane, each slot added into the fp16 out as packed fp16 atomics
    (prompt_experts.zig:150-155, prompt_experts.cu:785-797). Refused with rounding (prompt_experts.zig:147) and with a
    pair plane (:155). fp16 sums of 8 slots: each slot's value is rounded to fp16 and every add rounds, so the bar is
    1e-2 * RMS here (2e-3 for the fp32 modes)."""
    device, _, _, pe, synth = ea
    from ea_exl3._lib import EaError

    R, D = 20, 256
    host, ex, sc, x, pick, wts, dx, dp, dw = _prompt_case(ea, R, 16, D, 128, 8, 300, planes=False)
    out = device.zeros((R, D), torch.float32)
    with pytest.raises(EaError) as e:  # prompt_experts.zig:147: half sums and rounding together
        pe.run(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R,
               do_round=True, half_sums=True)
    assert e.value.code == 13
    sc_plane = pe.Scratch(ex, R, 8, planes=True)
    with pytest.raises(EaError) as e:  # prompt_experts.zig:155: the pair plane takes fp32 rows only
        pe.run(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc_plane, out.data_ptr(), R,
               do_round=False, half_sums=True)
    assert e.value.code == 13
    pick2 = pick.copy()
    pick2[0, 3] = -1  # a slot that is not an expert adds nothing
    want = orc.prompt_experts(x, pick2, wts, oracle_routed(host), R, 8, bf16=True)
    h = device.zeros((R, D), torch.float16)
    h.fill_(7.0)  # the pass clears its rows of out before the slots are added
    dp2 = device.upload(pick2)
    pe.run(device.stream(), dx.data_ptr(), D, dp2.data_ptr(), dw.data_ptr(), ex, sc, h.data_ptr(), R,
           do_round=False, half_sums=True)
    got = device.download(h).view(np.float16).astype(np.float32)
    assert_close_rms(got, want, 1e-2, "half sums (fp16 atomics)")
    assert device.device_status() == 0


@pytest.mark.parametrize("R,E,D,I,k2", [(130, 64, 512, 256, 8), (300, 256, 1024, 256, "mixed"), (40, 32, 256, 128, 6),
                                        (300, 32, 256, 128, 12), (260, 32, 512, 256, "wide-mixed")])
def test_prompt_experts_no_plane(ea, R, E, D, I, k2):
    """planes = 0, the reference's default mode 0: no pair plane and no combine; the down items add each pair's slot
    into out with fp32 atomics in arrival order (bits may differ run to run). Both item lists, the staged and the
    register-streaming (widths above 10) down GEMMs; out starts dirty and is cleared by the pass; do_round rounds the
    sums through bf16. Every run meets the oracle's bar and the planes-1 output's."""
    device, _, _, pe, synth = ea
    if k2 == "wide-mixed":
        k2v = np.array([(12, 8, 6, 16, 10, 11, 4, 14)[e % 8] for e in range(E)], np.int32)
    else:
        k2v = synth.mixed_widths(5, E) if k2 == "mixed" else k2
    host, ex, sc, x, pick, wts, dx, dp, dw = _prompt_case(ea, R, E, D, I, k2v, 700 + R, planes=False)
    assert sc.c.plane == 0
    want = orc.prompt_experts(x, pick, wts, oracle_routed(host), R, 8, bf16=True)
    sc_plane = pe.Scratch(ex, R, 8, planes=True)
    ref = device.zeros((R, D), torch.float32)
    pe.run(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc_plane, ref.data_ptr(), R,
           do_round=False)
    for rep in range(2):
        out = device.zeros((R, D), torch.float32)
        out.fill_(float("nan") if rep else 3.0)
        pe.run(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R,
               do_round=False)
        got = device.download(out)
        assert_close_rms(got, want, 2e-3, f"prompt experts, no plane, run {rep}")
        assert_close_rms(got, device.download(ref), 2e-3, f"no plane against the plane, run {rep}")
    pe.run(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R, do_round=True)
    r = device.download(out)
    np.testing.assert_array_equal(r, synth.bf16_to_f32(synth.bf16_bits(r)))  # every value a bf16
    # within the fp32 bar plus bf16's half ulp (2^-9 relative) of each value
    w64 = want.astype(np.float64)
    bound = 2e-3 * np.sqrt(np.mean(w64 ** 2)) + np.abs(w64) * 2.0 ** -8
    assert np.all(np.abs(r.astype(np.float64) - w64) <= bound), "no plane, rounded through bf16"
    assert device.device_status() == 0
