"""GPU parity of the decode path through the C ABI against the CPU oracle: trellis dequantisation (bit-exact),
grouping (exact), rot_in and the epilogues (bit-exact on the same inputs), the grouped GEMV (fp32 accumulation:
tolerance) and the whole moe.routed layer (max|diff| <= 2e-3 * RMS(out), the north star's bar)."""
import numpy as np
import pytest

import oracle as orc
from helpers import assert_close_rms, oracle_routed

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ea():
    from ea_exl3 import device, experts, moe, ops, synth

    device.init(0)
    return device, experts, moe, ops, synth


def _stream(ea):
    return ea[0].stream()


# ---- dequantisation ----------------------------------------------------------------------------------------------

@pytest.mark.parametrize("k2", list(range(2, 17)))
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_dequant_bit_exact(ea, k2, cb):
    device, _, _, _, synth = ea
    from ea_exl3._lib import check, lib

    K, N = 64, 256
    T = synth.trellis(11, 0, cb, k2, K, N, k2)
    want = orc.dequant_expert(T, K, N, k2, cb)
    dT = device.upload(T)
    dW = device.zeros((K, N), torch.int16)
    check(lib().ea_dequant(device.stream(), dT.data_ptr(), dW.data_ptr(), K, N, k2, cb), "dequant")
    np.testing.assert_array_equal(device.download(dW), want)


def test_dequant_full_expert_matrix(ea):
    """One gate matrix of a rank's shard at its real shape (6144 x 256, 4 bits) and one down matrix (3 bits)."""
    device, _, _, _, synth = ea
    from ea_exl3._lib import check, lib

    for K, N, k2 in ((6144, 256, 8), (256, 6144, 6)):
        T = synth.trellis(12, 0, 0, 0, K, N, k2)
        want = orc.dequant_expert(T, K, N, k2, 1)
        dT = device.upload(T)
        dW = device.zeros((K, N), torch.int16)
        check(lib().ea_dequant(device.stream(), dT.data_ptr(), dW.data_ptr(), K, N, k2, 1), "dequant")
        np.testing.assert_array_equal(device.download(dW), want)


# ---- grouping ------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("R,E", [(1, 256), (4, 256), (16, 256), (16, 64), (128, 256)])
def test_group_exact(ea, R, E):
    device, experts, _, _, synth = ea
    slots = 8
    pick = synth.picks_uniform(R * 31 + E, R, E, slots)
    if R >= 4:
        pick[1, 3] = -1  # a slot that is not an expert
        pick[2, 0] = E   # an id past the experts: skipped like -1
    maxm = R
    maxu = min(R * slots, E)
    uids_w, uc_w, mem_w = orc.group(pick, R, slots, E, maxm)
    k = experts.Kernels.load()
    dp = device.upload(pick)
    du = device.zeros(maxu, torch.int32)
    dc = device.zeros(1, torch.int32)
    dm = device.upload(np.full((maxu, maxm), -1, np.int32))
    k.group(device.stream(), dp.data_ptr(), du.data_ptr(), dc.data_ptr(), dm.data_ptr(), R, slots, E, maxm)
    assert int(device.download(dc)[0]) == uc_w
    np.testing.assert_array_equal(device.download(du)[:uc_w], uids_w[:uc_w])
    np.testing.assert_array_equal(device.download(dm)[:uc_w], mem_w[:uc_w])


# ---- rot_in and the epilogues -------------------------------------------------------------------------------------

def _layer(synth, seed, E, D, I, picked, k2=8):
    return synth.HostLayer(seed, experts=E, dims=D, width=I, k2=k2, only=np.unique(picked[picked >= 0]))


@pytest.mark.parametrize("x_dtype", [0, 1, 2])
def test_rot_in_bit_exact(ea, x_dtype):
    device, experts, _, _, synth = ea
    R, E, D, slots = 3, 32, 1024, 8
    pick = synth.picks_uniform(5, R, E, slots)
    pick[0, 2] = -1
    host = _layer(synth, 5, E, D, 256, pick)
    x = synth.activations(6, R, D, ["f16", "bf16", "f32"][x_dtype])
    o0, o1 = orc.rot_in(x, pick, host.suh_g, host.suh_u, R, D, slots, E, bf16=(x_dtype == 1))
    k = experts.Kernels.load()
    dx, dp = device.upload(x), device.upload(pick)
    sg, su = device.upload(host.suh_g), device.upload(host.suh_u)
    d0 = device.zeros((R * slots, D), torch.int16)
    d1 = device.zeros((R * slots, D), torch.int16)
    k.rot_in(device.stream(), dx.data_ptr(), D, dp.data_ptr(), sg.data_ptr(), su.data_ptr(), d0.data_ptr(),
             d1.data_ptr(), R, D, slots, E, x_dtype=x_dtype)
    np.testing.assert_array_equal(device.download(d0), o0)
    np.testing.assert_array_equal(device.download(d1), o1)


def test_gateup_epilogue_bit_exact(ea):
    device, experts, moe, _, synth = ea
    R, E, I, SK, slots = 4, 32, 256, 4, 8
    P = R * slots
    pick = synth.picks_uniform(8, R, E, slots)
    pick[1, 1] = -1
    host = _layer(synth, 8, E, 512, I, pick)
    Z = (np.random.default_rng(3).standard_normal((2, SK, P, I)) * 3).astype(np.float32)
    r = oracle_routed(host)
    for act_mode, limit in ((1, float("inf")), (0, 7.0), (1, 2.5)):
        want = orc.gateup_epilogue(Z, pick, r, R, P, I, SK, slots, E, limit, act_mode)
        k = experts.Kernels.load()
        dz, dp = device.upload(Z), device.upload(pick)
        sg, su, sd = device.upload(host.svh_g), device.upload(host.svh_u), device.upload(host.suh_d)
        xd = device.zeros((P, I), torch.int16)
        k.gateup_epilogue(device.stream(), dz.data_ptr(), dp.data_ptr(), sg.data_ptr(), su.data_ptr(), sd.data_ptr(),
                          xd.data_ptr(), R, P, I, SK, slots, E, limit, act_mode)
        got = device.download(xd)
        valid = (pick.reshape(-1) >= 0)
        np.testing.assert_array_equal(got[valid], want[valid])


def test_down_combine_bit_exact(ea):
    device, experts, _, _, synth = ea
    R, E, D, slots = 3, 32, 768, 8
    P = R * slots
    pick = synth.picks_uniform(9, R, E, slots)
    pick[2, 5] = -1  # reads y as the caller left it
    host = _layer(synth, 9, E, D, 256, pick)
    rng = np.random.default_rng(4)
    for SK in (1, 3):
        Z = rng.standard_normal((SK, P, D)).astype(np.float32)
        wts = synth.routing_weights(10, R, slots)
        y0 = rng.standard_normal((P, D)).astype(np.float32)
        r = oracle_routed(host)
        y_w, out_w = orc.down_combine(Z, pick, r, wts, R, P, D, SK, slots, E, y=y0.copy())
        k = experts.Kernels.load()
        dz, dp, dw = device.upload(Z), device.upload(pick), device.upload(wts)
        sv = device.upload(host.svh_d)
        dy = device.upload(y0)
        do = device.zeros((R, D), torch.float32)
        k.down_combine(device.stream(), dz.data_ptr(), dp.data_ptr(), sv.data_ptr(), dy.data_ptr(), dw.data_ptr(),
                       do.data_ptr(), R, P, D, SK, slots, E)
        np.testing.assert_array_equal(device.download(dy), y_w)
        np.testing.assert_array_equal(device.download(do), out_w)


# ---- the grouped GEMV ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("R,k2s", [(1, 8), (16, 8), (5, "mixed"), (16, "mixed")])
def test_grouped_gateup_and_down(ea, R, k2s):
    device, experts, moe, _, synth = ea
    E, D, I, slots = 64, 1024, 256, 8
    P = R * slots
    pick = synth.picks_uniform(20 + R, R, E, slots)
    k2 = synth.mixed_widths(21, E) if k2s == "mixed" else 8
    host = _layer(synth, 22, E, D, I, pick, k2=k2)
    r = oracle_routed(host)
    maxu = min(P, E)
    uids, uc, members = orc.group(pick, R, slots, E, R)
    x = synth.activations(23, P, D, "f16")
    xd = synth.activations(24, P, I, "f16")
    ex = moe.Routed(host)
    k = experts.Kernels.load()
    du, dc, dm = device.upload(uids), device.upload(np.array([uc], np.int32)), device.upload(members)
    for mats, (K, N, SK, xx) in (((0, 1), (D, I, 4, x)), ((2,), (I, D, 1, xd))):
        want = orc.grouped(xx, xx, r, mats, uids, uc, members, K, N, P, SK, slots)
        dx = device.upload(xx)
        z = device.zeros((len(mats), SK, P, N), torch.float32)
        k2min = int(min(host.k2[m].min() for m in mats))
        k2max = int(max(host.k2[m].max() for m in mats))
        a = experts.grouped_args(x0=dx.data_ptr(), x1=dx.data_ptr(), tp0=ex.ptr[mats[0]].data_ptr(),
                                 tp1=ex.ptr[mats[-1]].data_ptr(), k2_0=ex.k2[mats[0]].data_ptr(),
                                 k2_1=ex.k2[mats[-1]].data_ptr(), uids=du.data_ptr(), ucount=dc.data_ptr(),
                                 members=dm.data_ptr(), z=z.data_ptr(), K=K, N=N, P=P, SK=SK, maxm=R, slots=slots,
                                 nexp_max=maxu, mats=len(mats), cb=1, nt=8, warps=4, pf=1, lo=k2min, hi=k2max)
        k.grouped(device.stream(), a)
        got = device.download(z)
        rows = sorted({(c >> 5) * slots + (c & 31) for c in members[:uc].reshape(-1) if c >= 0})
        assert_close_rms(got[:, :, rows], want[:, :, rows], 1e-4, f"grouped mats={mats}")
        assert device.device_status() == 0


# ---- the whole layer ----------------------------------------------------------------------------------------------

def _routed_case(ea, R, E, D, I, k2, x_dtype, seed):
    device, experts, moe, _, synth = ea
    slots = 8
    pick = synth.picks_uniform(seed, R, E, slots)
    wts = synth.routing_weights(seed + 1, R, slots)
    host = _layer(synth, seed + 2, E, D, I, pick, k2=k2)
    x = synth.activations(seed + 3, R, D, ["f16", "bf16", "f32"][x_dtype])
    want = orc.moe_routed(x, pick, wts, oracle_routed(host), R, slots, bf16=(x_dtype == 1))
    ex = moe.Routed(host)
    sc = moe.Scratch(ex, R, slots)
    dx, dp, dw = device.upload(x), device.upload(pick), device.upload(wts)
    out = device.zeros((R, D), torch.float32)
    moe.routed(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R,
               x_dtype=x_dtype)
    got = device.download(out)
    assert device.device_status() == 0
    return got, want


# fp32 activations (x_dtype 2) take the six-launch sequence (the decode layer reads 16-bit rows only)
@pytest.mark.parametrize("R,x_dtype", [(1, 0), (4, 1), (16, 0), (4, 2), (16, 2)])
def test_moe_routed_reduced_width(ea, R, x_dtype):
    got, want = _routed_case(ea, R, 64, 1024, 256, 8, x_dtype, 30 + R)
    assert_close_rms(got, want, 2e-3, "moe.routed")


@pytest.mark.parametrize("R", [1, 12])
def test_moe_routed_3inst(ea, R):
    """3inst routed experts through moe.routed on a scratch of at most 16 rows (the decode layer's launches)."""
    device, experts, moe, _, synth = ea
    slots, E, D, I = 8, 64, 1024, 256
    pick = synth.picks_uniform(70 + R, R, E, slots)
    wts = synth.routing_weights(71 + R, R, slots)
    host = synth.HostLayer(72 + R, experts=E, dims=D, width=I, k2=8, cb=0, only=np.unique(pick))
    x = synth.activations(73 + R, R, D, "f16")
    want = orc.moe_routed(x, pick, wts, oracle_routed(host), R, slots)
    ex = moe.Routed(host)
    sc = moe.Scratch(ex, R, slots)
    dx, dp, dw = device.upload(x), device.upload(pick), device.upload(wts)
    out = device.zeros((R, D), torch.float32)
    moe.routed(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R, x_dtype=0)
    assert_close_rms(device.download(out), want, 2e-3, f"moe.routed 3inst R={R}")
    assert device.device_status() == 0


def test_moe_routed_full_shape_r1(ea):
    """BASELINE config 2's routed part at its real shape: D 6144, I 256, 256 experts, 4 bits, batch 1."""
    got, want = _routed_case(ea, 1, 256, 6144, 256, 8, 0, 40)
    assert_close_rms(got, want, 2e-3, "moe.routed R=1")


def test_moe_routed_full_shape_r16_mixed(ea):
    """BASELINE config 3's routed part: 16 rows, uniform top-8, 70% of experts at 3 bits."""
    device, experts, moe, _, synth = ea
    got, want = _routed_case(ea, 16, 256, 6144, 256, synth.mixed_widths(41, 256), 0, 42)
    assert_close_rms(got, want, 2e-3, "moe.routed R=16 mixed")


# ---- routing input and the shared expert's activation ---------------------------------------------------------------

def test_topk8_exact(ea):
    device, _, _, ops, synth = ea
    rows = 64
    logits, bias = synth.logits(50, rows)
    logits[3, :] = 0.25  # every expert tied: picks are ids 0..7 ordered by bias then id
    bias2 = bias.copy()
    logits[4, 10] = logits[4, 20] = 5.0  # an exact tie between two strong experts
    pick_w, wts_w = orc.topk8(logits, bias2)
    dl, db = device.upload(logits), device.upload(bias2)
    dp, dw = device.zeros((rows, 8), torch.int32), device.zeros((rows, 8), torch.float32)
    ops.topk(device.stream(), dl.data_ptr(), db.data_ptr(), dp.data_ptr(), dw.data_ptr(), rows, 2.5)
    np.testing.assert_array_equal(device.download(dp), pick_w)
    np.testing.assert_array_equal(device.download(dw), wts_w)


def test_swiglu2_exact(ea):
    device, _, _, ops, synth = ea
    rows, width = 7, 512
    g = synth.bf16_bits(np.random.default_rng(1).standard_normal((rows, width)) * 4)
    u = synth.bf16_bits(np.random.default_rng(2).standard_normal((rows, width)))
    want = orc.swiglu2(g, u)
    dg, du = device.upload(g), device.upload(u)
    do = device.zeros((rows, width), torch.int16)
    ops.swiglu2(device.stream(), dg.data_ptr(), du.data_ptr(), do.data_ptr(), rows, width)
    np.testing.assert_array_equal(device.download(do), want)
