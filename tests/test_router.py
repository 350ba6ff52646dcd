"""The router's logits (ops.zig:131-136: router_part native_ops.cu:1405-1460 + router_sum :335-362).

CPU: the oracle's or_router is pinned by the dense fp64 product (within the fp32 summation bound of its order), by
inputs whose every partial sum is an exact small integer (the result must equal the integer product exactly), by
one-hot activations (each logit must be the one weight it selects: a transposed or shifted operand fails) and by
the slice sums adding up, in slice order, to the logits bit for bit.

GPU: ea_router through the C ABI must give the oracle's bits (the same in-slice order: lane chunks by fma, then a
butterfly, then the slices in order) at the MoE router's shape (6144 x 256, one and sixteen rows, fp16 and bf16 x),
ragged rows and experts, the narrowest reduction the op takes (512), and the slice sums."""
import numpy as np
import pytest

import oracle as orc
from ea_exl3 import synth


def _bf16(a):
    return synth.bf16_bits(np.asarray(a, np.float32))


def _data(seed, m, d, ne):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, d)).astype(np.float32)
    w = (0.02 * rng.standard_normal((ne, d))).astype(np.float32)
    return x, w


def _f(bits, bf):
    b = np.asarray(bits, np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32) if bf else b.view(np.float16).astype(np.float32)


# ---- the oracle -------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("x_dtype", [0, 1])
def test_oracle_router_matches_fp64_product(x_dtype):
    m, d, ne = 3, 6144, 64
    x, w = _data(1, m, d, ne)
    xb = synth.f16_bits(x) if x_dtype == 0 else _bf16(x)
    wb = _bf16(w)
    got = orc.router(xb, wb, x_dtype)
    xf, wf = _f(xb, x_dtype == 1).astype(np.float64), _f(wb, True).astype(np.float64)
    want = xf @ wf.T
    # fp32 sums along the oracle's order: 12 + 6 sequential additions inside a slice, 7 across: bound 25 u sum|x w|
    bound = 26 * 2.0**-24 * (np.abs(xf) @ np.abs(wf).T)
    assert np.all(np.abs(got - want) <= bound)


def test_oracle_router_exact_on_integers():
    rng = np.random.default_rng(2)
    m, d, ne = 2, 2048, 40
    x = rng.integers(-3, 4, (m, d)).astype(np.float32)
    w = rng.integers(-3, 4, (ne, d)).astype(np.float32)
    got = orc.router(_bf16(x), _bf16(w), 1)
    np.testing.assert_array_equal(got, (x.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32))


def test_oracle_router_one_hot_selects_the_weight():
    rng = np.random.default_rng(3)
    d, ne = 1024, 16
    w = _bf16(0.02 * rng.standard_normal((ne, d)))
    ks = [0, 1, 3, 127, 128, 511, 512, 700, 1023]
    x = np.zeros((len(ks), d), np.float32)
    for i, k in enumerate(ks):
        x[i, k] = 1.0
    got = orc.router(_bf16(x), w, 1)
    np.testing.assert_array_equal(got, _f(w, True)[:, ks].T)


def test_oracle_router_slices_add_in_order():
    x, w = _data(4, 5, 4096, 32)
    out, part = orc.router(_bf16(x), _bf16(w), 1, with_part=True)
    acc = part[0].copy()
    for s in range(1, 8):
        acc = (acc + part[s]).astype(np.float32)
    np.testing.assert_array_equal(acc, out)
    # a slice sum covers only its slice: zeroing the activations of slice 3 zeroes part[3] alone
    xz = x.copy()
    xz[:, 3 * 512:4 * 512] = 0
    _, pz = orc.router(_bf16(xz), _bf16(w), 1, with_part=True)
    assert np.all(pz[3] == 0)
    np.testing.assert_array_equal(np.delete(pz, 3, axis=0), np.delete(part, 3, axis=0))


# ---- the GPU against the oracle -------------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def ea():
    torch = pytest.importorskip("torch")
    from ea_exl3 import device, ops

    device.init(0)
    return torch, device, ops


@pytest.mark.gpu
@pytest.mark.parametrize("m,d,ne,x_dtype", [(1, 6144, 256, 0), (1, 6144, 256, 1), (16, 6144, 256, 0),
                                            (37, 2048, 250, 1), (5, 512, 256, 0), (300, 1536, 64, 1)])
def test_gpu_router_bit_exact(ea, m, d, ne, x_dtype):
    torch, device, ops = ea
    x, w = _data(100 + m, m, d, ne)
    xb = synth.f16_bits(x) if x_dtype == 0 else _bf16(x)
    wb = _bf16(w)
    want, wpart = orc.router(xb, wb, x_dtype, with_part=True)
    dx, dw = device.upload(xb), device.upload(wb)
    out = device.zeros((m, ne), torch.float32)
    part = device.zeros((8, m, ne), torch.float32)
    print(f"router m={m} d={d} ne={ne} x_dtype={x_dtype}", flush=True)
    ops.router(device.stream(), dx.data_ptr(), d, dw.data_ptr(), part.data_ptr(), out.data_ptr(), m, d, ne, x_dtype)
    np.testing.assert_array_equal(device.download(out).view(np.uint32), want.view(np.uint32))
    np.testing.assert_array_equal(device.download(part).view(np.uint32), wpart.view(np.uint32))
    # without the slice sums, and with a row stride wider than d
    xs = np.zeros((m, d + 64), np.uint16)
    xs[:, :d] = xb
    dxs = device.upload(xs)
    out2 = device.zeros((m, ne), torch.float32)
    ops.router(device.stream(), dxs.data_ptr(), d + 64, dw.data_ptr(), 0, out2.data_ptr(), m, d, ne, x_dtype)
    np.testing.assert_array_equal(device.download(out2).view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
def test_gpu_router_errors(ea):
    torch, device, ops = ea
    from ea_exl3._lib import EaError

    x = device.zeros((2, 1024), torch.int16)
    w = device.zeros((8, 1024), torch.int16)
    out = device.zeros((2, 8), torch.float32)
    s = device.stream()
    for args, code in [((1000, 1000), 8), ((1024, 768), 8), ((1000, 1024), 9)]:
        stride, d = args
        with pytest.raises(EaError) as e:
            ops.router(s, x.data_ptr(), stride, w.data_ptr(), 0, out.data_ptr(), 2, d, 8)
        assert e.value.code == code
    with pytest.raises(EaError) as e:
        ops.router(s, x.data_ptr() + 2, 1024, w.data_ptr(), 0, out.data_ptr(), 2, 1024, 8)
    assert e.value.code == 18
