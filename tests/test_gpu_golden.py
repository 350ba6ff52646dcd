"""The HIP path against the committed golden fixtures (tests/golden/golden.npz): every tile decodes bit for bit, the
top-8 matches bit for bit, and the reduced-width layers through ea_moe_routed (both its paths: a scratch of 16 rows
takes the decode layer's launches, one of 32 rows the six-launch sequence) stay within 2e-3 * RMS."""
import os
import sys

import numpy as np
import pytest

from helpers import assert_close_rms

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as mg  # noqa: E402

G = np.load(os.path.join(HERE, "golden", "golden.npz"), allow_pickle=False)


@pytest.fixture(scope="module")
def ea():
    from ea_exl3 import device, moe, ops

    device.init(0)
    return device, moe, ops


def test_tiles_decode(ea):
    device, _, _ = ea
    from ea_exl3._lib import check, lib

    for k2 in mg.TILE_WIDTHS:
        for cb in range(3):
            dT = device.upload(G[f"tile_{k2}_{cb}_words"])  # bound: a freed upload's memory is handed out again
            dW = device.zeros((16, 16), torch.int16)
            check(lib().ea_dequant(device.stream(), dT.data_ptr(), dW.data_ptr(), 16, 16, k2, cb), "dq")
            np.testing.assert_array_equal(device.download(dW).view(np.uint16), G[f"tile_{k2}_{cb}_w"],
                                          err_msg=f"k2={k2} cb={cb}")


def test_topk(ea):
    device, _, ops = ea
    logits, bias = G["topk_logits"], G["topk_bias"]
    rows = logits.shape[0]
    dl, db = device.upload(logits), device.upload(bias)  # bound for the kernel's lifetime
    dp, dw = device.zeros((rows, 8), torch.int32), device.zeros((rows, 8), torch.float32)
    ops.topk(device.stream(), dl.data_ptr(), db.data_ptr(), dp.data_ptr(), dw.data_ptr(), rows, 2.5)
    np.testing.assert_array_equal(device.download(dp), G["topk_pick"])
    np.testing.assert_array_equal(device.download(dw), G["topk_wts"])


@pytest.mark.parametrize("R", [1, 16])
@pytest.mark.parametrize("cap", [16, 32])
def test_layer(ea, R, cap):
    device, moe, _ = ea
    host, x, pick, wts, _, digest = mg.layer_case(R)
    assert digest == str(G[f"layer_r{R}_inputs_sha256"])
    ex = moe.Routed(host)
    sc = moe.Scratch(ex, cap, 8)
    out = device.zeros((R, host.dims), torch.float32)
    dx, dp, dw = device.upload(x), device.upload(pick), device.upload(wts)  # bound for the kernels' lifetime
    moe.routed(device.stream(), dx.data_ptr(), host.dims, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R,
               x_dtype=0)
    assert device.device_status() == 0
    assert_close_rms(device.download(out), G[f"layer_r{R}_out"], 2e-3, f"golden layer R={R} cap={cap}")
