"""The allocation-free decode layer (ea_ffn_moe_decode_static, its scratch a file-scope device array the library
resolves per device at ea_init) against ea_ffn_moe_decode with a caller-owned scratch, through the C ABI: picks,
weights and outputs bit for bit on two calls in a row, the second with fewer rows and another layer, plus the
limits it rejects before launching."""
import numpy as np
import pytest

import oracle as orc
from helpers import assert_close_rms, oracle_routed

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ea():
    from ea_exl3 import device, linear, moe, synth

    device.init(0)
    return device, linear, moe, synth


def _layer(ea, seed, R, k2):
    device, linear, moe, synth = ea
    from test_gpu_decode_layer import SharedHost

    E, D, I = 256, 6144, 256
    logits, bias = synth.logits(seed, R)
    pick_w, wts_w = orc.topk8(logits, bias)
    host = synth.HostLayer(seed + 1, experts=E, dims=D, width=I, k2=k2, only=np.unique(pick_w))
    shared = SharedHost(linear, synth, seed + 2, D, I, 8, 1)
    x = synth.activations(seed + 3, R, D, "f16")
    return logits, bias, pick_w, wts_w, host, moe.Routed(host), shared, x


def _call(ea, fn, case, R, sc=None):
    device, linear, moe, synth = ea
    logits, bias, _, _, _, ex, shared, x = case
    D = ex.dims
    dx, dl, db = device.upload(x), device.upload(logits), device.upload(bias)
    dp, dw = device.zeros((R, 8), torch.int32), device.zeros((R, 8), torch.float32)
    out = device.zeros((R, D), torch.float32)
    args = (device.stream(), dx.data_ptr(), D, dl.data_ptr(), db.data_ptr(), 2.5, dp.data_ptr(), dw.data_ptr(), ex,
            [l.c for l in shared.lin])
    if sc is None:
        fn(*args, out.data_ptr(), R, x_dtype=0)
    else:
        fn(*args, sc, out.data_ptr(), R, x_dtype=0)
    return device.download(out), device.download(dp), device.download(dw)


def test_static_matches_scratch_entry_point(ea):
    device, linear, moe, synth = ea
    first = _layer(ea, 3000, 16, synth.mixed_widths(3010, 256))  # 16 rows, the array's full capacity
    second = _layer(ea, 3100, 1, 8)                               # then one row of another layer
    sc = moe.Scratch(first[5], 16, 8)
    for case, R in ((first, 16), (second, 1)):
        got = _call(ea, moe.ffn_decode_static, case, R)
        ref = _call(ea, moe.ffn_decode, case, R, sc)
        for g, r in zip(got, ref):
            np.testing.assert_array_equal(g, r)
        logits, bias, pick_w, wts_w, host, ex, shared, x = case
        np.testing.assert_array_equal(got[1], pick_w)
        want = orc.moe_routed(x, pick_w, wts_w, oracle_routed(host), R, 8) + shared.oracle(x, R, False)
        assert_close_rms(got[0], want, 2e-3, f"static R={R}")
    assert device.device_status() == 0


def test_static_rejects_beyond_its_limit(ea):
    device, linear, moe, synth = ea
    from ea_exl3._lib import EaError

    case = _layer(ea, 3200, 17, 8)
    with pytest.raises(EaError) as e:  # 17 rows: more than the array is carved for
        _call(ea, moe.ffn_decode_static, case, 17)
    assert e.value.code == 12
