"""HIP graph capture of the library's calls through torch.cuda.CUDAGraph: a prefill pass (its two item lists fork
onto the library's second stream and join back with events, so the capture follows the fork), the decode layer (one
launch at one row, five at four), moe.routed on a 40-row window (the prefill path in the scratch's prompt region) and
the EXL3 linear at one row (the tagged split-K slots, zeroed by each call's finisher) and at 40 rows (the per-pass
counters, reset by each call's last block). Each is captured once after an eager warm-up and replayed several times,
with eager work and synchronizations between the replays; every replay must give the eager result bit for bit (both
paths are deterministic: splits and slots are summed in a fixed order)."""
import numpy as np
import pytest

import oracle as orc

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ea():
    from ea_exl3 import device, linear, moe, prompt_experts, synth

    device.init(0)
    return device, linear, moe, prompt_experts, synth


def _capture_and_replay(device, call, out, replays=3):
    """call(stream) issues the library call on `stream`; out is the tensor it writes."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # eager warm-up off the default stream, as torch advises before a capture
        call(device.stream(side))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(device.stream())
    torch.cuda.synchronize()
    for i in range(replays):
        out.fill_(float("nan"))  # eager work between the replays
        junk = torch.randn(1 << 16, device="cuda").sum()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        np.testing.assert_array_equal(out.cpu().numpy(), eager.cpu().numpy(), err_msg=f"replay {i}")
    assert device.device_status() == 0


def test_prefill_graph_replays(ea):
    device, _, moe, pe, synth = ea
    R, E, D, I, slots = 130, 64, 512, 256, 8
    pick = synth.picks_zipf(900, R, 1.1, E, slots)
    wts = synth.routing_weights(901, R, slots)
    host = synth.HostLayer(902, experts=E, dims=D, width=I, k2=8, only=np.unique(pick))
    x = synth.activations(903, R, D, "bf16")
    ex = moe.Routed(host)
    sc = pe.Scratch(ex, R, slots)
    dx, dp, dw = device.upload(x), device.upload(pick), device.upload(wts)
    out = device.zeros((R, D), torch.float32)
    _capture_and_replay(device, lambda s: pe.run(s, dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc,
                                                 out.data_ptr(), R, do_round=False), out)


@pytest.mark.parametrize("R", [1, 4])
def test_decode_layer_graph_replays(ea, R):
    device, linear, moe, pe, synth = ea
    E, D, I = 256, 2048, 256
    logits, bias = synth.logits(910 + R, R)
    pick, _ = orc.topk8(logits, bias)
    host = synth.HostLayer(911, experts=E, dims=D, width=I, k2=8, only=np.unique(pick))
    shapes = [(D, I), (D, I), (I, D)]
    lin = [linear.Linear(synth.trellis(912, 0, m, 0, K, N, 8), synth.scales(913 + m, K, 1.0),
                         synth.scales(916 + m, N, 0.02), K, N, 8, 1) for m, (K, N) in enumerate(shapes)]
    ex = moe.Routed(host)
    sc = moe.Scratch(ex, 16, 8)
    x = synth.activations(920, R, D, "f16")
    dx, dl, db = device.upload(x), device.upload(logits), device.upload(bias)
    dp, dw = device.zeros((R, 8), torch.int32), device.zeros((R, 8), torch.float32)
    out = device.zeros((R, D), torch.float32)
    _capture_and_replay(device, lambda s: moe.ffn_decode(s, dx.data_ptr(), D, dl.data_ptr(), db.data_ptr(), 2.5,
                                                         dp.data_ptr(), dw.data_ptr(), ex, [l.c for l in lin], sc,
                                                         out.data_ptr(), R, x_dtype=0), out)


def test_window_graph_replays(ea):
    device, linear, moe, pe, synth = ea
    R, E, D, I, slots = 40, 64, 1024, 256, 8
    pick = synth.picks_uniform(930, R, E, slots)
    wts = synth.routing_weights(931, R, slots)
    host = synth.HostLayer(932, experts=E, dims=D, width=I, k2=8, only=np.unique(pick))
    ex = moe.Routed(host)
    sc = moe.Scratch(ex, 64, slots)
    assert sc.c.fused != 0  # the prompt region
    x = synth.activations(933, R, D, "f16")
    dx, dp, dw = device.upload(x), device.upload(pick), device.upload(wts)
    out = device.zeros((R, D), torch.float32)
    _capture_and_replay(device, lambda s: moe.routed(s, dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc,
                                                     out.data_ptr(), R, x_dtype=0), out)


@pytest.mark.parametrize("M", [1, 40])
def test_linear_graph_replays(ea, M):
    device, linear, moe, pe, synth = ea
    K, N = 6144, 256
    lin = linear.Linear(synth.trellis(940, 0, 0, 0, K, N, 8), synth.scales(941, K, 1.0), synth.scales(942, N, 0.02),
                        K, N, 8, 1)
    sc = linear.Scratch(M, K, lin.sk * M * N)
    x = synth.activations(943 + M, M, K, "f16")
    dx = device.upload(x)
    y = device.zeros((M, N), torch.float32)
    _capture_and_replay(device, lambda s: linear.call(s, sc, [lin], dx.data_ptr(), 0, M, [y.data_ptr()], [2]), y)
    assert int(device.download(lin.counters).sum()) == 0
