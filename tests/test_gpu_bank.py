"""A rank's shard loaded from a checkpoint into the decode path, and experts' widths changed under a captured graph.

  - moe.load (moe.zig:65-151) of rank 2 of 8 from a whole-matrix 4-bit checkpoint: the layer's routed experts
    (gate / up / down shares, 256-byte aligned slabs, ptr / k2 tables, stacked scales) run through ea_moe_routed and
    meet the oracle's layer on the same shares (max|diff| <= 2e-3 RMS);
  - expert_swap.swapLayer (expert_swap.zig:345-467): a decode layer captured in a HIP graph, then picked experts
    changed to 3 bits from a 3-bit bank (new slabs, their scales overwritten, the ptr / k2 tables rewritten in place):
    each replay follows the tables and meets the oracle of the new widths; changing them back to 4 bits from a 4-bit
    bank gives the first replay's bits again."""
import numpy as np
import pytest

import oracle as orc
from helpers import assert_close_rms

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

LAYER, E, D, WORLD, RANK, I_RANK = 3, 16, 512, 8, 2, 128


@pytest.fixture(scope="module")
def ea():
    from ea_exl3 import bank, device, moe, synth

    device.init(0)
    return bank, device, moe, synth


def _whole(synth, seed, k2):
    I = WORLD * I_RANK
    shapes = [(D, I), (D, I), (I, D)]
    T = [[synth.trellis(seed, LAYER, p, e, K, N, k2) for e in range(E)] for p, (K, N) in enumerate(shapes)]
    suh = [[synth.scales(seed + 1 + 100 * p + e, K, 1.0) for e in range(E)] for p, (K, N) in enumerate(shapes)]
    svh = [[synth.scales(seed + 2 + 100 * p + e, N, 0.02) for e in range(E)] for p, (K, N) in enumerate(shapes)]
    return T, suh, svh


def _oracle_layer(bank, readers_by_expert, width=I_RANK, cb=1):
    """The oracle's Routed over this rank's shares, read on the host per expert (Reader.get, pinned on the CPU)."""
    mats = [[], [], []]
    k2 = [np.zeros(E, np.int32) for _ in range(3)]
    sc = {k: [] for k in ("suh_g", "svh_g", "suh_u", "svh_u", "suh_d", "svh_d")}
    for e in range(E):
        r = readers_by_expert[e]
        for p, proj in enumerate(bank.PROJ):
            t = r.get(bank.expert_name(LAYER, e, proj, "trellis"))
            mats[p].append(np.ascontiguousarray(t).view(np.uint32).reshape(-1))
            k2[p][e] = t.shape[2] // 8
            key = "gud"[p]
            sc[f"suh_{key}"].append(r.get(bank.expert_name(LAYER, e, proj, "suh")).view(np.uint16))
            sc[f"svh_{key}"].append(r.get(bank.expert_name(LAYER, e, proj, "svh")).view(np.uint16))
    st = {k: np.stack(v) for k, v in sc.items()}
    return orc.Routed(mats, k2, st["suh_g"], st["suh_u"], st["svh_g"], st["svh_u"], st["suh_d"], st["svh_d"], D,
                      width, cb)


def test_load_rank_shard_and_swap_under_graph(ea, tmp_path):
    bank, device, moe, synth = ea
    ck4, bk4, bk3 = str(tmp_path / "ckpt4"), str(tmp_path / "bank4"), str(tmp_path / "bank3")
    T4, s4u, s4v = _whole(synth, 700, 8)
    T3, s3u, s3v = _whole(synth, 800, 6)
    bank.write_checkpoint_layer(ck4, LAYER, T4, s4u, s4v, cb=1)
    bank.reslice_layer(bank.layer_tensors(LAYER, T4, s4u, s4v, 1), LAYER, bk4, WORLD)
    bank.reslice_layer(bank.layer_tensors(LAYER, T3, s3u, s3v, 1), LAYER, bk3, WORLD)
    rd4 = bank.Reader(ck4, RANK, WORLD, WORLD)
    b4 = bank.Reader(bk4, RANK, WORLD, WORLD, fname=bank.bank_file(LAYER))
    b3 = bank.Reader(bk3, RANK, WORLD, WORLD, fname=bank.bank_file(LAYER))
    lay = bank.Layer(rd4, LAYER, E)
    assert (lay.c.count, lay.c.dims, lay.c.width, lay.c.cb) == (E, D, I_RANK, 1)
    assert tuple(lay.c.k2_gu) == (8, 8) and tuple(lay.c.k2_d) == (8, 8)

    R = 2
    pick = synth.picks_uniform(710, R, E, 8)
    wts = synth.routing_weights(711, R, 8)
    x = synth.activations(712, R, D, "f16")
    sc = moe.Scratch(lay, R, 8)
    dx, dp, dw = device.upload(x), device.upload(pick), device.upload(wts)
    out = device.zeros((R, D), torch.float32)

    def call(stream):
        moe.routed(stream, dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), lay, sc, out.data_ptr(), R, x_dtype=0)

    want4 = orc.moe_routed(x, pick, wts, _oracle_layer(bank, [rd4] * E), R, 8)
    # eager on a side stream, then the capture
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call(device.stream(side))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    eager = device.download(out)
    assert_close_rms(eager, want4, 2e-3, "rank shard from the checkpoint")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(device.stream())
    torch.cuda.synchronize()

    def replay():
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        return device.download(out)

    first = replay()
    np.testing.assert_array_equal(first, eager)

    # picked experts (and one that is not picked) to 3 bits under the captured graph
    changed = sorted(set(int(e) for e in pick.reshape(-1)))[:5] + [int(e) for e in range(E) if e not in pick][:1]
    cur = np.full(E, 4, np.uint8)
    tgt = cur.copy()
    tgt[changed] = 3
    st = lay.swap({3: b3}, tgt, cur)
    assert (st.experts, st.up, st.down) == (len(changed), 0, len(changed))
    assert tuple(lay.c.k2_gu) == (6, 8) and tuple(lay.c.k2_d) == (6, 8)
    want3 = orc.moe_routed(x, pick, wts, _oracle_layer(bank, [b3 if e in changed else rd4 for e in range(E)]), R, 8)
    for rep in range(2):
        got = replay()
        assert_close_rms(got, want3, 2e-3, f"replay {rep} after the change to 3 bits")
    assert np.max(np.abs(got.astype(np.float64) - want4)) > 1e-2 * np.sqrt(np.mean(want4.astype(np.float64) ** 2))

    # and back to 4 bits from the 4-bit bank: the first replay's bits
    st = lay.swap({4: b4}, cur, tgt)
    assert (st.experts, st.up, st.down) == (len(changed), len(changed), 0)
    np.testing.assert_array_equal(replay(), first)
    assert device.device_status() == 0

    # a width with no bank is refused before anything changes
    from ea_exl3._lib import EaError

    with pytest.raises(EaError) as e:
        lay.swap({3: b3}, np.full(E, 2, np.uint8), cur)
    assert e.value.code == 37  # SwapNoBank
    np.testing.assert_array_equal(replay(), first)
    # so is a width the kernels do not decode (6 bits), even with a bank for it
    with pytest.raises(EaError) as e:
        lay.swap({6: b3}, np.full(E, 6, np.uint8), cur)
    assert e.value.code == 36  # SwapWidthUnsupported
    np.testing.assert_array_equal(replay(), first)
    del g
    lay.free()


def test_load_mixed_widths_from_two_banks(ea, tmp_path):
    """moe.loadFrom with a per-expert pick of banks (an expert plan): experts 0..E-1 alternate between a 3-bit and a
    4-bit bank read by 4 ranks (two stored ranks joined a share); the loaded layer meets the oracle."""
    bank, device, moe, synth = ea
    world, rank = 4, 1
    bk4, bk3 = str(tmp_path / "b4"), str(tmp_path / "b3")
    T4, s4u, s4v = _whole(synth, 900, 8)
    T3, s3u, s3v = _whole(synth, 950, 6)
    bank.reslice_layer(bank.layer_tensors(LAYER, T4, s4u, s4v, 1), LAYER, bk4, WORLD)
    bank.reslice_layer(bank.layer_tensors(LAYER, T3, s3u, s3v, 1), LAYER, bk3, WORLD)
    b4 = bank.Reader(bk4, rank, world, WORLD, fname=bank.bank_file(LAYER))
    b3 = bank.Reader(bk3, rank, world, WORLD, fname=bank.bank_file(LAYER))
    pick_bank = np.array([e % 2 for e in range(E)], np.uint8)
    lay = bank.Layer([b4, b3], LAYER, E, pick=pick_bank)
    assert lay.c.width == 2 * I_RANK and tuple(lay.c.k2_gu) == (6, 8)
    R = 3
    pick = synth.picks_uniform(960, R, E, 8)
    wts = synth.routing_weights(961, R, 8)
    x = synth.activations(962, R, D, "bf16")
    sc = moe.Scratch(lay, R, 8)
    out = device.zeros((R, D), torch.float32)
    dx, dp, dw = device.upload(x), device.upload(pick), device.upload(wts)
    moe.routed(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), lay, sc, out.data_ptr(), R, x_dtype=1)
    want = orc.moe_routed(x, pick, wts, _oracle_layer(bank, [b3 if e % 2 else b4 for e in range(E)], 2 * I_RANK), R,
                          8, bf16=True)
    assert_close_rms(device.download(out), want, 2e-3, "two banks, four ranks")
    assert device.device_status() == 0
    lay.free()
