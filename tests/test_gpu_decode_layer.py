"""GPU parity of the one-launch decode layer through the C ABI. ea_ffn_moe_decode (top-8 from the router logits, the
routed experts, the shared expert's mlp and their sum) is checked against the oracle's composition of the same
reference steps (forward.zig:2361-2403): ops.topk -> moe.routed -> gate / up EXL3 linears with bf16 outputs ->
swiglu2 -> down linear (fp32) -> addF32. pick / wts must match bit for bit; out within 2e-3 * RMS(out), the north
star's bar. Calls repeat on one scratch with changing row counts, layer shapes and epochs, which exercises the
one-launch layer's tagged hand-off slots (a new tag every launch, never a cleared slot)."""
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


class SharedHost:
    """The shared expert of one rank as three EXL3 linears (gate, up: D -> I; down: I -> D) on the host and device."""

    def __init__(self, linear, synth, seed, D, I, k2, cb):
        self.D, self.I, self.k2, self.cb = D, I, k2, cb
        shapes = [(D, I), (D, I), (I, D)]
        self.T = [synth.trellis(seed, 0, m, 0, K, N, k2) for m, (K, N) in enumerate(shapes)]
        self.suh = [synth.scales(seed + 1 + m, K, 1.0) for m, (K, N) in enumerate(shapes)]
        self.svh = [synth.scales(seed + 4 + m, N, 0.02) for m, (K, N) in enumerate(shapes)]
        self.lin = [linear.Linear(self.T[m], self.suh[m], self.svh[m], K, N, k2, cb) for m, (K, N) in enumerate(shapes)]
        self.strips = [linear.strips(self.T[m], K, N, k2) for m, (K, N) in enumerate(shapes)]

    def oracle(self, x, R, bf16):
        """forward.mlp (forward.zig:2328-2341): bf16 gate / up, swiglu2, fp32 down."""
        tw = 4 * self.k2
        outs = []
        for m in range(2):
            xh = orc.exl3_rot_in(x, self.suh[m], R, self.D, bf16=bf16)
            outs.append(orc.exl3_linear(xh, self.strips[m], 8 * tw, (self.D // 16) * 8 * tw, self.svh[m], R, self.D,
                                        self.I, self.k2, self.cb, self.lin[m].sk, self.lin[m].wk, y_dtype=1))
        act = orc.swiglu2(outs[0], outs[1])
        xh = orc.exl3_rot_in(act, self.suh[2], R, self.I, bf16=True)
        return orc.exl3_linear(xh, self.strips[2], 8 * tw, (self.I // 16) * 8 * tw, self.svh[2], R, self.I, self.D,
                               self.k2, self.cb, self.lin[2].sk, self.lin[2].wk, y_dtype=2)


def _run(ea, host, shared, sc, ex, x, logits, bias, R, x_dtype):
    device, _, moe, _ = ea
    D = host.dims
    dx, dl, db = device.upload(x), device.upload(logits), device.upload(bias)
    dp, dw = device.zeros((R, 8), torch.int32), device.zeros((R, 8), torch.float32)
    out = device.zeros((R, D), torch.float32)
    moe.ffn_decode(device.stream(), dx.data_ptr(), D, dl.data_ptr(), db.data_ptr(), 2.5, dp.data_ptr(), dw.data_ptr(),
                   ex, None if shared is None else [l.c for l in shared.lin], sc, out.data_ptr(), R, x_dtype=x_dtype)
    got = device.download(out), device.download(dp), device.download(dw)
    assert device.device_status() == 0
    return got


def _want(host, shared, x, logits, bias, R, bf16):
    pick, wts = orc.topk8(logits, bias)
    want = orc.moe_routed(x, pick, wts, oracle_routed(host), R, 8, bf16=bf16)
    if shared is not None:
        want = want + shared.oracle(x, R, bf16)
    return want, pick, wts


def _layer_for(synth, seed, logits_list, bias, E, D, I, k2, cb):
    picks = np.concatenate([orc.topk8(l, bias)[0].reshape(-1) for l in logits_list])
    return synth.HostLayer(seed, experts=E, dims=D, width=I, k2=k2, cb=cb, only=np.unique(picks))


def _case(ea, rows_seq, D, I, k2, cb, shared_k2, shared_cb, x_dtype, seed, cap=16):
    device, linear, moe, synth = ea
    E = 256
    logits_list, bias = [], None
    for i, R in enumerate(rows_seq):
        l, b = synth.logits(seed + i, R)
        bias = b if bias is None else bias
        logits_list.append(l)
    host = _layer_for(synth, seed + 10, logits_list, bias, E, D, I, k2, cb)
    shared = None if shared_k2 is None else SharedHost(linear, synth, seed + 20, D, I, shared_k2, shared_cb)
    ex = moe.Routed(host)
    sc = moe.Scratch(ex, cap, 8)
    for i, R in enumerate(rows_seq):
        x = synth.activations(seed + 30 + i, R, D, ["f16", "bf16"][x_dtype])
        out, pick, wts = _run(ea, host, shared, sc, ex, x, logits_list[i], bias, R, x_dtype)
        want, pick_w, wts_w = _want(host, shared, x, logits_list[i], bias, R, x_dtype == 1)
        np.testing.assert_array_equal(pick, pick_w)
        np.testing.assert_array_equal(wts, wts_w)
        assert_close_rms(out, want, 2e-3, f"ffn decode R={R} call {i}")


def test_ffn_decode_config2_shape(ea):
    """BASELINE config 2 at its real shape: one token, D 6144, 256 experts x I 256 at 4 bits (mcg), the 4-bit shared
    expert; three calls on one scratch."""
    _case(ea, [1, 1, 1], 6144, 256, 8, 1, 8, 1, 0, 100)


def test_ffn_decode_rows_change(ea):
    """16 rows, then 3, then 16 again on one scratch; 3-bit routed experts, a 5-bit mul1 shared expert (the real
    checkpoints' format), bf16 activations."""
    _case(ea, [16, 3, 16], 6144, 256, 6, 1, 10, 2, 1, 200)


def test_ffn_decode_mixed_widths(ea):
    """Config 3's routed part: 16 rows, 70 % of the experts at 3 bits, the rest at 4; shared expert at 4 bits."""
    device, linear, moe, synth = ea
    _case(ea, [16], 6144, 256, synth.mixed_widths(301, 256), 1, 8, 1, 0, 300)


@pytest.mark.parametrize("k2", [2, 3, 4, 5, 7, 9])
def test_ffn_decode_every_width(ea, k2):
    """The widths the tests above leave out (K2 6, 8 and 10 are theirs), for the routed experts and the shared expert
    alike: one row (the one-launch layer), then four (the multi-row launches), mcg codebook, D 1024."""
    _case(ea, [1, 4], 1024, 256, k2, 1, k2, 1, 0, 700 + k2)


@pytest.mark.parametrize("shared_cb", [1, 2])
def test_ffn_decode_3inst_routed(ea, shared_cb):
    """3inst routed experts (the reference's grouped kernel takes every codebook) beside an mcg or a mul1 shared
    expert (the codebooks its linear takes), one row and then three."""
    _case(ea, [1, 3], 2048, 256, 8, 0, 8, shared_cb, 0, 800 + shared_cb)


def test_ffn_decode_routed_only_i128(ea):
    """No shared expert, I = 128 (a TP=16 shard), mul1 routed experts."""
    _case(ea, [5, 2], 2048, 128, 10, 2, None, None, 0, 400)


def test_moe_routed_fused_matches_sequence(ea):
    """ea_moe_routed takes the decode layer for a scratch of <= 16 rows, the prefill path's item GEMMs in the scratch's
    prompt region for 17..128 rows, and the six-launch sequence above that; all three meet the bar against the oracle on
    the same inputs (and agree with each other to the same bar)."""
    device, linear, moe, synth = ea
    R, E, D, I = 12, 256, 2048, 256
    pick = synth.picks_uniform(500, R, E, 8)
    pick[2, 3] = pick[2, 5]  # a row may name one expert twice (the caller's pick, not top-k's): two members
    pick[2, 5] = pick[2, 3]
    wts = synth.routing_weights(501, R, 8)
    host = synth.HostLayer(502, experts=E, dims=D, width=I, k2=8, only=np.unique(pick))
    x = synth.activations(503, R, D, "f16")
    want = orc.moe_routed(x, pick, wts, oracle_routed(host), R, 8)
    ex = moe.Routed(host)
    dx, dp, dw = device.upload(x), device.upload(pick), device.upload(wts)
    outs = []
    for cap in (16, 32, 200):
        sc = moe.Scratch(ex, cap, 8)
        assert (sc.c.fused != 0) == (cap <= 128)
        out = device.zeros((R, D), torch.float32)
        moe.routed(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R, x_dtype=0)
        outs.append(device.download(out))
        assert device.device_status() == 0
        assert_close_rms(outs[-1], want, 2e-3, f"moe.routed cap={cap}")
    assert_close_rms(outs[0], outs[1], 2e-3, "decode layer vs prefill path")
    assert_close_rms(outs[0], outs[2], 2e-3, "decode layer vs sequence")


def test_ffn_decode_one_row_routed_only_i128(ea):
    """One row (the down launch computes its own SwiGLU inputs from the gate|up partials) with no shared expert,
    I = 128 and bf16 activations."""
    _case(ea, [1, 1], 2048, 128, 8, 1, None, None, 1, 600)


@pytest.mark.parametrize("repeat,mixed", [(False, False), (True, False), (False, True), (True, True)])
def test_moe_routed_one_row_given_picks(ea, repeat, mixed):
    """One row with caller-given picks; with `mixed` one picked expert is 3-bit beside 4-bit ones. With `repeat` the
    picks name one expert three times: like the reference's grouping (exl3_experts.cu:83-86 with maxm = R,
    moe.zig:288) a unit keeps its first R pairs, so slots 4 and 6 are not computed and read y as it is (zero in a new
    scratch). The reference's combine reads its shared z scratch for such a slot instead, which then holds another
    pair's gate|up partials, so the expected output is the oracle's with those two slots empty."""
    device, linear, moe, synth = ea
    R, E, D, I = 1, 64, 1024, 256
    pick = synth.picks_uniform(700, R, E, 8)
    if repeat:
        pick[0, 4] = pick[0, 1]
        pick[0, 6] = pick[0, 1]
    wts = synth.routing_weights(701, R, 8)
    k2 = np.full(E, 8, np.int32)
    if mixed:
        k2[pick[0, 2]] = 6
    host = synth.HostLayer(702, experts=E, dims=D, width=I, k2=k2, only=np.unique(pick))
    x = synth.activations(703, R, D, "f16")
    computed = pick.copy()
    if repeat:
        computed[0, 4] = computed[0, 6] = -1
    want = orc.moe_routed(x, computed, wts, oracle_routed(host), R, 8)
    ex = moe.Routed(host)
    sc = moe.Scratch(ex, 1, 8)
    assert sc.c.fused != 0
    dx, dp, dw = device.upload(x), device.upload(pick), device.upload(wts)
    out = device.zeros((R, D), torch.float32)
    moe.routed(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R, x_dtype=0)
    got = device.download(out)
    assert device.device_status() == 0
    assert_close_rms(got, want, 2e-3, f"moe.routed R=1 repeat={repeat} mixed={mixed}")


def test_topk8_nan_policy_both_paths(ea):
    """One NaN rule for both top-8 paths (ea_topk8 and the decode layer's per-block top-8), the oracle's: a NaN choice
    ranks below every number (-inf included), NaNs among themselves by the lower id. Rows where fewer than eight
    choices are numbers pick NaN experts (their wts are then NaN, as the sum is)."""
    device, linear, moe, synth = ea
    from ea_exl3 import ops

    R, E, D, I = 5, 256, 2048, 128
    logits, bias = synth.logits(900, R)
    bias[17] = -np.inf
    logits[1, [7, 100, 200]] = np.nan
    logits[2, :] = np.nan
    logits[2, [9, 40, 41, 250, 3, 17]] = [0.5, -1.0, 2.0, 0.0, -np.inf, 1.0]
    logits[3, :] = np.nan
    pick_w, wts_w = orc.topk8(logits, bias)
    dl, db = device.upload(logits), device.upload(bias)
    dp, dw = device.zeros((R, 8), torch.int32), device.zeros((R, 8), torch.float32)
    ops.topk(device.stream(), dl.data_ptr(), db.data_ptr(), dp.data_ptr(), dw.data_ptr(), R, 2.5)
    np.testing.assert_array_equal(device.download(dp), pick_w)
    np.testing.assert_array_equal(device.download(dw), wts_w)
    host = synth.HostLayer(901, experts=E, dims=D, width=I, k2=8, only=np.unique(pick_w))
    ex = moe.Routed(host)
    for rows in (R, 1):  # the multi-row route launch, and the one-row per-block routing (row 2 alone)
        lg = logits if rows == R else logits[2:3]
        sc = moe.Scratch(ex, rows, 8)
        x = synth.activations(902, rows, D, "f16")
        _, pick, wts = _run(ea, host, None, sc, ex, x, lg, bias, rows, 0)
        np.testing.assert_array_equal(pick, pick_w if rows == R else pick_w[2:3])
        np.testing.assert_array_equal(wts, wts_w if rows == R else wts_w[2:3])


def _epoch_word(sc):
    """The one-row launch's epoch word: the first word of the scratch's decode-layer region."""
    return sc.c.fused - sc.buf.data_ptr()


def test_one_row_epoch_wraps(ea):
    """The epoch word set just below its wrap: three launches tag with 0xFFFFFFFF, then 1 (0, a cleared slot's tag, is
    skipped), then 2; each launch's output meets the oracle, and the word holds the last launch's tag."""
    device, linear, moe, synth = ea
    E, D, I = 256, 1024, 128
    logits_list, bias = [], None
    for i in range(3):
        l, b = synth.logits(1400 + i, 1)
        bias = b if bias is None else bias
        logits_list.append(l)
    host = _layer_for(synth, 1410, logits_list, bias, E, D, I, 8, 1)
    shared = SharedHost(linear, synth, 1420, D, I, 8, 1)
    ex = moe.Routed(host)
    sc = moe.Scratch(ex, 1, 8)
    off = _epoch_word(sc)
    torch.cuda.synchronize()
    sc.buf[off:off + 4] = torch.tensor([0xFE, 0xFF, 0xFF, 0xFF], dtype=torch.uint8, device="cuda")
    tags = []
    for i in range(3):
        x = synth.activations(1430 + i, 1, D, "f16")
        out, pick, wts = _run(ea, host, shared, sc, ex, x, logits_list[i], bias, 1, 0)
        want, pick_w, wts_w = _want(host, shared, x, logits_list[i], bias, 1, False)
        np.testing.assert_array_equal(pick, pick_w)
        assert_close_rms(out, want, 2e-3, f"launch {i} across the epoch's wrap")
        tags.append(int(sc.buf[off:off + 4].cpu().numpy().view(np.uint32)[0]))
    assert tags == [0xFFFFFFFF, 1, 2], tags


def test_one_row_scratch_across_layer_shapes(ea):
    """One scratch (made for the larger layer) used by two layer shapes in turn, D 2048 / I 256 and D 1024 / I 128: the
    tagged slots sit at the same offsets for every shape and a slot's tag half only ever holds tags, so no launch
    takes another shape's stale values for its own."""
    device, linear, moe, synth = ea
    E = 256
    layers = []
    for j, (D, I) in enumerate(((2048, 256), (1024, 128))):
        ls, bias = [], None
        for i in range(2):
            l, b = synth.logits(1500 + 10 * j + i, 1)
            bias = b if bias is None else bias
            ls.append(l)
        host = _layer_for(synth, 1520 + j, ls, bias, E, D, I, 8, 1)
        layers.append((D, I, host, moe.Routed(host), SharedHost(linear, synth, 1530 + j, D, I, 8, 1), ls, bias))
    sc = moe.Scratch(layers[0][3], 1, 8)
    for n, j in enumerate((0, 1, 0, 1)):
        D, I, host, ex, shared, ls, bias = layers[j]
        x = synth.activations(1540 + n, 1, D, "f16")
        lg = ls[n // 2]
        out, pick, wts = _run(ea, host, shared, sc, ex, x, lg, bias, 1, 0)
        want, pick_w, wts_w = _want(host, shared, x, lg, bias, 1, False)
        np.testing.assert_array_equal(pick, pick_w)
        assert_close_rms(out, want, 2e-3, f"call {n}: D {D}, I {I}")


def test_one_row_topk_ties_and_wide_spread(ea):
    """The one-row layer's top-8 (a selection: the eighth largest key, then ties by the lower id, then each pick's
    slot by rank) against the oracle's eight argmax rounds, bit for bit, on rows built to stress it: every expert
    tied, an exact tie between two strong experts, logits on a coarse grid (many ties at every level), eight equal
    maxima, the largest choices at the highest ids, and logits spread over many binades."""
    device, linear, moe, synth = ea
    E, D, I = 256, 1024, 128
    logits, bias = synth.logits(1300, 8)
    logits[0, :] = 0.25
    logits[1, 10] = logits[1, 20] = 5.0
    logits[2] = np.round(logits[2] * 2) / 2
    logits[3, :] = -1.0
    logits[3, [200, 3, 77, 150, 9, 255, 0, 128]] = 3.0
    logits[4] = np.linspace(-6, 6, 256, dtype=np.float32)
    logits[5] = (np.sign(logits[5]) * np.exp2(np.abs(logits[5]) * 20)).astype(np.float32)
    logits[6, :] = 0.25
    logits[6, 250:] = 0.5
    logits[7] = np.round(logits[7])
    bias0 = np.zeros_like(bias)
    for b in (bias0, bias):
        pick_w, wts_w = orc.topk8(logits, b)
        host = synth.HostLayer(1301, experts=E, dims=D, width=I, k2=8, only=np.unique(pick_w))
        ex = moe.Routed(host)
        sc = moe.Scratch(ex, 1, 8)
        x = synth.activations(1302, 1, D, "f16")
        for r in range(logits.shape[0]):
            _, pick, wts = _run(ea, host, None, sc, ex, x, logits[r:r + 1], b, 1, 0)
            np.testing.assert_array_equal(pick, pick_w[r:r + 1], err_msg=f"row {r}")
            np.testing.assert_array_equal(wts, wts_w[r:r + 1], err_msg=f"row {r}")


def test_unsupported_width_poisons_output(ea):
    """A width table entry the decode layer has no decoder for (an expert at K2 12 in a layer whose host tables claim
    widths 8..8): the kernels record EA_UNSUPPORTED_WIDTH (19) in the status word, which ea_device_status_address
    exposes for asynchronous checks, and store NaN in place of that expert's sums, so the row's output is NaN. The
    condition is set from the host; every load stays inside the expert's real trellis and every kernel exits."""
    import ctypes as C

    device, linear, moe, synth = ea
    from ea_exl3._lib import lib

    R, E, D, I = 1, 64, 1024, 256
    pick = synth.picks_uniform(950, R, E, 8)
    wts = synth.routing_weights(951, R, 8)
    k2 = np.full(E, 8, np.int32)
    k2[pick[0, 2]] = 12
    host = synth.HostLayer(952, experts=E, dims=D, width=I, k2=k2, only=np.unique(pick))
    ex = moe.Routed(host)
    ex.k2_gu, ex.k2_d = (8, 8), (8, 8)  # what the host claims: the decode layer's path
    ex.c = ex.struct()
    sc = moe.Scratch(ex, 1, 8)
    assert sc.c.fused != 0
    x = synth.activations(953, R, D, "f16")
    dx, dp, dw = device.upload(x), device.upload(pick), device.upload(wts)
    out = device.zeros((R, D), torch.float32)
    assert device.device_status() == 0
    moe.routed(device.stream(), dx.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc, out.data_ptr(), R, x_dtype=0)
    torch.cuda.synchronize()
    addr = C.c_void_p(0)
    assert lib().ea_device_status_address(C.byref(addr)) == 0 and addr.value
    word = C.c_int32(0)
    hip = C.CDLL("libamdhip64.so")
    assert hip.hipMemcpy(C.byref(word), addr, C.c_size_t(4), 2) == 0  # hipMemcpyDeviceToHost
    assert word.value == 19
    assert np.isnan(device.download(out)).all()
    assert device.device_status() == 19  # read and cleared
    assert device.device_status() == 0


@pytest.mark.parametrize("rows_seq,x_dtype", [([1, 1], 0), ([16, 4], 1), ([1], 1)])
def test_ffn_decode_from_router(ea, rows_seq, x_dtype):
    """ea_ffn_moe_decode_router: the router's logits (bf16 router weight [256, D], ops.router's ordered slices) written
    to the caller's buffer and then routed, as forward.zig:2350-2403 does. The logits must be the oracle router's bits,
    pick / wts the oracle top-8's of them, out within 2e-3 * RMS(out); one and sixteen rows on one scratch."""
    device, linear, moe, synth = ea
    E, D, I, seed = 256, 6144, 256, 1300
    rng = np.random.default_rng(seed)
    rw = synth.bf16_bits((0.02 * rng.standard_normal((E, D))).astype(np.float32))
    xs = [synth.activations(seed + 1 + i, R, D, ["f16", "bf16"][x_dtype]) for i, R in enumerate(rows_seq)]
    _, bias = synth.logits(seed, 1)
    logits_list = [orc.router(x, rw, x_dtype) for x in xs]
    host = _layer_for(synth, seed + 10, logits_list, bias, E, D, I, 8, 1)
    shared = SharedHost(linear, synth, seed + 20, D, I, 8, 1)
    ex = moe.Routed(host)
    sc = moe.Scratch(ex, 16, 8)
    drw, db = device.upload(rw), device.upload(bias)
    for i, R in enumerate(rows_seq):
        x = xs[i]
        print(f"decode from router R={R} x_dtype={x_dtype}", flush=True)
        dx = device.upload(x)
        dl = device.zeros((R, E), torch.float32)
        dp, dw = device.zeros((R, 8), torch.int32), device.zeros((R, 8), torch.float32)
        out = device.zeros((R, D), torch.float32)
        moe.ffn_decode_router(device.stream(), dx.data_ptr(), D, drw.data_ptr(), dl.data_ptr(), db.data_ptr(), 2.5,
                              dp.data_ptr(), dw.data_ptr(), ex, [l.c for l in shared.lin], sc, out.data_ptr(), R,
                              x_dtype=x_dtype)
        np.testing.assert_array_equal(device.download(dl).view(np.uint32), logits_list[i].view(np.uint32))
        want, pick_w, wts_w = _want(host, shared, x, logits_list[i], bias, R, x_dtype == 1)
        np.testing.assert_array_equal(device.download(dp), pick_w)
        np.testing.assert_array_equal(device.download(dw), wts_w)
        assert_close_rms(device.download(out), want, 2e-3, f"ffn decode from router R={R}")
        assert device.device_status() == 0
