"""Pins the oracle's arithmetic above the trellis decode: number-format rounding against numpy / exact rationals,
the path's exp, grouping / routing / top-8 against brute force, and whole layers (decode path, prefill path, EXL3
linear) against the dense fp64 linear algebra they must equal: W = diag(suh) (H / sqrt 128) W_q (H / sqrt 128)
diag(svh). A transposed operand, a dropped scale or a wrong rotation side fails these by orders of magnitude over
their tolerance. CPU only."""
import math
from fractions import Fraction

import numpy as np
import pytest

import oracle as orc
from ea_exl3 import synth
from helpers import assert_close_rms, h2f, oracle_routed


# ---- number formats ------------------------------------------------------------------------------------------------

def test_f2h_matches_numpy_everywhere():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[np.isfinite(f)]
    # focus on the fp16 range, subnormals and overflow edges too
    f = np.concatenate([f, (rng.standard_normal(100000) * 10.0 ** rng.integers(-9, 6, 100000)).astype(np.float32),
                        np.array([65504, 65519.99, 65520, -65520, 2**-24, 2**-25, 3 * 2**-26, 2**-14], np.float32)])
    L = orc.lib()
    got = np.array([L.or_f2h(float(v)) for v in f[:60000]], np.uint16)
    want = f[:60000].astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)


def test_d2h_rounds_exact_values_once():
    # values exactly halfway between fp16 neighbours in double, and just off the halfway point
    for m in range(1024, 2048, 37):
        for e in (-20, -14, -3, 0, 5, 14):
            lo = Fraction(m) * Fraction(2) ** (e - 10)
            half = lo + Fraction(2) ** (e - 11)
            d = float(half)
            got = orc.d2h(d)
            want = np.float16(float(lo) if m % 2 == 0 else float(lo + Fraction(2) ** (e - 10)))
            if e >= -14 and want != np.inf:
                assert got == int(np.array([want]).view(np.uint16)[0]), (m, e)


def test_expf_within_two_ulp():
    xs = np.concatenate([np.linspace(-100, 88, 20001), np.random.default_rng(1).standard_normal(5000) * 20])
    for x in xs.astype(np.float32):
        got = orc.expf(float(x))
        want = math.exp(float(x))
        if want < 1e-37:  # subnormal results: absolute bar
            assert abs(got - want) < 1e-44
            continue
        assert abs(got - want) <= 2 * np.spacing(np.float32(want)), (x, got, want)
    assert orc.expf(0.0) == 1.0


# ---- grouping, routing and top-8 -------------------------------------------------------------------------------------

@pytest.mark.parametrize("R,E", [(1, 256), (16, 256), (16, 40), (64, 256)])
def test_group_brute_force(R, E):
    slots = 8
    pick = synth.picks_uniform(R + E, R, E, slots)
    pick[0, 0] = -1
    if R > 1:
        pick[1, 7] = E + 3
    uids, uc, members = orc.group(pick, R, slots, E, R)
    valid = sorted({int(e) for e in pick.reshape(-1) if 0 <= e < E})
    assert uc == len(valid)
    assert list(uids[:uc]) == valid
    for u, e in enumerate(valid):
        want = [r * 32 + s for r in range(R) for s in range(slots) if pick[r, s] == e]
        got = [m for m in members[u] if m >= 0]
        assert got == want[:R]
        assert all(m == -1 for m in members[u][len(got):])


@pytest.mark.parametrize("R", [1, 16, 600])
def test_route_items_cover_every_pair(R):
    slots, E, ipm = 8, 256, 112
    pick = synth.picks_zipf(R, R, 1.1, E, slots)
    pick[0, 1] = -1
    n = R * slots
    max_items = n // ipm + min(n, E)
    sorted_, items, ic = orc.route(pick, n, E, ipm, max_items)
    flat = pick.reshape(-1)
    counts = np.bincount(flat[flat >= 0], minlength=E)
    off, it = 0, 0
    for e in range(E):
        for f in range(0, counts[e], ipm):
            assert tuple(items[it]) == (e, off + f, min(ipm, counts[e] - f))
            it += 1
        assert sorted(sorted_[off: off + counts[e]]) == sorted(np.nonzero(flat == e)[0])
        off += counts[e]
    assert ic == it


def test_topk_brute_force_and_ties():
    """The top-8 against a sort: the larger choice first, the lower id on a tie, a NaN choice below every number
    (-inf included) and NaNs among themselves by id."""
    logits, bias = synth.logits(3, 40)
    logits[0, :] = 0.0
    bias[:] = np.round(bias, 1)  # many exact ties in choice
    logits[1, 5] = logits[1, 9] = 3.0
    logits[2, [7, 100, 200]] = np.nan  # NaN choices that are never reached
    bias[17] = -np.inf  # a choice of -inf wherever expert 17's logit is a number
    logits[3, :] = np.nan  # six numbers (one choice -inf), so two NaN picks follow them
    logits[3, [9, 40, 41, 250, 3, 17]] = [0.5, -1.0, 2.0, 0.0, -np.inf, 1.0]
    logits[4, :] = np.nan  # NaN everywhere: ids 0..7
    pick, wts = orc.topk8(logits, bias)
    for r in range(logits.shape[0]):
        score = np.array([np.float32(1) / (np.float32(orc.expf(-float(l))) + np.float32(1)) for l in logits[r]],
                         np.float32)
        choice = (score + bias).astype(np.float32)
        order = sorted(range(256), key=lambda e: (1, 0.0, e) if np.isnan(choice[e]) else (0, -float(choice[e]), e))[:8]
        assert list(pick[r]) == order
        total = np.float32(0)
        for e in order:
            total = np.float32(total + score[e])
        want = (score[order] / np.float32(total + np.float32(1e-20)) * np.float32(2.5)).astype(np.float32)
        np.testing.assert_array_equal(wts[r], want)


# ---- dense fp64 identities -----------------------------------------------------------------------------------------

def _hadamard():
    i = np.arange(128)
    pc = np.vectorize(lambda v: bin(v).count("1"))(i[:, None] & i[None, :])
    return np.where(pc % 2 == 0, 1.0, -1.0)


def _block_h(n):
    H = _hadamard() / math.sqrt(128.0)
    return np.kron(np.eye(n // 128), H)


def dense_weight(T, K, N, k2, cb, suh_bits, svh_bits):
    """W [K, N] fp64 such that y = x @ W is what an EXL3 linear computes (before fp16 roundings)."""
    Wq = h2f(orc.dequant_expert(T, K, N, k2, cb)).astype(np.float64)
    return (h2f(suh_bits).astype(np.float64)[:, None] * _block_h(K)) @ Wq @ _block_h(N) * \
        h2f(svh_bits).astype(np.float64)[None, :]


def dense_layer(host, x, pick, wts, R, slots):
    D, I = host.dims, host.width
    out = np.zeros((R, D))
    for r in range(R):
        for k in range(slots):
            e = int(pick[r, k])
            if e < 0:
                continue
            Wg = dense_weight(host.matrix(0, e), D, I, int(host.k2[0][e]), host.cb, host.suh_g[e * D:(e + 1) * D],
                              host.svh_g[e * I:(e + 1) * I])
            Wu = dense_weight(host.matrix(1, e), D, I, int(host.k2[1][e]), host.cb, host.suh_u[e * D:(e + 1) * D],
                              host.svh_u[e * I:(e + 1) * I])
            Wd = dense_weight(host.matrix(2, e), I, D, int(host.k2[2][e]), host.cb, host.suh_d[e * I:(e + 1) * I],
                              host.svh_d[e * D:(e + 1) * D])
            g = x[r] @ Wg
            u = x[r] @ Wu
            act = g / (1.0 + np.exp(-g)) * u
            out[r] += float(wts[r, k]) * (act @ Wd)
    return out


@pytest.mark.parametrize("R,k2", [(1, 8), (3, 6), (2, "mixed")])
def test_moe_routed_equals_dense_layer(R, k2):
    E, D, I, slots = 16, 512, 256, 8
    pick = synth.picks_uniform(70 + R, R, E, slots)
    wts = synth.routing_weights(71, R, slots)
    k2v = synth.mixed_widths(72, E) if k2 == "mixed" else k2
    host = synth.HostLayer(73, experts=E, dims=D, width=I, k2=k2v)
    x16 = synth.activations(74, R, D, "f16")
    got = orc.moe_routed(x16, pick, wts, oracle_routed(host), R, slots)
    want = dense_layer(host, h2f(x16).astype(np.float64), pick, wts, R, slots)
    assert_close_rms(got, want, 2e-3, "oracle moe.routed vs dense fp64")


def test_prompt_experts_equals_dense_layer():
    E, D, I, slots, R = 16, 256, 128, 8, 20
    pick = synth.picks_zipf(80, R, 1.1, E, slots)
    wts = synth.routing_weights(81, R, slots)
    host = synth.HostLayer(82, experts=E, dims=D, width=I, k2=8)
    x = synth.activations(83, R, D, "bf16")
    got = orc.prompt_experts(x, pick, wts, oracle_routed(host), R, slots, bf16=True)
    want = dense_layer(host, synth.bf16_to_f32(x).astype(np.float64), pick, wts, R, slots)
    assert_close_rms(got, want, 2e-3, "oracle prompt experts vs dense fp64")
    rounded = orc.prompt_experts(x, pick, wts, oracle_routed(host), R, slots, do_round=True, bf16=True)
    np.testing.assert_array_equal(rounded, synth.bf16_to_f32(synth.bf16_bits(got)))


@pytest.mark.parametrize("M,K,N,k2,cb", [(1, 512, 256, 8, 1), (5, 256, 384, 10, 2), (17, 768, 128, 6, 1)])
def test_exl3_linear_equals_dense(M, K, N, k2, cb):
    T = synth.trellis(90, 0, 0, M, K, N, k2)
    suh = synth.scales(91, K, 1.0)
    svh = synth.scales(92, N, 0.02)
    x = synth.activations(93, M, K, "bf16")
    S = orc.expert_to_strips(T, K, N, k2)
    tw = 4 * k2
    sk, wk = orc.linear_plan(K, N)
    xh = orc.exl3_rot_in(x, suh, M, K, bf16=True)
    y = orc.exl3_linear(xh, S, 8 * tw, (K // 16) * 8 * tw, svh, M, K, N, k2, cb, sk, wk)
    want = synth.bf16_to_f32(x).astype(np.float64) @ dense_weight(T, K, N, k2, cb, suh, svh)
    assert_close_rms(y, want, 2e-3, "oracle exl3 linear vs dense fp64")


# ---- the shared expert's activation --------------------------------------------------------------------------------

def test_swiglu2_against_float64_and_closed_forms():
    """swiglu2 (native_ops.cu:429-441): out = bf16(bf16(silu(g)) * u). Against float64 silu with the same two bf16
    rounding points the result may differ by one bf16 ulp (the fp32 exp); silu(0) = 0 exactly; for g >= 20,
    silu(g) rounds to g in bf16, so out = bf16(g * u); a sign flip of u flips the output's sign."""
    rng = np.random.default_rng(7)
    g = synth.bf16_bits(rng.standard_normal(4096) * 4)
    u = synth.bf16_bits(rng.standard_normal(4096))
    got = synth.bf16_to_f32(orc.swiglu2(g, u)).astype(np.float64)
    gf, uf = synth.bf16_to_f32(g).astype(np.float64), synth.bf16_to_f32(u).astype(np.float64)
    s = synth.bf16_to_f32(synth.bf16_bits(gf / (1.0 + np.exp(-gf)))).astype(np.float64)
    want = synth.bf16_to_f32(synth.bf16_bits(s * uf)).astype(np.float64)
    ulp = np.abs(want) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(got - want) <= ulp)
    zero = synth.bf16_bits(np.zeros(8))
    assert np.all(synth.bf16_to_f32(orc.swiglu2(zero, u[:8])) == 0.0)
    big = synth.bf16_bits(np.full(8, 24.0))
    np.testing.assert_array_equal(orc.swiglu2(big, u[:8]), synth.bf16_bits(24.0 * synth.bf16_to_f32(u[:8])))
    neg = synth.bf16_bits(-synth.bf16_to_f32(u))
    np.testing.assert_array_equal(synth.bf16_to_f32(orc.swiglu2(g, neg)), -synth.bf16_to_f32(orc.swiglu2(g, u)))


# ---- the gate / up epilogue's activation modes, against float64 ------------------------------------------------------

def _epilogue_fp64(Z, pick, svh_g, svh_u, suh_d, P, N, SK, limit):
    """xd [P, N] in float64: splits summed, H / sqrt(128) per 128 columns, svh, SwiGLU with the limit's clamps, suh_d,
    H / sqrt(128) again (exl3_experts.cu:142-184, no roundings)."""
    Hb = _block_h(N)
    out = np.full((P, N), np.nan)
    for p in range(P):
        e = int(pick.reshape(-1)[p])
        if e < 0:
            continue
        g = Z[0, :, p, :].astype(np.float64).sum(axis=0) @ Hb * h2f(svh_g[e]).astype(np.float64)
        u = Z[1, :, p, :].astype(np.float64).sum(axis=0) @ Hb * h2f(svh_u[e]).astype(np.float64)
        g = np.minimum(g, limit)
        u = np.clip(u, -limit, limit)
        act = g / (1.0 + np.exp(-g)) * u
        out[p] = (act * h2f(suh_d[e]).astype(np.float64)) @ Hb
    return out


def test_gateup_epilogue_act_modes_against_fp64():
    """The oracle's epilogue in both activation modes against a float64 restatement built from the Sylvester matrix:
    act_mode 1 (fp32) within fp16 output rounding, act_mode 0 within its three bf16 roundings, and act_mode 0 apart
    from act_mode 1 by about those roundings (so they happen). A dropped or swapped clamp, g and u exchanged, or a
    missing Hadamard fails by far more; the limit is small enough that about a fifth of the values are clamped."""
    from types import SimpleNamespace

    rng = np.random.default_rng(5)
    R, E, N, SK, slots = 3, 16, 256, 4, 8
    P = R * slots
    pick = synth.picks_uniform(21, R, E, slots)
    pick[0, 3] = -1
    Z = (rng.standard_normal((2, SK, P, N)) * 2.0).astype(np.float32)
    svh_g, svh_u, suh_d = (synth.scales(31 + i, E * N, 1.0).reshape(E, N) for i in range(3))
    r = SimpleNamespace(svh_g=svh_g, svh_u=svh_u, suh_d=suh_d)
    limit = 5.0
    want = _epilogue_fp64(Z, pick, svh_g, svh_u, suh_d, P, N, SK, limit)
    ok = pick.reshape(-1) >= 0
    ref = want[ok]
    rms = float(np.sqrt(np.mean(ref ** 2)))
    # how much the clamps bite: the same activation without them differs by far more than the bars below
    g_all = np.concatenate([Z[0, :, p, :].sum(axis=0) @ _block_h(N) * h2f(svh_g[int(pick.reshape(-1)[p])])
                            for p in np.nonzero(ok)[0]])
    assert 0.1 < float(np.mean(np.abs(g_all) > limit)) < 0.4
    got = {}
    for mode in (1, 0):
        xd = orc.gateup_epilogue(Z, pick, r, R, P, N, SK, slots, E, limit, mode)
        got[mode] = h2f(xd).astype(np.float64)[ok]
    d1 = got[1] - ref
    assert np.all(np.abs(d1) <= 2.0 ** -10 * np.abs(ref) + 1e-5 * rms), "act_mode 1 off the float64 epilogue"
    d0 = got[0] - ref
    assert float(np.sqrt(np.mean(d0 ** 2))) < 0.01 * rms, "act_mode 0 off the float64 epilogue"
    assert float(np.max(np.abs(d0))) < 0.08 * rms
    sep = float(np.sqrt(np.mean((got[0] - got[1]) ** 2)))
    assert 2e-4 * rms < sep < 0.01 * rms, f"act_mode 0 vs 1: {sep / rms:.2e} of RMS (the bf16 roundings)"
