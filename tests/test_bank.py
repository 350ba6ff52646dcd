"""Expert banks on the host (no GPU): the library's checkpoint reader (weights.zig Reader over split.zig's rules)
against numpy slicing of the same whole matrices.

  - a rank's share of a whole-matrix checkpoint: gate / up trellis cut on the tile columns and svh on its rows, down
    trellis and suh on the rows, the other scale and the codebook marker whole (split.zig:43-58, weights.zig cut);
  - the same shares from a pre-sharded bank (assemble.py:173-237's "...P_proj.rank{r}.S" layout) read with as many
    ranks as were stored, and with fewer (two stored ranks joined a share: weights.zig join);
  - the refusals: a share that would cut a Hadamard block (split.zig:69), an axis that does not divide, a missing
    tensor, stored ranks that are not a multiple of the ranks, an index without a weight_map."""
import json
import os

import numpy as np
import pytest

from ea_exl3 import bank, synth
from ea_exl3._lib import EaError

LAYER, E, D, WORLD = 5, 3, 256, 8


def _layer(I_total, seed=50, k2s=(8, 6, 8)):
    """Whole matrices of E experts: gate / up [D, I_total], down [I_total, D]."""
    shapes = [(D, I_total), (D, I_total), (I_total, D)]
    T = [[synth.trellis(seed, LAYER, p, e, K, N, k2s[e]) for e in range(E)] for p, (K, N) in enumerate(shapes)]
    suh = [[synth.scales(seed + 1 + 10 * p + e, K, 1.0) for e in range(E)] for p, (K, N) in enumerate(shapes)]
    svh = [[synth.scales(seed + 2 + 10 * p + e, N, 0.02) for e in range(E)] for p, (K, N) in enumerate(shapes)]
    return T, suh, svh


def _whole(T, suh, svh, p, e, part):
    K, N = len(suh[p][e]), len(svh[p][e])
    if part == "trellis":
        w = np.asarray(T[p][e], np.uint32).view(np.int16)
        return w.reshape(K // 16, N // 16, -1)
    return np.asarray((suh if part == "suh" else svh)[p][e], np.uint16).view(np.float16)


def _want(T, suh, svh, p, e, part, rank, world):
    a = _whole(T, suh, svh, p, e, part)
    down = p == 2
    if part == "trellis":
        n = a.shape[0 if down else 1] // world
        return a[rank * n:(rank + 1) * n] if down else a[:, rank * n:(rank + 1) * n]
    if (part == "suh") == down:
        n = a.shape[0] // world
        return a[rank * n:(rank + 1) * n]
    return a


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("ckpt"))
    T, suh, svh = _layer(WORLD * 128)
    bank.write_checkpoint_layer(d, LAYER, T, suh, svh, cb=1)
    b = str(tmp_path_factory.mktemp("bank"))
    bank.reslice_layer(bank.layer_tensors(LAYER, T, suh, svh, 1), LAYER, b, WORLD)
    return d, b, (T, suh, svh)


@pytest.mark.parametrize("rank", [0, 3, 7])
def test_checkpoint_shares_match_numpy(ckpt, rank):
    d, _, (T, suh, svh) = ckpt
    r = bank.Reader(d, rank, WORLD, WORLD)
    for e in range(E):
        for p, proj in enumerate(bank.PROJ):
            for part in ("trellis", "suh", "svh"):
                got = r.get(bank.expert_name(LAYER, e, proj, part))
                want = _want(T, suh, svh, p, e, part, rank, WORLD)
                assert got.shape == want.shape, (proj, part)
                np.testing.assert_array_equal(got.view(np.uint8), np.ascontiguousarray(want).view(np.uint8))
            assert r.has(bank.expert_name(LAYER, e, proj, "mcg"))
            assert not r.has(bank.expert_name(LAYER, e, proj, "mul1"))
    r.close()


@pytest.mark.parametrize("world,rank", [(8, 5), (4, 1), (2, 1), (1, 0)])
def test_bank_shares_join_stored_ranks(ckpt, world, rank):
    """A bank of 8 stored ranks read by `world` ranks: each share joins 8 / world stored ranks in order and equals
    the whole matrix cut for `world`."""
    _, b, (T, suh, svh) = ckpt
    r = bank.Reader(b, rank, world, WORLD, fname=bank.bank_file(LAYER))
    for e in range(E):
        for p, proj in enumerate(bank.PROJ):
            for part in ("trellis", "suh", "svh"):
                got = r.get(bank.expert_name(LAYER, e, proj, part))
                want = _want(T, suh, svh, p, e, part, rank, world)
                np.testing.assert_array_equal(got.view(np.uint8), np.ascontiguousarray(want).view(np.uint8))
            assert r.has(bank.expert_name(LAYER, e, proj, "mcg"))


def test_refusals(ckpt, tmp_path):
    d, b, _ = ckpt
    # a share of 64 columns (4 tiles) would cut a Hadamard block: I_total = 8 x 64
    T, suh, svh = _layer(WORLD * 64, seed=60)
    d2 = str(tmp_path / "narrow")
    bank.write_checkpoint_layer(d2, LAYER, T, suh, svh, cb=1)
    r = bank.Reader(d2, 1, WORLD, WORLD)
    with pytest.raises(EaError) as e:
        r.get(bank.expert_name(LAYER, 0, "gate", "trellis"))
    assert e.value.code == 26  # StraddlesHadamard
    with pytest.raises(EaError) as e:
        r.get(bank.expert_name(LAYER, 0, "up", "svh"))
    assert e.value.code == 26
    # an axis that does not divide: 7 ranks
    r7 = bank.Reader(d, 1, 7, 7)
    with pytest.raises(EaError) as e:
        r7.get(bank.expert_name(LAYER, 0, "down", "trellis"))
    assert e.value.code == 8  # UnevenSplit
    # a tensor that is not there, whole or stored
    r8 = bank.Reader(d, 0, WORLD, WORLD)
    with pytest.raises(EaError) as e:
        r8.get(bank.expert_name(LAYER, E, "gate", "trellis"))
    assert e.value.code == 24  # MissingTensor
    with pytest.raises(EaError) as e:  # a name with no split rule fails on the rule first (weights.zig:213-214)
        r8.get("model.layers.5.mystery")
    assert e.value.code == 25  # NoSplitRule
    # stored ranks not a multiple of the ranks
    with pytest.raises(EaError) as e:
        bank.Reader(b, 0, 3, WORLD, fname=bank.bank_file(LAYER))
    assert e.value.code == 27  # StoredWorldNotMultiple
    # an index without a weight_map
    bad = tmp_path / "badindex"
    bad.mkdir()
    (bad / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}}))
    with pytest.raises(EaError) as e:
        bank.Reader(str(bad), 0, 1, 1)
    assert e.value.code == 23  # BadIndex
    # a file whose header runs past its end
    junk = tmp_path / "junk"
    junk.mkdir()
    (junk / "x.safetensors").write_bytes((1 << 20).to_bytes(8, "little") + b"{}")
    with pytest.raises(EaError) as e:
        bank.Reader(str(junk), 0, 1, 1, fname="x.safetensors")
    assert e.value.code == 22  # BadSafetensors


def test_header_json_forms(tmp_path):
    """The header reader takes what JSON allows: whitespace, escaped names, a metadata object, any key order."""
    d = tmp_path / "j"
    d.mkdir()
    data = np.arange(12, dtype=np.float32)
    hdr = ('{ "__metadata__" : {"format":"pt","n":"1"},\n "a\\u0062c" : { "shape" : [3, 4], "data_offsets":[0,48],'
           ' "dtype":"F32" } }').encode()
    (d / "t.safetensors").write_bytes(len(hdr).to_bytes(8, "little") + hdr + data.tobytes())
    r = bank.Reader(str(d), 0, 1, 1, fname="t.safetensors")
    assert r.has("abc")
    with pytest.raises(EaError) as e:  # no split rule for a name outside the model's
        r.get("abc")
    assert e.value.code == 25  # NoSplitRule


def test_zero_size_and_overflowing_shapes(tmp_path):
    """A legal zero-size tensor is an empty share of the cut shape on every rank (no division by its zero axis); a
    header whose shape product overflows 64 bits is refused as BadSafetensors, not wrapped around."""
    d = tmp_path / "z"
    d.mkdir()
    name = bank.expert_name(LAYER, 0, "down", "suh")  # down's suh: cut on its rows
    hdr = json.dumps({name: {"dtype": "F16", "shape": [0], "data_offsets": [0, 0]}}).encode()
    (d / "z.safetensors").write_bytes(len(hdr).to_bytes(8, "little") + hdr)
    for rank in (0, 3):
        got = bank.Reader(str(d), rank, 4, 4, fname="z.safetensors").get(name)
        assert got.shape == (0,) and got.nbytes == 0
    tname = bank.expert_name(LAYER, 0, "gate", "trellis")  # gate's trellis: cut on its tile columns
    hdr = json.dumps({tname: {"dtype": "I16", "shape": [4, 0, 64], "data_offsets": [0, 0]}}).encode()
    (d / "t.safetensors").write_bytes(len(hdr).to_bytes(8, "little") + hdr)
    got = bank.Reader(str(d), 1, 2, 2, fname="t.safetensors").get(tname)
    assert got.shape == (4, 0, 64)
    big = 1 << 40
    hdr = json.dumps({name: {"dtype": "F16", "shape": [big, big], "data_offsets": [0, 0]}}).encode()
    (d / "o.safetensors").write_bytes(len(hdr).to_bytes(8, "little") + hdr)
    with pytest.raises(EaError) as e:
        bank.Reader(str(d), 0, 1, 1, fname="o.safetensors")
    assert e.value.code == 22  # BadSafetensors
