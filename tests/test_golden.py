"""The oracle and the seeded generator against the committed golden fixtures (tests/golden/golden.npz, written by
tests/golden/make_golden.py): codebook tables, tiles of every width and codebook, the router's top-8 and two
reduced-width MoE layers must reproduce bit for bit."""
import os
import sys

import numpy as np
import pytest

import oracle as orc

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as mg  # noqa: E402

G = np.load(os.path.join(HERE, "golden", "golden.npz"), allow_pickle=False)


def test_codebook_tables():
    for cb in range(3):
        assert mg.sha(orc.codebook_lut(cb)) == str(G["cb_lut_sha256"][cb])


@pytest.mark.parametrize("k2", mg.TILE_WIDTHS)
def test_tiles(k2):
    for cb in range(3):
        T, W = mg.tile_case(k2, cb)
        np.testing.assert_array_equal(T, G[f"tile_{k2}_{cb}_words"])
        np.testing.assert_array_equal(W, G[f"tile_{k2}_{cb}_w"])


def test_topk():
    logits, bias, pick, wts = mg.topk_case()
    np.testing.assert_array_equal(logits, G["topk_logits"])
    np.testing.assert_array_equal(pick, G["topk_pick"])
    np.testing.assert_array_equal(wts, G["topk_wts"])


@pytest.mark.parametrize("R", [1, 16])
def test_layer(R):
    _, _, _, _, out, digest = mg.layer_case(R)
    assert digest == str(G[f"layer_r{R}_inputs_sha256"]), "the seeded generator changed"
    np.testing.assert_array_equal(out, G[f"layer_r{R}_out"])
