"""The lane algorithm of the 8-values-a-lane FWHT (fwht128_x8 in csrc/ea_device.hpp), restated on the CPU in fp32 and
checked bit for bit against the plain butterflies (value-index bits 0..6 in order, lower + upper and lower - upper,
decode.cuh:146-161): lane l of a 16-lane group holds values 8 g(l) .. + 7 with g(l) = l ^ (3 * bit 2 of l); bits 0..2
are butterflies inside the lane; bits 3..6 are steps v + s * partner across lane distances 1, 2, 7, 8 (s = -1 in the
lane whose group has the step's bit set); the result is each lane's values times (-1)^popcount(g)."""
import numpy as np


def _plain(x):
    v = x.astype(np.float32).copy()
    for b in range(7):
        m = 1 << b
        idx = np.arange(128)
        lo = idx[(idx & m) == 0]
        a, c = v[lo].copy(), v[lo | m].copy()
        v[lo], v[lo | m] = a + c, a - c
    return v


def _group(l):
    return l ^ (((l >> 2) & 1) * 3)


def _lanes(x, fold=True, dists=((0, 1), (1, 2), (2, 7), (3, 8))):
    L = np.stack([x[8 * _group(l): 8 * _group(l) + 8] for l in range(16)]).astype(np.float32)
    for b in range(3):
        m = 1 << b
        j = np.arange(8)
        lo = j[(j & m) == 0]
        a, c = L[:, lo].copy(), L[:, lo | m].copy()
        L[:, lo], L[:, lo | m] = a + c, a - c
    for bit, dist in dists:
        P = L.copy()
        for l in range(16):
            s = np.float32(-1.0 if (_group(l) >> bit) & 1 else 1.0)
            L[l] = P[l] + s * P[l ^ dist]
    out = np.empty(128, np.float32)
    for l in range(16):
        nu = np.float32(-1.0 if fold and bin(_group(l)).count("1") & 1 else 1.0)
        out[8 * _group(l): 8 * _group(l) + 8] = L[l] * nu
    return out


def test_lane_groups_are_a_permutation_with_one_pattern_distances():
    assert sorted(_group(l) for l in range(16)) == list(range(16))
    # the partner of each step holds the group that differs in exactly the step's bit
    for bit, dist in ((0, 1), (1, 2), (2, 7), (3, 8)):
        for l in range(16):
            assert _group(l ^ dist) == _group(l) ^ (1 << bit)


def test_lane_fwht_matches_the_plain_butterflies_bit_for_bit():
    rng = np.random.default_rng(0)
    for _ in range(200):
        x = (rng.standard_normal(128) * np.exp(rng.uniform(-20, 20, 128))).astype(np.float32)
        assert np.array_equal(_plain(x).view(np.uint32), _lanes(x).view(np.uint32))
    # planted mistakes are caught: the sign not folded, or the plain distance 4 for bit 2 without the lane groups
    x = rng.standard_normal(128).astype(np.float32)
    assert not np.array_equal(_plain(x), _lanes(x, fold=False))
    assert not np.array_equal(_plain(x), _lanes(x, dists=((0, 1), (1, 2), (2, 4), (3, 8))))
