"""Shared test helpers: the oracle's view of a synthetic layer and the comparison bars."""
from __future__ import annotations

import numpy as np

import oracle as orc
from ea_exl3.synth import HostLayer


def oracle_routed(host: HostLayer) -> orc.Routed:
    """The oracle's Routed over the host layer; experts that were not generated point at a zero placeholder the
    oracle never reads (it only touches picked experts)."""
    mats = []
    for m in range(3):
        real = [t for t in host.trellis[m] if t is not None]
        ph = np.zeros_like(real[0])
        mats.append([t if t is not None else ph for t in host.trellis[m]])
    return orc.Routed(mats, host.k2, host.suh_g, host.suh_u, host.svh_g, host.svh_u, host.suh_d, host.svh_d,
                      host.dims, host.width, host.cb)


def rms(a) -> float:
    a = np.asarray(a, dtype=np.float64)
    return float(np.sqrt(np.mean(a * a)))


def assert_close_rms(got, want, frac: float, what: str = "") -> float:
    """max |got - want| <= frac * RMS(want): the north star's bar for layer outputs is frac = 2e-3."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    r = rms(want)
    err = float(np.max(np.abs(got - want))) if got.size else 0.0
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert err <= frac * r, f"{what}: max|diff| {err:.3e} > {frac} * RMS {r:.3e} (ratio {err / max(r, 1e-30):.2e})"
    return err / max(r, 1e-30)


def h2f(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)
