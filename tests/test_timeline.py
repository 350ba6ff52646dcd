"""The timeline build's boundary and the stamp reader, without a GPU: the product library exports no stamp entry
point (the marks are compiled out of it), and timeline.py's tables read a synthetic stamp region the way the kernels
lay it out (entry [block * 16 + point], 100 MHz ticks, the block's descriptor in the last point)."""
import os
import sys

import numpy as np

from ea_exl3 import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "expertatlas-glm5.3_amd"))
import timeline  # noqa: E402


def test_product_library_has_no_stamp_entry_points():
    L = _lib.lib()
    assert os.path.basename(_lib.LIB_PATH) == "libea_exl3.so"
    for name in ("ea_stamps_attach_layer", "ea_stamps_attach_linear"):
        assert not hasattr(L, name), name


def _region(rows):
    st = np.zeros((len(rows), timeline.POINTS), np.int64)
    for b, (desc, pts) in enumerate(rows):
        st[b, timeline.POINTS - 1] = desc
        for p, t in pts.items():
            st[b, p] = t
    return st


def test_layer_stats_reads_the_layout():
    base = 10_000_000  # ticks; times below are ticks after it (100 a µs)
    rows = [
        (1, {0: base + 10, 1: base + 380}),                                   # router
        (2 | 0 << 8, {0: base, 5: base + 250, 6: base + 500, 2: base + 600}),  # shared gate|up
        (3 | 1 << 8, {0: base + 20, 1: base + 260, 5: base + 600, 6: base + 900, 2: base + 1000}),  # pick 0
        (3 | 8 << 8 | 1 << 20 | 23 << 24,  # pick 7, the epilogue item of its column block
         {0: base + 30, 1: base + 430, 5: base + 700, 6: base + 1100, 2: base + 1200, 3: base + 1500,
          4: base + 1600}),
        (4 | 2 << 8, {0: base + 40, 1: base + 560, 2: base + 1100, 3: base + 1300, 4: base + 1350, 5: base + 1400}),
        (5 | 8 << 8, {0: base + 50, 1: base + 600, 2: base + 1200, 3: base + 1650, 4: base + 1700, 5: base + 1800,
                      6: base + 1820}),
    ]
    cells = timeline.layer_stats(_region(rows + [(0, {})]))  # an unused block (no start stamp) is ignored
    assert cells[("blocks start", "shared gate|up")] == (0.0, 0.0, 0.0)
    assert cells[("routed", "router")] == (3.8, 3.8, 3.8)
    assert cells[("routed", "routed gate|up")] == (2.6, 3.45, 4.3)
    assert cells[("partial sums / outputs stored", "routed gate|up")] == (10.0, 11.0, 12.0)
    assert cells[("epilogue polls done", "routed gate|up")] == (15.0, 15.0, 15.0)
    assert cells[("epilogue stored", "routed gate|up")] == (16.0, 16.0, 16.0)
    assert cells[("epilogue stored", "shared gate|up")] is None
    assert cells[("pick 7: routed", "routed gate|up")] == (4.3, 4.3, 4.3)
    assert cells[("pick 0: sums stored", "routed gate|up")] == (10.0, 10.0, 10.0)
    assert cells[("down inputs seen", "down")] == (13.0, 13.0, 13.0)
    assert cells[("combine done", "combiners")] == (18.2, 18.2, 18.2)
    md = timeline.table(cells, ["router", "shared gate|up", "routed gate|up", "down", "combiners"])
    assert "| routed | 3.80–3.80 (3.80) | — | 2.60–4.30 (3.45) |" in md


def test_linear_stats_and_run_medians():
    base = 5_000_000
    runs = []
    for shift in (0, 10, 20):  # three runs: each figure of a cell is the median over them
        rows = [(1, {0: base + 5, 1: base + 200 + shift, 6: base + 600 + shift}),
                (2, {0: base, 1: base + 210 + shift, 6: base + 610 + shift, 7: base + 800 + shift,
                     8: base + 850 + shift})]
        runs.append(timeline.linear_stats(_region(rows)))
    cells = timeline._median_cells(runs)
    assert cells[("trellis landed (wave 0)", "writers")] == (2.1, 2.1, 2.1)  # from the earliest start, the finisher's
    assert cells[("polls done", "finishers")] == (8.1, 8.1, 8.1)
    assert cells[("polls done", "writers")] is None
