#!/usr/bin/env python3
"""Per-block timelines of the config-2 decode layer (`layer1_kernel`) and the config-1 EXL3 linear
(`lin_small_kernel`, tagged form) from the timeline build's stage stamps.

    python expertatlas-glm5.3_amd/build.py --stamps        # libea_exl3_stamps.so beside the product library
    python expertatlas-glm5.3_amd/timeline.py [--layers 11] [--runs 5] [--json out.json]

The timeline build is the product source compiled with EA_STAMPS (csrc/ea_stamps.hpp): at marked points a block's
marking thread stores the 100 MHz constant clock into a region attached here. This script loads that build (through
EA_EXL3_LIB, before the package is imported), sets up the same workloads as `bench.py --config decode` / `--config
linear` (eight resident layers or linears, fresh router logits every layer), launches `--layers` of them back to back
with the region attached, and reads the stamps the last launch left. Times are µs from the launch's first block start;
a cell is min–max (median) over the blocks of that kind, each figure the median over `--runs` runs.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
STAMPS_LIB = os.path.join(HERE, "ea_exl3", "libea_exl3_stamps.so")
POINTS = 16         # stamps a block (csrc/ea_stamps.hpp: STAMP_POINTS); the last is the block's descriptor
MAX_BLOCKS = 8192   # the region's blocks (the config-2 layer launches 1,297, the config-1 linear 256)
TICKS_PER_US = 100.0


def _cell(vals: list[float]) -> tuple[float, float, float] | None:
    import numpy as np

    if not vals:
        return None
    a = np.asarray(vals)
    return float(a.min()), float(np.median(a)), float(a.max())


def _fmt(c) -> str:
    return "—" if c is None else f"{c[0]:.2f}–{c[2]:.2f} ({c[1]:.2f})"


def _median_cells(runs: list[dict]) -> dict:
    """Each (row, column) cell's min, median and max as the median over the runs."""
    import numpy as np

    out = {}
    for key in runs[0]:
        cs = [r[key] for r in runs if r.get(key) is not None]
        out[key] = None if not cs else tuple(float(np.median([c[i] for c in cs])) for i in range(3))
    return out


def layer_stats(st) -> dict:
    """Cells of one launch's stamps ([blocks, POINTS] int64) of layer1_kernel: (stage, kind) -> (min, median, max)."""
    import numpy as np

    used = st[:, 0] != 0
    st = st[used]
    t0 = st[:, 0].min()
    us = lambda v: (float(v) - float(t0)) / TICKS_PER_US
    desc = st[:, POINTS - 1]
    kind = desc & 0xff
    unit = (desc >> 8) & 0xff
    cells: dict = {}

    def put(stage: str, col: str, rows, point: int):
        vals = [us(v) for v in st[rows, point] if v != 0]
        cells[(stage, col)] = _cell(vals)

    router, shared_gu, routed_gu = kind == 1, kind == 2, kind == 3
    down, comb = kind == 4, kind == 5
    epi = (kind >= 2) & (kind <= 3) & (st[:, 3] != 0)
    for col, rows in (("router", router), ("shared gate|up", shared_gu), ("routed gate|up", routed_gu),
                      ("down", down), ("combiners", comb)):
        put("blocks start", col, rows, 0)
    put("routed", "router", router, 1)
    put("routed", "routed gate|up", routed_gu, 1)
    put("routed", "down", down, 1)
    put("routed", "combiners", comb, 1)
    put("activations rotated, trellis landed", "shared gate|up", shared_gu, 5)
    put("activations rotated, trellis landed", "routed gate|up", routed_gu, 5)
    put("tiles decoded and multiplied", "shared gate|up", shared_gu, 6)
    put("tiles decoded and multiplied", "routed gate|up", routed_gu, 6)
    put("partial sums / outputs stored", "shared gate|up", shared_gu, 2)
    put("partial sums / outputs stored", "routed gate|up", routed_gu, 2)
    put("partial sums / outputs stored", "down", down, 5)
    put("epilogue polls done", "shared gate|up", epi & shared_gu, 3)
    put("epilogue polls done", "routed gate|up", epi & routed_gu, 3)
    put("epilogue stored", "shared gate|up", epi & shared_gu, 4)
    put("epilogue stored", "routed gate|up", epi & routed_gu, 4)
    put("down pre-decode done", "down", down, 2)
    put("down pre-decode done", "combiners", comb, 2)
    put("down inputs seen", "down", down, 3)
    put("down inputs seen", "combiners", comb, 3)
    put("down MFMAs done", "down", down, 4)
    put("down MFMAs done", "combiners", comb, 4)
    put("other units' outputs seen", "combiners", comb, 5)
    put("combine done", "combiners", comb, 6)
    # the routed gate|up items by pick (unit 1 + k with the shared expert as unit 0)
    hs = bool(shared_gu.any())
    for k in range(8):
        rows = routed_gu & (unit == k + (1 if hs else 0))
        put(f"pick {k}: routed", "routed gate|up", rows, 1)
        put(f"pick {k}: sums stored", "routed gate|up", rows, 2)
        put(f"pick {k}: epilogue stored", "routed gate|up", rows & epi, 4)
    return cells


def linear_stats(st) -> dict:
    """Cells of one launch's stamps of lin_small_kernel (tagged form): (stage, kind) -> (min, median, max)."""
    used = st[:, 0] != 0
    st = st[used]
    t0 = st[:, 0].min()
    us = lambda v: (float(v) - float(t0)) / TICKS_PER_US
    kind = st[:, POINTS - 1] & 0xff
    cells: dict = {}
    for col, rows in (("writers", kind == 1), ("finishers", kind == 2)):
        for stage, p in (("blocks start", 0), ("trellis landed (wave 0)", 1), ("tiles decoded (wave 0)", 2),
                         ("activations in LDS, every wave's tiles decoded", 3), ("rotated", 4), ("MFMAs done", 5),
                         ("sums stored (finisher: kept)", 6), ("polls done", 7), ("finished", 8)):
            cells[(stage, col)] = _cell([us(v) for v in st[rows, p] if v != 0])
    return cells


def table(cells: dict, cols: list[str]) -> str:
    stages = []
    for (s, _c) in cells:
        if s not in stages:
            stages.append(s)
    lines = ["| stage | " + " | ".join(cols) + " |", "|---|" + "---|" * len(cols)]
    for s in stages:
        row = [_fmt(cells.get((s, c))) for c in cols]
        if all(r == "—" for r in row):
            continue
        lines.append(f"| {s} | " + " | ".join(row) + " |")
    return "\n".join(lines)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--layers", type=int, default=11, help="launches back to back a run; the last one is read")
    ap.add_argument("--runs", type=int, default=5)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--json", default=None, help="also write the cells here")
    args = ap.parse_args()
    if not os.path.exists(STAMPS_LIB):
        sys.exit(f"{STAMPS_LIB} is missing: build it with `python expertatlas-glm5.3_amd/build.py --stamps`")
    os.environ["EA_EXL3_LIB"] = STAMPS_LIB
    sys.path.insert(0, ROOT)
    sys.path.insert(0, HERE)
    import torch

    import bench
    from ea_exl3 import device, linear
    from ea_exl3._lib import Linear as _Linear, check, lib
    from ea_exl3.resident import DeviceLinear

    device.init(0)
    L = lib()
    for name in ("ea_stamps_attach_layer", "ea_stamps_attach_linear"):
        getattr(L, name).argtypes = [C.c_void_p]
        getattr(L, name).restype = C.c_int
    region = torch.zeros((MAX_BLOCKS, POINTS), dtype=torch.int64, device="cuda")
    result = {}

    # the config-2 layer
    db = bench.DecodeBench(1, 8, 1, False, args.seed, args.layers * args.runs + 1, "fused")
    db.launch(0)  # first use outside the stamped runs
    torch.cuda.synchronize()
    runs = []
    check(L.ea_stamps_attach_layer(region.data_ptr()), "stamps_attach_layer")
    for r in range(args.runs):
        region.zero_()
        torch.cuda.synchronize()
        for j in range(args.layers):
            db.launch(1 + r * args.layers + j)
        torch.cuda.synchronize()
        runs.append(layer_stats(region.cpu().numpy()))
        print(f"layer run {r} done", flush=True)
    check(L.ea_stamps_attach_layer(None), "stamps_attach_layer")
    check(device.device_status(), "device status after the layer runs")
    cells = _median_cells(runs)
    cols = ["router", "shared gate|up", "routed gate|up", "down", "combiners"]
    print("\nConfig-2 layer (layer1_kernel), µs from the first block's start, min–max (median):\n")
    print(table({k: v for k, v in cells.items() if not k[0].startswith("pick")}, cols))
    print("\nRouted gate|up items by pick, µs, min–max (median):\n")
    print(table({k: v for k, v in cells.items() if k[0].startswith("pick")}, ["routed gate|up"]))
    result["layer"] = {f"{s} / {c}": v for (s, c), v in cells.items()}
    del db
    torch.cuda.empty_cache()

    # the config-1 linear
    K, N = 6144, 2048
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed)
    lins = [DeviceLinear(gen, K, N, 8, 1) for _ in range(8)]
    x = torch.randn((1, K), device="cuda", generator=gen).to(torch.float16)
    y = torch.zeros((1, N), dtype=torch.float32, device="cuda")
    sc = linear.Scratch(1, K, lins[0].sk * N)
    s = device.stream()
    arrs = [(C.POINTER(_Linear) * 1)(C.pointer(l.c)) for l in lins]
    outs = (C.c_uint64 * 1)(y.data_ptr())
    dts = (C.c_int * 1)(2)

    def call(i):
        check(L.ea_linear_call(s, C.byref(sc.c), arrs[i % len(arrs)], 1, x.data_ptr(), 0, 1, outs, dts),
              "linear.call")

    call(0)
    torch.cuda.synchronize()
    runs = []
    check(L.ea_stamps_attach_linear(region.data_ptr()), "stamps_attach_linear")
    for r in range(args.runs):
        region.zero_()
        torch.cuda.synchronize()
        for j in range(args.layers):
            call(1 + j)
        torch.cuda.synchronize()
        runs.append(linear_stats(region.cpu().numpy()))
        print(f"linear run {r} done", flush=True)
    check(L.ea_stamps_attach_linear(None), "stamps_attach_linear")
    check(device.device_status(), "device status after the linear runs")
    cells = _median_cells(runs)
    print("\nConfig-1 linear (lin_small_kernel, tagged form), µs from the first block's start, min–max (median):\n")
    print(table(cells, ["writers", "finishers"]))
    result["linear"] = {f"{s} / {c}": v for (s, c), v in cells.items()}
    if args.json:
        with open(args.json, "w") as f:
            json.dump(result, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
