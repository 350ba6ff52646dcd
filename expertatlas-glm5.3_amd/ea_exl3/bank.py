"""Expert banks over the C ABI, mirroring weights.Reader (weights.zig:20-240), moe.load / loadFrom (moe.zig:57-151)
and expert_swap.swapLayer (expert_swap.zig:345-467), plus writers of the two on-disk forms a rank reads:

  - a checkpoint of whole matrices (ExLlamaV3's per-layer files: "model.layers.L.mlp.experts.e.P_proj.{trellis, suh,
    svh, mcg | mul1}", trellis i16 [K/16, N/16, 8 K2]) with its model.safetensors.index.json;
  - a bank: "experts-layer-LLL.safetensors" with every projection pre-sharded for `world` tensor-parallel ranks
    ("...P_proj.rank{r}.S": gate / up trellis cut on the tile columns and svh on its rows, down trellis and suh on
    the rows; markers and the other scale whole), the layout assemble.py:173-237 (reslice_layer) writes.

The writers make fixtures from this package's synthetic trellis and scales; real banks come from the reference's own
converter and read the same way."""
from __future__ import annotations

import ctypes as C
import json
import os

import numpy as np

from ._lib import Routed as _Routed, ShareInfo, SwapStats, check, lib

DTYPES = ["BOOL", "U8", "I8", "U16", "I16", "F16", "BF16", "U32", "I32", "F32", "U64", "I64", "F64"]
NP = {"BOOL": np.bool_, "U8": np.uint8, "I8": np.int8, "U16": np.uint16, "I16": np.int16, "F16": np.float16,
      "BF16": np.uint16, "U32": np.uint32, "I32": np.int32, "F32": np.float32, "U64": np.uint64, "I64": np.int64,
      "F64": np.float64}
PROJ = ("gate", "up", "down")


def expert_name(layer: int, e: int, proj: str, part: str) -> str:
    return f"model.layers.{layer}.mlp.experts.{e}.{proj}_proj.{part}"


def bank_file(layer: int) -> str:
    """The file a width's bank holds a layer in (expert_swap.zig:304)."""
    return f"experts-layer-{layer:03d}.safetensors"


class Reader:
    """weights.Reader: the directory's index (model.safetensors.index.json), or one file of it (fname), read for rank
    `rank` of `world`; pre-sharded tensors of `stored_world` stored ranks are joined."""

    def __init__(self, directory: str, rank: int = 0, world: int = 1, stored_world: int = 1, fname: str | None = None):
        h = C.c_void_p()
        if fname is None:
            check(lib().ea_bank_open(directory.encode(), rank, world, stored_world, C.byref(h)), "Reader.open")
        else:
            check(lib().ea_bank_open_file(directory.encode(), fname.encode(), rank, world, stored_world, C.byref(h)),
                  "Reader.openFile")
        self.h = h
        self.rank, self.world, self.stored_world = rank, world, stored_world

    def has(self, name: str) -> bool:
        return bool(lib().ea_bank_has(self.h, name.encode()))

    def get(self, name: str) -> np.ndarray:
        """This rank's share of `name` (Reader.get)."""
        info = ShareInfo()
        check(lib().ea_bank_share(self.h, name.encode(), C.byref(info), None, 0), f"Reader.get {name}")
        shape = tuple(int(info.shape[i]) for i in range(info.rank))
        out = np.empty(shape, dtype=NP[DTYPES[info.dtype]])
        assert out.nbytes == info.bytes
        check(lib().ea_bank_share(self.h, name.encode(), C.byref(info), out.ctypes.data_as(C.c_void_p), out.nbytes),
              f"Reader.get {name}")
        return out

    def close(self) -> None:
        if self.h:
            lib().ea_bank_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Layer:
    """moe.Routed loaded from banks (moe.loadFrom): the layer owns its device slabs, tables and scales; `c` is the
    ea_routed the kernels read (it follows a swap)."""

    def __init__(self, readers, layer: int, experts: int, pick=None):
        rs = readers if isinstance(readers, (list, tuple)) else [readers]
        arr = (C.c_void_p * len(rs))(*[r.h for r in rs])
        pk = None if pick is None else np.ascontiguousarray(pick, dtype=np.uint8)
        h = C.c_void_p()
        check(lib().ea_layer_load(arr, len(rs), None if pk is None else pk.ctypes.data_as(C.c_void_p), layer, experts,
                                  C.byref(h)), "moe.load")
        self.h, self.layer, self.experts = h, layer, experts
        self._readers = rs
        self.c = lib().ea_layer_routed(h).contents

    def swap(self, banks: dict, target, current) -> SwapStats:
        """expert_swap.swapLayer: experts whose target width differs from the current one are read from the bank of
        their target width (banks: bits -> Reader), the tables rewritten in place."""
        arr = (C.c_void_p * 9)(*[(banks[b].h if b in banks else None) for b in range(9)])
        t = np.ascontiguousarray(target, dtype=np.uint8)
        c = np.ascontiguousarray(current, dtype=np.uint8)
        st = SwapStats()
        check(lib().ea_layer_swap(self.h, arr, self.layer, t.ctypes.data_as(C.c_void_p), c.ctypes.data_as(C.c_void_p),
                                  C.byref(st)), "swapLayer")
        return st

    def free(self) -> None:
        if self.h:
            lib().ea_layer_free(self.h)
            self.h = None
            self.c = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ---- writers --------------------------------------------------------------------------------------------------------

def _save(path: str, tensors: dict, metadata: dict | None = None) -> None:
    """A safetensors file in name order (8-byte header length, JSON header, data)."""
    header, blobs, off = {}, [], 0
    for name in sorted(tensors):
        dtype, a = tensors[name]
        b = np.ascontiguousarray(a).tobytes()
        header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    if metadata:
        header["__metadata__"] = metadata
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path + ".part", "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for b in blobs:
            f.write(b)
    os.replace(path + ".part", path)


def write_index(directory: str, files: dict) -> None:
    """model.safetensors.index.json for {file name: [tensor names]}."""
    wm = {n: f for f, names in files.items() for n in names}
    with open(os.path.join(directory, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": dict(sorted(wm.items()))}, f)


def layer_tensors(layer: int, trellis, suh, svh, cb: int = 1) -> dict:
    """The whole-matrix tensors of one layer's routed experts: trellis[p][e] u32 words of expert layout [K, N] (tile
    (kt, nt) at ((kt N/16) + nt) 4 K2 words), suh[p][e] / svh[p][e] fp16 bits; p = gate, up, down."""
    out = {}
    marker = {1: "mcg", 2: "mul1"}.get(cb)
    for p, proj in enumerate(PROJ):
        for e, T in enumerate(trellis[p]):
            K, N = len(suh[p][e]), len(svh[p][e])
            words = np.ascontiguousarray(T, dtype=np.uint32)
            tw2 = words.size * 2 // ((K // 16) * (N // 16))
            out[expert_name(layer, e, proj, "trellis")] = ("I16", words.view(np.int16).reshape(K // 16, N // 16, tw2))
            out[expert_name(layer, e, proj, "suh")] = ("F16", np.asarray(suh[p][e], np.uint16))
            out[expert_name(layer, e, proj, "svh")] = ("F16", np.asarray(svh[p][e], np.uint16))
            if marker:
                out[expert_name(layer, e, proj, marker)] = ("I16", np.zeros(1, np.int16))
    return out


def write_checkpoint_layer(directory: str, layer: int, trellis, suh, svh, cb: int = 1) -> str:
    """One layer of whole matrices as model.layers.L.safetensors, and the directory's index over every such file."""
    os.makedirs(directory, exist_ok=True)
    fname = f"model.layers.{layer}.safetensors"
    t = layer_tensors(layer, trellis, suh, svh, cb)
    _save(os.path.join(directory, fname), t, {"format": "pt"})
    files = {}
    for f in sorted(os.listdir(directory)):
        if f.endswith(".safetensors"):
            files[f] = list(_header_names(os.path.join(directory, f)))
    write_index(directory, files)
    return fname


def _header_names(path: str):
    with open(path, "rb") as f:
        n = int.from_bytes(f.read(8), "little")
        h = json.loads(f.read(n))
    return [k for k in h if k != "__metadata__"]


def _share(a: np.ndarray, rule: str, r: int, world: int) -> np.ndarray:
    if rule == "rep":
        return a
    axis = 0 if rule == "row" else 1
    n = a.shape[axis] // world
    return a[r * n:(r + 1) * n] if axis == 0 else a[:, r * n:(r + 1) * n]


def reslice_layer(tensors: dict, layer: int, directory: str, world: int) -> str:
    """A bank file (experts-layer-LLL.safetensors) of one layer for `world` ranks from its whole-matrix tensors (the
    output of layer_tensors): every projection's parts as "...P_proj.rank{r}.S"."""
    os.makedirs(directory, exist_ok=True)
    out = {}
    for name, (dtype, a) in tensors.items():
        stem, part = name.rsplit(".", 1)
        down = stem.endswith("down_proj")
        if part == "trellis":
            rule = "row" if down else "dim1"
        elif part in ("suh", "svh"):
            rule = "row" if (part == "suh") == down else "rep"
        else:
            rule = "rep"
        for r in range(world):
            out[f"{stem}.rank{r}.{part}"] = (dtype, np.ascontiguousarray(_share(a, rule, r, world)))
    fname = bank_file(layer)
    _save(os.path.join(directory, fname), out,
          {"format": "pt", "reshard": f"whole matrices -> tp{world} (tile re-slice, no requantization)"})
    return fname
