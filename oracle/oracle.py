"""ctypes wrapper of the CPU oracle (oracle/exl3_oracle.c): TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, as the checker or the
CPU baseline. Every array is numpy; fp16 and bf16 travel as uint16 bit patterns.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

P = C.c_void_p
I = C.c_int
I64 = C.c_int64
F = C.c_float


def build() -> None:
    subprocess.check_call(["make", "-s", "-C", _HERE])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L):
    sig = {
        "or_h2f": (F, [C.c_uint16]),
        "or_f2h": (C.c_uint16, [F]),
        "or_d2h": (C.c_uint16, [C.c_double]),
        "or_bf2f": (F, [C.c_uint16]),
        "or_f2bf": (C.c_uint16, [F]),
        "or_expf": (F, [F]),
        "or_stream_end": (I, [I, I]),
        "or_state": (C.c_uint32, [P, I, I]),
        "or_tile_states": (None, [P, I, P]),
        "or_cb_value": (C.c_uint16, [I, C.c_uint32]),
        "or_codebook_lut": (None, [I, P]),
        "or_value_row": (I, [I]),
        "or_value_col": (I, [I]),
        "or_decode_tile": (None, [P, I, I, P]),
        "or_dequant_expert": (None, [P, I, I, I, I, P]),
        "or_unpack": (None, [P, I, I, I, I, I64, I64, P]),
        "or_expert_to_strips": (None, [P, I, I, I, P]),
        "or_fwht128": (None, [P]),
        "or_group": (None, [P, I, I, I, I, P, P, P]),
        "or_rot_in": (None, [P, I, I, P, P, P, P, P, I, I, I, I]),
        "or_gateup_epilogue": (None, [P, P, P, P, P, P, I, I, I, I, I, I, F, I]),
        "or_down_combine": (None, [P, P, P, P, P, P, I, I, I, I, I, I]),
        "or_moe_routed": (None, [P, I, I, P, P, P, I, I, P, P]),
        "or_route": (I, [P, I, I, I, I, P, P, P]),
        "or_prompt_experts": (None, [P, I, I, P, P, P, I, I, I, P]),
        "or_linear_plan": (None, [I, I, P, P]),
        "or_exl3_rot_in": (None, [P, I, P, P, I, I]),
        "or_exl3_linear": (None, [P, P, I64, I64, P, P, P, I, I, I, I, I, I, I, I]),
        "or_router": (None, [P, I, I, P, I, I, I, P, P]),
        "or_topk8": (None, [P, P, I, I, F, P, P]),
        "or_swiglu2": (None, [P, P, P, I]),
        "or_mix64": (C.c_uint64, [C.c_uint64]),
        "or_fill_words": (None, [C.c_uint64, P, C.c_size_t]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data


DT = {np.dtype(np.float16): 0, "bf16": 1, np.dtype(np.float32): 2}


def _x_dtype(x: np.ndarray, bf16: bool) -> int:
    if bf16:
        assert x.dtype == np.uint16
        return 1
    if x.dtype == np.float32:
        return 2
    assert x.dtype in (np.float16, np.uint16)
    return 0


# ---- scalar helpers -------------------------------------------------------------------------------------------

def f2h(f: float) -> int:
    return lib().or_f2h(f)


def d2h(d: float) -> int:
    return lib().or_d2h(d)


def expf(x: float) -> float:
    return lib().or_expf(x)


def stream_end(k2: int, p: int) -> int:
    return lib().or_stream_end(k2, p)


def tile_states(tile: np.ndarray, k2: int) -> np.ndarray:
    tile = np.ascontiguousarray(tile, dtype=np.uint32)
    out = np.zeros(256, np.uint16)
    lib().or_tile_states(_p(tile), k2, _p(out))
    return out


def codebook_lut(cb: int) -> np.ndarray:
    out = np.zeros(65536, np.uint16)
    lib().or_codebook_lut(cb, _p(out))
    return out


def decode_tile(tile: np.ndarray, k2: int, cb: int) -> np.ndarray:
    tile = np.ascontiguousarray(tile, dtype=np.uint32)
    out = np.zeros((16, 16), np.uint16)
    lib().or_decode_tile(_p(tile), k2, cb, _p(out))
    return out


def dequant_expert(T: np.ndarray, K: int, N: int, k2: int, cb: int) -> np.ndarray:
    T = np.ascontiguousarray(T, dtype=np.uint32)
    assert T.size == (K // 16) * (N // 16) * 4 * k2
    W = np.zeros((K, N), np.uint16)
    lib().or_dequant_expert(_p(T), K, N, k2, cb, _p(W))
    return W


def unpack(T: np.ndarray, K: int, N: int, k2: int, cb: int, stride_k: int, stride_nb: int) -> np.ndarray:
    T = np.ascontiguousarray(T, dtype=np.uint32)
    W = np.zeros((K, N), np.uint16)
    lib().or_unpack(_p(T), K, N, k2, cb, stride_k, stride_nb, _p(W))
    return W


def expert_to_strips(T: np.ndarray, K: int, N: int, k2: int) -> np.ndarray:
    T = np.ascontiguousarray(T, dtype=np.uint32)
    S = np.zeros_like(T)
    lib().or_expert_to_strips(_p(T), K, N, k2, _p(S))
    return S


def fwht128(v: np.ndarray) -> np.ndarray:
    v = np.array(v, dtype=np.float32, copy=True)
    lib().or_fwht128(_p(v))
    return v


# ---- routed experts ------------------------------------------------------------------------------------------

def group(pick: np.ndarray, R: int, slots: int, E: int, maxm: int):
    pick = np.ascontiguousarray(pick, dtype=np.int32)
    maxu = min(R * slots, E)
    uids = np.zeros(maxu, np.int32)
    ucount = np.zeros(1, np.int32)
    members = np.full((maxu, maxm), -1, np.int32)
    lib().or_group(_p(pick), R, slots, E, maxm, _p(uids), _p(ucount), _p(members))
    return uids, int(ucount[0]), members


def rot_in(x, pick, suh0, suh1, rows, K, slots, E, x_stride=None, bf16=False):
    x = np.ascontiguousarray(x)
    pick = np.ascontiguousarray(pick, dtype=np.int32)
    out0 = np.zeros((rows * slots, K), np.uint16)
    out1 = np.zeros((rows * slots, K), np.uint16)
    lib().or_rot_in(_p(x), _x_dtype(x, bf16), x_stride or K, _p(pick), _p(suh0), _p(suh1), _p(out0), _p(out1),
                    rows, K, slots, E)
    return out0, out1


class Routed:
    """One layer's routed experts on the host, laid out as moe.zig's Routed (moe.zig:19-37): per matrix (gate, up,
    down) one trellis array per expert, a K2 per expert, and stacked suh / svh [E, width] fp16 bits."""

    def __init__(self, trellis, k2, suh_g, suh_u, svh_g, svh_u, suh_d, svh_d, dims, width, cb=1):
        self.trellis = [[np.ascontiguousarray(t, dtype=np.uint32) for t in m] for m in trellis]
        self.k2 = [np.ascontiguousarray(k, dtype=np.int32) for k in k2]
        self.suh_g, self.suh_u, self.svh_g, self.svh_u, self.suh_d, self.svh_d = (
            np.ascontiguousarray(a, dtype=np.uint16) for a in (suh_g, suh_u, svh_g, svh_u, suh_d, svh_d))
        self.count = len(self.trellis[0])
        self.dims, self.width, self.cb = dims, width, cb
        self._ptr_arrays = [(C.c_void_p * self.count)(*[t.ctypes.data for t in m]) for m in self.trellis]

        class _S(C.Structure):
            _fields_ = [("ptr", C.c_void_p * 3), ("k2", C.c_void_p * 3), ("suh_g", P), ("suh_u", P), ("svh_g", P),
                        ("svh_u", P), ("suh_d", P), ("svh_d", P), ("count", I), ("dims", I), ("width", I),
                        ("cb", I)]

        s = _S()
        for i in range(3):
            s.ptr[i] = C.cast(self._ptr_arrays[i], C.c_void_p)
            s.k2[i] = self.k2[i].ctypes.data
        s.suh_g, s.suh_u, s.svh_g, s.svh_u, s.suh_d, s.svh_d = (
            a.ctypes.data for a in (self.suh_g, self.suh_u, self.svh_g, self.svh_u, self.suh_d, self.svh_d))
        s.count, s.dims, s.width, s.cb = self.count, dims, width, cb
        self._s = s

    def ref(self):
        return C.byref(self._s)

    def ptr_table(self, mat):
        return self._ptr_arrays[mat]


def grouped(x0, x1, routed: Routed, mats_idx, uids, ucount, members, K, N, P_, SK, slots, warps=4, z=None):
    """or_grouped over routed's matrices mats_idx = (gate, up) or (down,)."""

    class _A(C.Structure):
        _fields_ = [("x0", P), ("x1", P), ("tp0", P), ("tp1", P), ("k2_0", P), ("k2_1", P), ("uids", P),
                    ("ucount", P), ("members", P), ("z", P), ("K", I), ("N", I), ("P", I), ("SK", I), ("maxm", I),
                    ("slots", I), ("nexp_max", I), ("mats", I), ("cb", I), ("warps", I), ("ns", I)]

    mats = len(mats_idx)
    if z is None:
        z = np.zeros((mats, SK, P_, N), np.float32)
    uc = np.array([ucount], np.int32)
    a = _A()
    a.x0, a.x1 = x0.ctypes.data, x1.ctypes.data
    a.tp0 = C.cast(routed.ptr_table(mats_idx[0]), C.c_void_p)
    a.tp1 = C.cast(routed.ptr_table(mats_idx[-1]), C.c_void_p)
    a.k2_0, a.k2_1 = routed.k2[mats_idx[0]].ctypes.data, routed.k2[mats_idx[-1]].ctypes.data
    a.uids, a.ucount, a.members, a.z = uids.ctypes.data, uc.ctypes.data, members.ctypes.data, z.ctypes.data
    a.K, a.N, a.P, a.SK, a.maxm, a.slots = K, N, P_, SK, members.shape[1], slots
    a.nexp_max, a.mats, a.cb, a.warps, a.ns = uids.shape[0], mats, routed.cb, warps, 0
    fn = lib().or_grouped
    fn.restype = None
    fn.argtypes = [C.c_void_p]
    fn(C.addressof(a))
    return z


def gateup_epilogue(Z, pick, routed: Routed, rows, P_, N, SK, slots, E, limit=float("inf"), act_mode=1):
    xd = np.zeros((P_, N), np.uint16)
    lib().or_gateup_epilogue(_p(Z), _p(pick), _p(routed.svh_g), _p(routed.svh_u), _p(routed.suh_d), _p(xd), rows,
                             P_, N, SK, slots, E, limit, act_mode)
    return xd


def down_combine(Z, pick, routed: Routed, wts, rows, P_, D, SK, slots, E, y=None):
    y = np.zeros((P_, D), np.float32) if y is None else y
    out = np.zeros((rows, D), np.float32)
    lib().or_down_combine(_p(Z), _p(pick), _p(routed.svh_d), _p(y), _p(wts), _p(out), rows, P_, D, SK, slots, E)
    return y, out


def moe_routed(x, pick, wts, routed: Routed, R, slots, x_stride=None, bf16=False, y=None):
    x = np.ascontiguousarray(x)
    pick = np.ascontiguousarray(pick, dtype=np.int32)
    wts = np.ascontiguousarray(wts, dtype=np.float32)
    y = np.zeros((R * slots, routed.dims), np.float32) if y is None else y
    out = np.zeros((R, routed.dims), np.float32)
    lib().or_moe_routed(_p(x), _x_dtype(x, bf16), x_stride or routed.dims, _p(pick), _p(wts), routed.ref(), R, slots,
                        _p(y), _p(out))
    return out


_cpu = None


def _cpu_lib():
    global _cpu
    if _cpu is None:
        L = C.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), "libcpulayer.so"))
        L.cpu_moe_routed.restype = None
        L.cpu_moe_routed.argtypes = [P, I, I, P, P, P, I, I, P]
        L.cpu_exl3_linear.restype = None
        L.cpu_exl3_linear.argtypes = [P, I, P, P, I64, I64, P, P, I, I, I, I, I]
        _cpu = L
    return _cpu


def cpu_moe_routed(x, pick, wts, routed: Routed, R, slots, x_stride=None, bf16=False):
    """The tuned CPU baseline (libcpulayer.so, cpu_layer.c) of moe_routed: the same function, decoded straight into
    the products, OpenMP over column tiles; fp32 sums in a different order than the oracle's."""
    _cpu_lib()
    x = np.ascontiguousarray(x)
    out = np.zeros((R, routed.dims), np.float32)
    _cpu.cpu_moe_routed(_p(x), _x_dtype(x, bf16), x_stride or routed.dims, _p(np.ascontiguousarray(pick, np.int32)),
                        _p(np.ascontiguousarray(wts, np.float32)), routed.ref(), R, slots, _p(out))
    return out


def route(pick, n, E, ipm, max_items):
    pick = np.ascontiguousarray(pick, dtype=np.int32)
    sorted_ = np.zeros(max(n, 1), np.int32)
    items = np.zeros(3 * max(max_items, 1), np.int32)
    ic = np.zeros(1, np.int32)
    lib().or_route(_p(pick), n, E, ipm, max_items, _p(sorted_), _p(items), _p(ic))
    return sorted_[:n], items.reshape(-1, 3), int(ic[0])


def prompt_experts(x, pick, wts, routed: Routed, R, slots, do_round=False, x_stride=None, bf16=False):
    x = np.ascontiguousarray(x)
    out = np.zeros((R, routed.dims), np.float32)
    lib().or_prompt_experts(_p(x), _x_dtype(x, bf16), x_stride or routed.dims,
                            _p(np.ascontiguousarray(pick, dtype=np.int32)),
                            _p(np.ascontiguousarray(wts, dtype=np.float32)), routed.ref(), R, slots, int(do_round),
                            _p(out))
    return out


# ---- EXL3 linear ---------------------------------------------------------------------------------------------

def linear_plan(k: int, n: int):
    sk, wk = C.c_int(), C.c_int()
    lib().or_linear_plan(k, n, C.byref(sk), C.byref(wk))
    return sk.value, wk.value


def cpu_exl3_linear(x, suh, T_strips, svh, M, K, N, k2, cb, bf16=False):
    """The tuned CPU baseline (libcpulayer.so, cpu_layer.c) of exl3_rot_in then exl3_linear with fp32 out: the same
    function on words in the strips layout, OpenMP over column tiles; fp32 sums in a different order than the
    oracle's."""
    _cpu_lib()
    x = np.ascontiguousarray(x)
    y = np.zeros((M, N), np.float32)
    tw = 4 * k2
    _cpu.cpu_exl3_linear(_p(x), _x_dtype(x, bf16), _p(np.ascontiguousarray(suh, dtype=np.uint16)),
                         _p(np.ascontiguousarray(T_strips, dtype=np.uint32)), 8 * tw, (K // 16) * 8 * tw,
                         _p(np.ascontiguousarray(svh, dtype=np.uint16)), _p(y), M, K, N, k2, cb)
    return y


def exl3_rot_in(x, suh, M, K, bf16=False):
    x = np.ascontiguousarray(x)
    xh = np.zeros((M, K), np.uint16)
    lib().or_exl3_rot_in(_p(x), _x_dtype(x, bf16), _p(np.ascontiguousarray(suh, dtype=np.uint16)), _p(xh), M, K)
    return xh


def exl3_linear(xh, T, stride_k, stride_nb, svh, M, K, N, k2, cb, SK, WK, bias=None, y_dtype=2):
    y = np.zeros((M, N), np.float32 if y_dtype == 2 else np.uint16)
    lib().or_exl3_linear(_p(xh), _p(np.ascontiguousarray(T, dtype=np.uint32)), stride_k, stride_nb, _p(svh),
                         _p(bias), _p(y), y_dtype, M, K, N, k2, cb, SK, WK)
    return y


# ---- router and shared expert ----------------------------------------------------------------------------------

def router(x, w, x_dtype=1, with_part=False):
    """logits f32 [m, ne] of x 16-bit [m, d] (x_dtype 0 fp16, 1 bf16) by w bf16 [ne, d]; with the slice sums
    [8, m, ne] too when with_part."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    m, d = x.shape
    ne = w.shape[0]
    out = np.zeros((m, ne), np.float32)
    part = np.zeros((8, m, ne), np.float32) if with_part else None
    lib().or_router(_p(x), x_dtype, d, _p(w), m, d, ne, _p(part), _p(out))
    return (out, part) if with_part else out


def topk8(logits, bias, scale=2.5):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    rows, E = logits.shape
    pick = np.zeros((rows, 8), np.int32)
    wts = np.zeros((rows, 8), np.float32)
    lib().or_topk8(_p(logits), _p(np.ascontiguousarray(bias, dtype=np.float32)), rows, E, scale, _p(pick), _p(wts))
    return pick, wts


def swiglu2(g, u):
    g = np.ascontiguousarray(g, dtype=np.uint16)
    out = np.zeros_like(g)
    lib().or_swiglu2(_p(g), _p(np.ascontiguousarray(u, dtype=np.uint16)), _p(out), g.size)
    return out


def fill_words(seed: int, n: int) -> np.ndarray:
    w = np.zeros(n, np.uint32)
    lib().or_fill_words(seed, _p(w), n)
    return w
