"""ctypes binding of libea_exl3.so (include/ea_exl3.h). Loading fails loudly when the library is missing: there
is no fallback path. EA_EXL3_LIB names another build of the same library to load instead (for A/B timing)."""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("EA_EXL3_LIB") or os.path.join(_HERE, "libea_exl3.so")

U64, I64, U32, I32, F32, P = C.c_uint64, C.c_int64, C.c_uint32, C.c_int32, C.c_float, C.c_void_p
MAX_JOBS = 3


class EaError(RuntimeError):
    def __init__(self, code: int, where: str):
        self.code = code
        super().__init__(f"{where}: {strerror(code)} (status {code})")


class GroupedArgs(C.Structure):
    _fields_ = [("x0", U64), ("x1", U64), ("tp0", U64), ("tp1", U64), ("k2_0", U64), ("k2_1", U64),
                ("uids", U64), ("ucount", U64), ("members", U64), ("z", U64),
                ("K", U32), ("N", U32), ("P", U32), ("SK", U32), ("maxm", U32), ("slots", U32), ("nexp_max", U32),
                ("mats", U32), ("cb", U32), ("nt", U32), ("warps", U32), ("pf", U32), ("lo", U32), ("hi", U32),
                ("ns", U32)]


class Routed(C.Structure):
    _fields_ = [("ptr", U64 * 3), ("k2", U64 * 3), ("suh_g", U64), ("suh_u", U64), ("svh_g", U64), ("svh_u", U64),
                ("suh_d", U64), ("svh_d", U64), ("count", U32), ("dims", U32), ("width", U32), ("cb", U32),
                ("k2_gu", U32 * 2), ("k2_d", U32 * 2)]


class MoeScratch(C.Structure):
    _fields_ = [("xg", U64), ("xu", U64), ("xd", U64), ("z", U64), ("y", U64), ("ids", U64), ("count", U64),
                ("members", U64), ("sync", U64), ("fused", U64), ("rows", U32), ("slots", U32)]


class PromptScratch(C.Structure):
    _fields_ = [("sorted", U64), ("items", U64), ("count", U64), ("xd", U64), ("plane", U64), ("xg", U64),
                ("xu", U64), ("z", U64), ("zp", U64), ("pclass", U64), ("rows", U32), ("slots", U32),
                ("max_items", U32)]


class Job(C.Structure):
    _fields_ = [("xh", U64), ("T", U64), ("stride_k", I64), ("stride_nb", I64), ("svh", U64), ("bias", U64),
                ("y", U64), ("Z", U64), ("counters", U64), ("y_dtype", I32), ("N", I32), ("SK", I32),
                ("start", I32)]


class Jobs(C.Structure):
    _fields_ = [("j", Job * MAX_JOBS), ("n", I32)]


class RotJobs(C.Structure):
    _fields_ = [("suh", U64 * MAX_JOBS), ("xh", U64 * MAX_JOBS)]


class Linear(C.Structure):
    _fields_ = [("words", U64), ("suh", U64), ("svh", U64), ("counters", U64), ("k", U32), ("n", U32), ("k2", U32),
                ("cb", U32), ("sk", U32), ("wk", U32)]


class LinearScratch(C.Structure):
    _fields_ = [("xh", U64 * MAX_JOBS), ("z", U64 * MAX_JOBS)]


class ShareInfo(C.Structure):
    _fields_ = [("dtype", I32), ("rank", U32), ("shape", U64 * 8), ("bytes", U64)]


class SwapStats(C.Structure):
    _fields_ = [("experts", U32), ("up", U32), ("down", U32), ("read_bytes", U64)]


assert C.sizeof(Job) == 88 and C.sizeof(Jobs) == 272 and C.sizeof(RotJobs) == 48  # exl3.zig:30-32

# name -> (restype, argtypes); every entry point of include/ea_exl3.h
SIGNATURES = {
    "ea_strerror": (C.c_char_p, [I32]),
    "ea_init": (I32, [I32]),
    "ea_fini": (I32, []),
    "ea_device_status": (I32, [C.POINTER(I32)]),
    "ea_device_status_address": (I32, [C.POINTER(C.c_void_p)]),
    "ea_dequant": (I32, [P, P, P, U32, U32, U32, U32]),
    "ea_exl3_unpack": (I32, [P, P, P, U32, U32, U32, U32, I64, I64]),
    "ea_experts_group": (I32, [P, P, P, P, P, U32, U32, U32, U32]),
    "ea_experts_rot_in": (I32, [P, P, I32, U32, P, P, P, P, P, U32, U32, U32, U32]),
    "ea_experts_grouped": (I32, [P, C.POINTER(GroupedArgs)]),
    "ea_experts_gateup_epilogue": (I32, [P, P, P, P, P, P, P, U32, U32, U32, U32, U32, U32, F32, U32]),
    "ea_experts_down_combine": (I32, [P, P, P, P, P, P, P, U32, U32, U32, U32, U32, U32]),
    "ea_moe_scratch_bytes": (C.c_size_t, [C.POINTER(Routed), U32, U32]),
    "ea_moe_scratch_init": (I32, [P, C.POINTER(MoeScratch), P, C.c_size_t, C.POINTER(Routed), U32, U32]),
    "ea_moe_routed": (I32, [P, P, I32, U32, P, P, C.POINTER(Routed), C.POINTER(MoeScratch), P, U32]),
    "ea_prompt_experts_supported": (I32, [C.POINTER(Routed), C.POINTER(I32)]),
    "ea_prompt_scratch_bytes": (C.c_size_t, [C.POINTER(Routed), U32, U32, I32]),
    "ea_prompt_scratch_init": (I32, [P, C.POINTER(PromptScratch), P, C.c_size_t, C.POINTER(Routed), U32, U32, I32]),
    "ea_prompt_experts_run": (I32, [P, P, I32, U32, P, P, C.POINTER(Routed), C.POINTER(PromptScratch), P, U32, I32,
                                    I32]),
    "ea_exl3_rot_in": (I32, [P, P, I32, C.POINTER(RotJobs), U32, U32, U32]),
    "ea_exl3_linear": (I32, [P, C.POINTER(Jobs), U32, U32, U32, U32, U32, U32]),
    "ea_linear_plan": (None, [U32, U32, C.POINTER(U32), C.POINTER(U32)]),
    "ea_linear_call": (I32, [P, C.POINTER(LinearScratch), C.POINTER(C.POINTER(Linear)), U32, P, I32, U32,
                             C.POINTER(U64), C.POINTER(C.c_int)]),
    "ea_linear_call_rotated": (I32, [P, C.POINTER(LinearScratch), C.POINTER(C.POINTER(Linear)), U32, U32,
                                     C.POINTER(U64), C.POINTER(C.c_int)]),
    "ea_topk8": (I32, [P, P, P, P, P, U32, F32, P]),
    "ea_router": (I32, [P, P, I32, U32, P, P, P, U32, U32, U32]),
    "ea_swiglu2": (I32, [P, P, P, P, U32, U32]),
    "ea_add_f32": (I32, [P, P, P, C.c_size_t]),
    "ea_bank_open": (I32, [C.c_char_p, U32, U32, U32, C.POINTER(P)]),
    "ea_bank_open_file": (I32, [C.c_char_p, C.c_char_p, U32, U32, U32, C.POINTER(P)]),
    "ea_bank_close": (None, [P]),
    "ea_bank_has": (I32, [P, C.c_char_p]),
    "ea_bank_share": (I32, [P, C.c_char_p, C.POINTER(ShareInfo), P, U64]),
    "ea_layer_load": (I32, [C.POINTER(P), U32, P, U32, U32, C.POINTER(P)]),
    "ea_layer_routed": (C.POINTER(Routed), [P]),
    "ea_layer_free": (None, [P]),
    "ea_layer_swap": (I32, [P, C.POINTER(P), U32, P, P, C.POINTER(SwapStats)]),
    "ea_profile_enable": (I32, [I32]),
    "ea_profile_stages": (I32, [P, U32]),
    "ea_ffn_moe_decode": (I32, [P, P, I32, U32, P, P, F32, P, P, C.POINTER(Routed), P, C.POINTER(MoeScratch), P, U32]),
    "ea_ffn_moe_decode_router": (I32, [P, P, I32, U32, P, P, P, F32, P, P, C.POINTER(Routed), P,
                                       C.POINTER(MoeScratch), P, U32]),
    "ea_ffn_moe_decode_static": (I32, [P, P, I32, U32, P, P, F32, P, P, C.POINTER(Routed), P, P, U32]),
}

_lib = None


def lib():
    """The loaded library with every entry point typed. Raises if the library was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python expertatlas-glm5.3_amd/build.py`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name, None)
            if f is None:
                MISSING.append(name)
                continue
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


# entry points of include/ea_exl3.h that the loaded library does not export (must stay empty)
MISSING: list = []


def strerror(code: int) -> str:
    return lib().ea_strerror(code).decode()


def check(code: int, where: str) -> None:
    if code != 0:
        raise EaError(code, where)
