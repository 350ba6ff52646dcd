"""Device plumbing for the host mirror: torch tensors hold device memory, their addresses go through the C ABI.
torch is used for allocation and streams only; every kernel is the HIP library's."""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from ._lib import check, lib

_ready = set()


def init(device: int = 0) -> None:
    """ea_init on `device` (the reference's Kernels.load)."""
    if not torch.cuda.is_available():
        raise RuntimeError("the EXL3 expert path needs a GPU (gfx950); none is visible")
    if device not in _ready:
        torch.cuda.set_device(device)
        check(lib().ea_init(device), "ea_init")
        _ready.add(device)


def stream(s: torch.cuda.Stream | None = None) -> int:
    """A hipStream_t handle: the given torch stream or the current one."""
    return (s or torch.cuda.current_stream()).cuda_stream


def addr(t: torch.Tensor | None) -> int:
    return 0 if t is None else t.data_ptr()


def upload(a: np.ndarray, dtype=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.to("cuda", non_blocking=False)


def empty(shape, dtype) -> torch.Tensor:
    return torch.empty(shape, dtype=dtype, device="cuda")


def zeros(shape, dtype) -> torch.Tensor:
    return torch.zeros(shape, dtype=dtype, device="cuda")


def download(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    if t.dtype in (torch.float16, torch.bfloat16):
        t = t.view(torch.int16)
    a = t.cpu().numpy()
    return a.view(np.uint16) if a.dtype == np.int16 else a


def device_status() -> int:
    """The kernels' recorded error code since the last call (0 = none); synchronous."""
    v = C.c_int32(0)
    check(lib().ea_device_status(C.byref(v)), "ea_device_status")
    return v.value
