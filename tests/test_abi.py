"""The C ABI without a GPU: the library loads, exports every entry point include/ea_exl3.h declares, the structs
match the reference's byte layouts, and the host-only calls (status strings, the linear plan) behave. No kernel is
launched here."""
import ctypes as C
import os
import re

import pytest

from ea_exl3 import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "ea_exl3.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ea_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_entry_point():
    L = _lib.lib()
    names = declared_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(L, n)]
    assert missing == [], missing
    assert _lib.MISSING == []
    # and the binding types every one of them
    assert set(names) <= set(_lib.SIGNATURES), set(names) - set(_lib.SIGNATURES)


def test_struct_layouts_match_reference():
    # exl3.zig:30-32
    assert C.sizeof(_lib.Job) == 88 and C.sizeof(_lib.Jobs) == 272 and C.sizeof(_lib.RotJobs) == 48
    assert _lib.Job.y_dtype.offset == 72 and _lib.Jobs.n.offset == 264


def test_status_strings_name_the_reference_errors():
    s = _lib.strerror
    assert s(0) == "ok"
    assert s(8).startswith("UnevenSplit")        # experts.zig error.UnevenSplit
    assert s(12).startswith("ScratchTooSmall")   # moe.zig error.ScratchTooSmall
    assert s(2).startswith("UnportedLinearWalk")  # exl3.zig error.UnportedLinearWalk
    assert s(14).startswith("NotGroupable")      # linear.zig error.NotGroupable
    assert s(999) == "unknown status"


@pytest.mark.parametrize("k,n,sk,wk", [
    # linear.zig:190-204, the reference's own plan() test on GLM-5.3 TP=4 shapes
    (2048, 4096, 4, 4), (4096, 6144, 4, None), (6144, 2048, 8, None), (6144, 640, 8, None), (512, 6144, 1, None),
    # the TP=8 shared expert of this path: gate/up (6144 -> 256) and down (256 -> 6144)
    (6144, 256, 8, 4), (256, 6144, 1, 4),
])
def test_linear_plan_matches_reference(k, n, sk, wk):
    from ea_exl3 import linear
    import oracle as orc

    got = linear.plan(k, n)
    assert got[0] == sk
    if wk is not None:
        assert got[1] == wk
    assert orc.linear_plan(k, n) == got


@pytest.mark.parametrize("rows", [512, 2048, 4096, 6000])
def test_prompt_scratch_sized_by_planes(rows):
    """ea_prompt_scratch_bytes honours `planes` (prompt_experts.zig:105-122): planes 1 holds the pair plane, fp32
    [min(rows, 4096) * slots, D], planes 0 does not; a shard the atomic down epilogue does not take (I above 256)
    keeps the plane either way. Host-only arithmetic, no device memory touched."""
    L = _lib.lib()
    r = _lib.Routed()
    r.count, r.dims, r.width, r.cb = 256, 6144, 256, 1
    with_plane = L.ea_prompt_scratch_bytes(C.byref(r), rows, 8, 1)
    without = L.ea_prompt_scratch_bytes(C.byref(r), rows, 8, 0)
    n = min(rows, 4096) * 8
    assert with_plane - without == n * 6144 * 4
    r.width = 512
    assert L.ea_prompt_scratch_bytes(C.byref(r), rows, 8, 0) == L.ea_prompt_scratch_bytes(C.byref(r), rows, 8, 1)
