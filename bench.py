#!/usr/bin/env python3
"""Benchmark of the EXL3 routed-expert path on one MI355X (gfx950).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config decode|multi|stack|linear|prefill512|prefill2048]

A step is one pass of the hot path over one batch of synthetic input, with every input already in HBM:
  decode (default): one GLM-5.3 MoE layer of a TP=8 rank at batch 1 -- router top-8 from logits,
      the routed experts (moe.routed), the shared expert (EXL3 linears + SwiGLU) and their sum: ea_ffn_moe_decode,
      one launch at one row, five above (route, gate|up, epilogue, down, combine);
  multi (config 3): the same layer at 16 rows, uniform top-8 (no router bias), 70 % of the experts at 3 bits;
  stack (config 5): 75 resident layers (3-bit for 70 % of the experts), one token through all of them (us / token);
  linear (config 1): one 4-bit EXL3 linear 6144 x 2048 at one row (linear.call);
  prefill512 / prefill2048 (config 4): prompt_experts.run over 512 / 2048 rows with Zipf(1.1) routing (a _planes0
      suffix: without the pair plane, the reference's default atomic mode).
The default run times config 2 and then, into the same line as objects of their own, the workloads named by --legs
(the other BASELINE configs). Every GPU leg runs before any CPU work: a leg spins up on its own work (--spin-up
seconds of untimed calls), runs one layer outside the timed region whose output it keeps, does its W warm-up steps,
times exactly K steps launched one by one between synchronized events (the start event queued behind a GPU sleep
kernel that lasts while the host enqueues the K steps, so they run back to back from the first; a HIP graph replay of
the same steps is reported beside it), and reads the library's device status word afterwards. Then, on the host, the oracle recomputes
each kept layer (the check: max|diff| <= 2e-3 RMS(out), picks bit-exact; "parity" in the line) and the tuned CPU
layer is timed on a bounded sample ("cpu_baseline"). The run exits 1 when a check fails or a status word is set.

The decode configs cycle through several distinct resident layers and draw fresh router logits every layer, so the
touched experts are not sitting in the 256 MB Infinity Cache. Prints one JSON line, with the library's path and hash
and the device it ran on.

The dominant kernel's roofline is measured live: HIP events around each of its launches (on the stream the launches
go to) over a further pass identical to the timed one; its algorithmic bytes per launch are the trellis + scales of
every distinct expert the launch touches, the shared expert, the activations, logits and outputs. Its rocprof kernel
duration and HBM traffic a launch come from the committed counter summaries under profiles/.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "expertatlas-glm5.3_amd"))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
FP16_PEAK_TFLOPS = 2500.0    # MI355X dense fp16 MFMA, TFLOP/s
D, I, E, SLOTS = 6144, 256, 256, 8
ROUTED_SCALE = 2.5           # config.zig:97,165 routed_scaling
EXTRA_LEGS_DEFAULT = ("prefill512", "prefill512_planes0", "prefill2048", "prefill2048_planes0", "linear", "multi",
                      "stack")


def baseline_metric() -> str:
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        return json.load(f)["metric"]


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="decode",
                    choices=["decode", "multi", "stack", "window64", "window128", "linear", "prefill512",
                             "prefill2048", "prefill512_planes0", "prefill2048_planes0"])
    ap.add_argument("--legs", default=",".join(EXTRA_LEGS_DEFAULT),
                    help="decode: the further workloads timed into the same line, each as an object of its own")
    ap.add_argument("--no-extra", "--no-prefill", dest="no_extra", action="store_true",
                    help="decode: the config-2 layer alone")
    ap.add_argument("--layers", type=int, default=8, help="distinct resident layers the decode configs cycle through")
    ap.add_argument("--path", default="fused", choices=["fused", "sequence"],
                    help="decode configs: ea_ffn_moe_decode, or the reference's launch sequence (topk, "
                         "moe.routed's six launches, the shared expert's linears, swiglu2, add)")
    ap.add_argument("--planes", type=int, default=1, choices=[0, 1],
                    help="prefill legs without a _planes0 suffix: 1 the pair plane and slot-ordered combine, 0 atomics")
    ap.add_argument("--spin-up", type=float, default=0.3,
                    help="seconds of untimed calls of each leg's own work before its warm-up steps")
    ap.add_argument("--cpu-budget", type=float, default=8.0, help="seconds of CPU work each leg's CPU baseline samples")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--router", action="store_true",
                    help="decode configs: compute each layer's logits from x by a bf16 router weight "
                         "(ea_ffn_moe_decode_router) instead of reading given logits")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain device copy of known size (for HBM counter calibration)")
    ap.add_argument("--seed", type=int, default=1234)
    return ap.parse_args()


# ---- the decode workloads ------------------------------------------------------------------------------------------

class DecodeBench:
    """`per_step` layers a step (1, or 75 for the stack), each router top-8 + routed experts + shared expert + sum on
    R rows; layer launch j uses resident layer j mod n_layers."""

    def __init__(self, R: int, n_layers: int, per_step: int, mixed: bool, seed: int, steps_total: int, path: str,
                 uniform: bool = False, router: bool = False):
        import numpy as np
        import torch
        from ea_exl3 import device, experts, linear, moe, ops, synth
        from ea_exl3._lib import Linear as _Linear, lib
        from ea_exl3.resident import DeviceRouted, DeviceShared

        self.torch, self.np = torch, np
        self.device, self.experts, self.linear, self.moe, self.ops = device, experts, linear, moe, ops
        self.R, self.per_step, self.path = R, per_step, path
        k2 = synth.mixed_widths(seed, E) if mixed else 8
        self.layers = [DeviceRouted(seed + 17 * l, E, D, I, k2=k2, cb=1) for l in range(n_layers)]
        self.shared = [DeviceShared(seed + 1000 + l, D, I, 8, 1) for l in range(n_layers)]
        gen = torch.Generator(device="cuda")
        gen.manual_seed(seed + 7)
        self.x = torch.randn((R, D), device="cuda", generator=gen).to(torch.float16)
        launches = steps_total * per_step
        self.logits = torch.randn((launches, R, E), device="cuda", generator=gen)
        # uniform routing (config 3): no bias, so a row's top-8 of i.i.d. logits is a uniformly random 8-subset
        self.bias = (0.0 if uniform else 0.1) * torch.randn(E, device="cuda", generator=gen)
        self.pick = torch.zeros((launches, R, SLOTS), dtype=torch.int32, device="cuda")
        self.wts = torch.zeros((launches, R, SLOTS), dtype=torch.float32, device="cuda")
        self.out = torch.zeros((R, D), dtype=torch.float32, device="cuda")
        self.sy = torch.zeros((R, D), dtype=torch.float32, device="cuda")
        self.g = torch.zeros((R, I), dtype=torch.bfloat16, device="cuda")
        self.u = torch.zeros((R, I), dtype=torch.bfloat16, device="cuda")
        self.act = torch.zeros((R, I), dtype=torch.bfloat16, device="cuda")

        class _Ex:  # moe.Routed's interface over a DeviceRouted
            def __init__(s, dr):
                s.c = dr.c

        self.ex = [_Ex(l) for l in self.layers]
        self.scratch = moe.Scratch(self.ex[0], R, SLOTS)
        sk_max = max(self.shared[0].gate.sk, self.shared[0].down.sk)
        self.lscratch = linear.Scratch(R, D, sk_max * R * D)
        self.k = experts.Kernels.load()
        self.s = device.stream()
        # ea_ffn_moe_decode's arguments, built once: a layer costs the host one foreign call
        self.fn = lib().ea_ffn_moe_decode
        self._sh_arrays = [(C.POINTER(_Linear) * 3)(C.pointer(sh.gate.c), C.pointer(sh.up.c), C.pointer(sh.down.c))
                           for sh in self.shared]
        self._sh_ptr = [C.addressof(a) for a in self._sh_arrays]
        self._ex_ref = [C.byref(e.c) for e in self.ex]
        self._sc_ref = C.byref(self.scratch.c)
        self._logits0, self._pick0, self._wts0 = self.logits.data_ptr(), self.pick.data_ptr(), self.wts.data_ptr()
        # with `router`, each layer computes its logits from x by its own bf16 router weight [256, D]
        # (ea_ffn_moe_decode_router) instead of reading given ones
        self.router = router
        if router:
            self.router_w = [(0.02 * torch.randn((E, D), device="cuda", generator=gen)).to(torch.bfloat16)
                             for _ in range(n_layers)]
            self.fn_router = lib().ea_ffn_moe_decode_router
        self._x, self._bias, self._out = self.x.data_ptr(), self.bias.data_ptr(), self.out.data_ptr()

    def layer_of(self, j: int) -> int:
        return j % len(self.layers)

    def launch(self, j: int, stream: int | None = None) -> None:
        """Layer launch j, on the bench's stream or on `stream` (a graph capture's)."""
        if self.path != "fused":
            self.sequence(j)
            return
        if self.R > 16:  # a window the decode layer does not take: ops.topk, moe.routed, the shared expert, add
            self.window(j, stream)
            return
        l, R = self.layer_of(j), self.R
        if self.router:
            r = self.fn_router(stream or self.s, self._x, 0, D, self.router_w[l].data_ptr(),
                               self._logits0 + j * R * E * 4, self._bias, ROUTED_SCALE, self._pick0 + j * R * SLOTS * 4,
                               self._wts0 + j * R * SLOTS * 4, self._ex_ref[l], self._sh_ptr[l], self._sc_ref,
                               self._out, R)
            if r:
                from ea_exl3._lib import check

                check(r, "ffn_decode_router")
            return
        r = self.fn(stream or self.s, self._x, 0, D, self._logits0 + j * R * E * 4, self._bias, ROUTED_SCALE,
                    self._pick0 + j * R * SLOTS * 4, self._wts0 + j * R * SLOTS * 4, self._ex_ref[l],
                    self._sh_ptr[l], self._sc_ref, self._out, R)
        if r:
            from ea_exl3._lib import check

            check(r, "ffn_decode")

    def step(self, i: int, stream: int | None = None) -> None:
        for q in range(self.per_step):
            self.launch(i * self.per_step + q, stream)

    def window(self, j: int, stream: int | None = None, ev: list | None = None) -> None:
        """A window of more than 16 rows as forward.ffnMain issues it (forward.zig:2361-2403): ops.topk, moe.routed
        (ea_moe_routed: the prefill path's item GEMMs in the scratch's prompt region), the shared expert's mlp and the
        add; with ev, torch events on the launch stream around moe.routed."""
        torch = self.torch
        l, R = self.layer_of(j), self.R
        s = stream or self.s
        pick, wts = self._pick0 + j * R * SLOTS * 4, self._wts0 + j * R * SLOTS * 4
        self.ops.topk(s, self._logits0 + j * R * E * 4, self._bias, pick, wts, R)
        if ev is not None:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
        self.moe.routed(s, self._x, D, pick, wts, self.ex[l], self.scratch, self._out, R, x_dtype=0)
        if ev is not None:
            e1.record()
            ev.append((j, e0, e1, "routed"))
        sh = self.shared[l]
        self.linear.call(s, self.lscratch, [sh.gate, sh.up], self._x, 0, R, [self.g.data_ptr(), self.u.data_ptr()],
                         [1, 1])
        self.ops.swiglu2(s, self.g.data_ptr(), self.u.data_ptr(), self.act.data_ptr(), R, I)
        self.linear.call(s, self.lscratch, [sh.down], self.act.data_ptr(), 1, R, [self.sy.data_ptr()], [2])
        self.ops.add_f32(s, self._out, self.sy.data_ptr(), R * D)

    def step_events(self, i: int, ev: list) -> None:
        """Step i again, timing its launches: the fused path's launches from the library's stage events
        (recorded on the launch stream), the sequence path's grouped launches from torch events on the same stream."""
        for q in range(self.per_step):
            j = i * self.per_step + q
            if self.path == "fused" and self.R > 16:
                self.window(j, ev=ev)
            elif self.path == "fused":
                self.launch(j)
                ms = (C.c_float * 4)()
                from ea_exl3._lib import check, lib

                check(lib().ea_profile_stages(ms, 4), "profile_stages")
                ev.append((j, list(ms)))
            else:
                self.sequence(j, ev)

    # the reference's launch sequence: ops.topk, moe.routed's six launches, forward.mlp, glue.addF32
    def sequence(self, j: int, ev: list | None = None) -> None:
        torch = self.torch
        l = self.layer_of(j)
        s, R = self.s, self.R
        sc, ex = self.scratch.c, self.ex[l].c
        pick, wts = self.pick[j].data_ptr(), self.wts[j].data_ptr()
        P = R * SLOTS
        maxu = min(P, E)
        self.ops.topk(s, self.logits[j].data_ptr(), self._bias, pick, wts, R)
        if ev is not None:
            e_in = torch.cuda.Event(enable_timing=True)
            e_in.record()
        k = self.k
        k.group(s, pick, sc.ids, sc.count, sc.members, R, SLOTS, E, R)
        k.rot_in(s, self._x, D, pick, ex.suh_g, ex.suh_u, sc.xg, sc.xu, R, D, SLOTS, E, x_dtype=0)
        a = self.experts.grouped_args(x0=sc.xg, x1=sc.xu, tp0=ex.ptr[0], tp1=ex.ptr[1], k2_0=ex.k2[0], k2_1=ex.k2[1],
                                      uids=sc.ids, ucount=sc.count, members=sc.members, z=sc.z, K=D, N=I, P=P, SK=4,
                                      maxm=R, slots=SLOTS, nexp_max=maxu, mats=2, cb=1, nt=8, warps=4, pf=1,
                                      lo=ex.k2_gu[0], hi=ex.k2_gu[1])
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        k.grouped(s, a)
        e1.record()
        k.gateup_epilogue(s, sc.z, pick, ex.svh_g, ex.svh_u, ex.suh_d, sc.xd, R, P, I, 4, SLOTS, E, float("inf"), 1)
        d = self.experts.grouped_args(x0=sc.xd, x1=sc.xd, tp0=ex.ptr[2], tp1=ex.ptr[2], k2_0=ex.k2[2], k2_1=ex.k2[2],
                                      uids=sc.ids, ucount=sc.count, members=sc.members, z=sc.z, K=I, N=D, P=P, SK=1,
                                      maxm=R, slots=SLOTS, nexp_max=maxu, mats=1, cb=1, nt=8, warps=4, pf=1,
                                      lo=ex.k2_d[0], hi=ex.k2_d[1])
        e2, e3 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e2.record()
        k.grouped(s, d)
        e3.record()
        if ev is not None:
            ev.append((j, e0, e1, "gateup"))
            ev.append((j, e2, e3, "down"))
            e4 = torch.cuda.Event(enable_timing=True)
            ev.append((j, e_in, e4, "routed"))  # the sequence's moe.routed: group to down_combine
        k.down_combine(s, sc.z, pick, ex.svh_d, sc.y, wts, self._out, R, P, D, 1, SLOTS, E)
        if ev is not None:
            ev[-1][2].record()
        sh = self.shared[l]
        self.linear.call(s, self.lscratch, [sh.gate, sh.up], self._x, 0, R, [self.g.data_ptr(), self.u.data_ptr()],
                         [1, 1])
        self.ops.swiglu2(s, self.g.data_ptr(), self.u.data_ptr(), self.act.data_ptr(), R, I)
        self.linear.call(s, self.lscratch, [sh.down], self.act.data_ptr(), 1, R, [self.sy.data_ptr()], [2])
        self.ops.add_f32(s, self._out, self.sy.data_ptr(), R * D)

    def launch_bytes(self, j: int, picks) -> tuple[int, int]:
        """Algorithmic bytes and flops of layer launch j: the trellis + scales of every distinct expert it touches,
        the shared expert, the activations in, the logits and bias, pick / wts and the fp32 output."""
        l = self.layer_of(j)
        distinct = sorted(set(int(e) for e in picks[j].reshape(-1)))
        b = sum(self.layers[l].expert_bytes(e) for e in distinct) + self.shared[l].bytes()
        b += self.R * D * 2 + self.R * E * 4 + E * 4 + self.R * D * 4 + 2 * self.R * SLOTS * 4
        f = 2 * (self.R * SLOTS + self.R) * 3 * D * I
        if self.router:  # the router weight read once, its product
            b += E * D * 2
            f += 2 * self.R * E * D
        return b, f

    def gateup_bytes(self, j: int, picks) -> int:
        """Algorithmic bytes of the gate|up launch of layer launch j: gate and up trellis and suh of every distinct
        expert it touches, the shared expert's gate and up (words, suh), the activations, logits and bias."""
        l = self.layer_of(j)
        lay, sh = self.layers[l], self.shared[l]
        distinct = sorted(set(int(e) for e in picks[j].reshape(-1)))
        b = sum(int(lay.bytes[0][e] + lay.bytes[1][e]) + 2 * 2 * D for e in distinct)
        b += sh.gate.words.numel() * 4 + sh.up.words.numel() * 4 + 2 * 2 * D
        return b + self.R * D * 2 + self.R * E * 4 + E * 4

    def grouped_bytes(self, j: int, picks, which: str) -> int:
        """The sequence path's grouped launches: touched experts' trellis, rotated inputs read, partial sums written."""
        lay = self.layers[self.layer_of(j)]
        distinct = sorted(set(int(e) for e in picks[j].reshape(-1)))
        P = self.R * SLOTS
        if which == "gateup":
            return sum(int(lay.bytes[0][e] + lay.bytes[1][e]) for e in distinct) + 2 * P * D * 2 + 2 * 4 * P * I * 4
        return sum(int(lay.bytes[2][e]) for e in distinct) + P * I * 2 + P * D * 4


_HOLD = {}
HOLD_NOTE = ("; the start event is queued behind a GPU sleep kernel that covers the host's enqueueing of the K steps, "
             "so they run back to back from the first (the first launch's host latency is not timed)")


def hold_gpu(torch, us: float) -> float:
    """Queue a sleep kernel of about `us` microseconds on the current stream (torch's spin kernel, calibrated once
    against events), so that the GPU is busy while the host enqueues the launches that follow it: a timed region's
    start event recorded after the hold then does not include the first launch's host latency (about 20 us from
    Python, one extra microsecond a layer at 20 layers). Nothing of the measured work runs in it. Returns the hold's
    length in microseconds (0 where torch has no spin kernel)."""
    if not hasattr(torch.cuda, "_sleep") or us <= 0:
        return 0.0
    if "cyc_per_us" not in _HOLD:
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        torch.cuda._sleep(2_000_000)
        e1.record()
        torch.cuda.synchronize()
        _HOLD["cyc_per_us"] = 2_000_000 / max(e0.elapsed_time(e1) * 1e3, 1.0)
    torch.cuda._sleep(int(_HOLD["cyc_per_us"] * us))
    return us


def time_steps(fn, steps: int, warmup: int, torch, first: int = 0, spin=None) -> float:
    """Milliseconds a step over `steps` steps after `warmup` untimed ones, between two synchronised events; `spin()`
    (untimed calls of the leg's own work) runs right before the warm-up, with no idle gap after it. The start event is
    queued behind a GPU hold as long as 1.5 times the host's enqueue time of the timed steps (measured on the warm-up
    steps), so the steps run back to back from the first, as in a model whose host runs ahead of the GPU."""
    if spin is not None:
        spin()
    t0 = time.perf_counter()
    for i in range(warmup):
        fn(first + i)
    host_us = (time.perf_counter() - t0) * 1e6 / max(warmup, 1)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    hold_gpu(torch, min(1.5 * host_us * steps + 50.0, 300000.0))
    e0.record()
    for i in range(steps):
        fn(first + warmup + i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def _hip_runtime():
    """The HIP runtime library this process already uses (torch's), for calls torch does not wrap."""
    import ctypes

    with open("/proc/self/maps") as f:
        for line in f:
            path = line.split()[-1] if len(line.split()) >= 6 else ""
            if "libamdhip64.so" in path:
                return ctypes.CDLL(path)
    return ctypes.CDLL("libamdhip64.so")


def upload_graph(g, stream: int, torch) -> None:
    """hipGraphUpload of a captured graph's executable on `stream`: the executable's one-time set-up on the device,
    which its first replay would otherwise include. Nothing of the graph runs."""
    import ctypes

    hip = _hip_runtime()
    hip.hipGraphUpload.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    r = hip.hipGraphUpload(ctypes.c_void_p(g.raw_cuda_graph_exec()), ctypes.c_void_p(stream))
    if r != 0:
        raise RuntimeError(f"hipGraphUpload failed: {r}")
    torch.cuda.synchronize()


def time_graph(step, steps: int, warmup: int, torch, first: int = 0, spin=None) -> float:
    """Milliseconds a step, the steps replayed from a HIP graph: `warmup` steps captured into one graph and `steps`
    into another (step(i, stream) issues step i on the capture stream); both uploaded to the device (hipGraphUpload:
    the executable's one-time set-up, which a first replay would otherwise include; no step runs), the warm-up graph
    replayed untimed, then the timed graph once between two synchronised events."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # one eager step off the default stream before the captures, as torch advises
        step(first, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    graphs = []
    for lo, n in ((first, warmup), (first + warmup, steps)):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            cs = torch.cuda.current_stream().cuda_stream
            for i in range(n):
                step(lo + i, cs)
        graphs.append(g)
    torch.cuda.synchronize()
    for g in graphs:
        upload_graph(g, side.cuda_stream, torch)
    if spin is not None:
        spin()
    graphs[0].replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    hold_gpu(torch, 500.0)  # the replay's host submission behind the hold, as in time_steps
    e0.record()
    graphs[1].replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def library_identity() -> dict:
    """The HIP library the run loaded: its path relative to the repository (or as given) and a hash of its bytes."""
    import hashlib

    from ea_exl3._lib import LIB_PATH

    with open(LIB_PATH, "rb") as f:
        digest = hashlib.sha256(f.read()).hexdigest()[:16]
    rel = os.path.relpath(LIB_PATH, ROOT)
    return {"path": rel if not rel.startswith("..") else LIB_PATH, "sha256_16": digest,
            "override": bool(os.environ.get("EA_EXL3_LIB"))}


def device_identity(torch) -> dict:
    p = torch.cuda.get_device_properties(0)
    return {"name": p.name, "arch": getattr(p, "gcnArchName", ""), "cus": p.multi_processor_count}


def copy_calibration(torch) -> None:
    """A plain device copy of 512 MiB, four times: the FETCH_SIZE / WRITE_SIZE counters of this copy per dispatch
    calibrate the counters read for the expert kernels."""
    a = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    for _ in range(4):
        b.copy_(a)
    torch.cuda.synchronize()
    print(f"# copy calibration: 4 copies of {512 << 20} bytes", file=sys.stderr)


# ---- the CPU baseline -------------------------------------------------------------------------------------------------

def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_decode(seed: int, R: int = 1, mixed: bool = False, budget_s: float = 12.0, layers_per_unit: int = 1,
                        unit: str = "us/layer") -> dict:
    """The tuned CPU layer (oracle/libcpulayer.so: -O3, x86-64-v3, OpenMP over every column tile of every product) on
    the decode layer's work: R rows, 8 routed experts a row (fresh routing per layer) and the shared expert, here a
    ninth expert of every row with weight 1 (the same bytes and products; routed-expert arithmetic). A bounded sample:
    whole layers until `budget_s` seconds have passed."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    from ea_exl3 import synth

    rng = np.random.default_rng(seed)
    x = synth.activations(seed, R, D, "f16")
    k2 = synth.mixed_widths(seed, E) if mixed else np.full(E, 8, np.int32)
    k2 = np.concatenate([k2, [8]]).astype(np.int32)  # the shared expert: expert E, 4 bits

    # host data built outside the clock
    cases = []
    for i in range(3):
        pick = np.stack([np.concatenate([np.sort(rng.choice(E, SLOTS, replace=False)), [E]]) for _ in range(R)])
        wts = np.concatenate([synth.routing_weights(seed + i, R, SLOTS), np.ones((R, 1), np.float32)], axis=1)
        host = synth.HostLayer(seed + i, experts=E + 1, dims=D, width=I, k2=k2, only=np.unique(pick))
        cases.append((pick.astype(np.int32), wts.astype(np.float32), _oracle_routed(orc, host)))

    def run(case):
        pick, wts, r = case
        return orc.cpu_moe_routed(x, pick, wts, r, R, SLOTS + 1)

    run(cases[0])
    n, t_total = 0, 0.0
    while t_total < budget_s and n < 400:
        t0 = time.perf_counter()
        run(cases[n % len(cases)])
        t_total += time.perf_counter() - t0
        n += 1
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    per_layer = t_total / n * 1e6
    bits = "3/4-bit mixed" if mixed else "4-bit"
    sample = (f"{n} layers of {R} row(s) (8 routed {bits} experts a row + a 4-bit shared expert, D 6144, I 256) "
              f"through the tuned CPU layer (oracle/cpu_layer.c: -O3 x86-64-v3, tiles decoded into the products, "
              f"OpenMP over column tiles), {threads} threads on {cpu_model()}")
    if layers_per_unit > 1:
        sample += f"; the per-layer time x {layers_per_unit} layers"
    return {"value": round(per_layer * layers_per_unit, 1), "unit": unit, "cores": threads, "kind": "port",
            "sample": sample}


def _timed(fn, budget_s: float, max_n: int) -> tuple[int, float]:
    """Calls of fn until budget_s seconds have passed (at least two, at most max_n), after one untimed call."""
    fn(0)
    n, t_total = 0, 0.0
    while n < 2 or (t_total < budget_s and n < max_n):
        t0 = time.perf_counter()
        fn(n)
        t_total += time.perf_counter() - t0
        n += 1
    return n, t_total


def cpu_baseline_linear(seed: int, budget_s: float = 10.0) -> dict:
    """Config 1 on the host: the tuned CPU linear (oracle/libcpulayer.so, cpu_exl3_linear: rot_in, the product decoded
    straight into the sums with OpenMP over column tiles, the output rotation) at K 6144 x N 2048, one fp16 row, fp32
    out, over four distinct 4-bit linears in turn."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    from ea_exl3 import linear, synth

    K, N, k2 = 6144, 2048, 8
    lins = [(linear.strips(synth.trellis(seed + 10 * i, 0, 0, 0, K, N, k2), K, N, k2),
             synth.scales(seed + 10 * i + 1, K, 1.0), synth.scales(seed + 10 * i + 2, N, 0.02)) for i in range(4)]
    x = synth.activations(seed + 3, 1, K, "f16")

    def call(i):
        S, suh, svh = lins[i % len(lins)]
        orc.cpu_exl3_linear(x, suh, S, svh, 1, K, N, k2, 1)

    n, t = _timed(call, budget_s, 5000)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round(t / n * 1e6, 1), "unit": "us/linear", "cores": threads, "kind": "port",
            "sample": f"{n} calls of one 4-bit EXL3 linear (K 6144 x N 2048, one fp16 row, fp32 out; four distinct "
                      f"linears in turn) through the tuned CPU linear (oracle/cpu_layer.c: -O3 x86-64-v3, tiles "
                      f"decoded into the sums, OpenMP over column tiles), {threads} threads on {cpu_model()}"}


_CPU_PREFILL: dict = {}


def cpu_baseline_prefill(seed: int, R: int, budget_s: float = 10.0) -> dict:
    """cpu_baseline_prefill_run once per (seed, R, budget): both prefill modes compute the same function."""
    key = (seed, R, budget_s)
    if key not in _CPU_PREFILL:
        _CPU_PREFILL[key] = cpu_baseline_prefill_run(seed, R, budget_s)
    return _CPU_PREFILL[key]


def cpu_baseline_prefill_run(seed: int, R: int, budget_s: float = 10.0) -> dict:
    """Config 4 on the host: the tuned CPU layer (cpu_moe_routed, the prefill's function: the routed experts' sum of
    every row) over R rows with the bench's Zipf(1.1) top-8 routing, 4-bit experts, each expert's tiles decoded once
    for all of its rows."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as orc
    from ea_exl3 import synth

    pick = synth.picks_zipf(seed + 1, R, 1.1, E, SLOTS)
    wts = synth.routing_weights(seed + 2, R, SLOTS)
    host = synth.HostLayer(seed + 4, experts=E, dims=D, width=I, k2=8, only=np.unique(pick))
    r = _oracle_routed(orc, host)
    x = synth.activations(seed + 3, R, D, "f16")
    n, t = _timed(lambda i: orc.cpu_moe_routed(x, pick, wts, r, R, SLOTS), budget_s, 50)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round(t / n * 1e6, 1), "unit": "us/layer", "cores": threads, "kind": "port",
            "sample": f"{n} layers of {R} rows (Zipf(1.1) top-8 over 256 4-bit experts, D 6144, I 256) through the "
                      f"tuned CPU layer (oracle/cpu_layer.c: -O3 x86-64-v3, each expert's tiles decoded once into "
                      f"the sums of all of its rows, OpenMP over column tiles), {threads} threads on {cpu_model()}"}


def _oracle_routed(orc, host):
    import numpy as np

    mats = []
    for m in range(3):
        real = [t for t in host.trellis[m] if t is not None]
        ph = np.zeros_like(real[0])
        mats.append([t if t is not None else ph for t in host.trellis[m]])
    return orc.Routed(mats, host.k2, host.suh_g, host.suh_u, host.svh_g, host.svh_u, host.suh_d, host.svh_d,
                      host.dims, host.width, host.cb)


# ---- the checks of the timed kernels' outputs (run in the CPU phase, after every GPU leg) -----------------------

CHECK_BAR = 2e-3  # max|diff| <= 2e-3 * RMS(out): the north star's bar for layer outputs


def spin_up(fn, torch, seconds: float, span: int, max_calls: int = 100000) -> int:
    """Untimed calls fn(0), fn(1), .. fn(span - 1), fn(0), .. until `seconds` of GPU-bound wall time have passed (at
    least three calls; a synchronisation every 8 calls keeps the host near the GPU). Called right before a timed
    region's warm-up steps: after an idle spell the GPU runs the first milliseconds of work slower (512-token prefill,
    20 timed layers after 5 warm-up ones: 381-391 us a layer, against 322 us over 200), so the clocks come up on the
    leg's own work, not on the W warm-up steps."""
    t0 = time.perf_counter()
    n = 0
    while n < 3 or (time.perf_counter() - t0 < seconds and n < max_calls):
        fn(n % max(span, 1))
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return n


def _status_after(device) -> int:
    """The library's device status word after a leg's timed region (0: no kernel recorded an error); clears it."""
    return int(device.device_status())


def _ratio(got, want) -> tuple[float, bool]:
    import numpy as np

    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    rms = float(np.sqrt(np.mean(want * want)))
    err = float(np.max(np.abs(got - want))) if got.size else 0.0
    finite = bool(np.all(np.isfinite(got)))
    return (err / rms if rms > 0 else float("inf")), finite


def _host_routed(orc, hc: dict):
    """The oracle's Routed over a layer's host copy; experts not copied point at a zero placeholder the oracle never
    reads (it touches the picked experts only)."""
    import numpy as np

    mats = []
    for m in range(3):
        copied = hc["trellis"][m]
        ph = np.zeros_like(next(iter(copied.values())))
        mats.append([copied.get(e, ph) for e in range(hc["count"])])
    k2 = hc["k2"]
    return orc.Routed(mats, [k2, k2, k2], hc["suh_g"], hc["suh_u"], hc["svh_g"], hc["svh_u"], hc["suh_d"],
                      hc["svh_d"], hc["dims"], hc["width"], hc["cb"])


def _shared_oracle(orc, sh: list, x, R: int):
    """forward.mlp (forward.zig:2328-2341) on the oracle: bf16 gate / up linears, swiglu2, the fp32 down linear."""
    outs = []
    for m in range(2):
        L = sh[m]
        tw = 4 * L["k2"]
        xh = orc.exl3_rot_in(x, L["suh"], R, L["k"])
        outs.append(orc.exl3_linear(xh, L["words"], 8 * tw, (L["k"] // 16) * 8 * tw, L["svh"], R, L["k"], L["n"],
                                    L["k2"], L["cb"], L["sk"], L["wk"], y_dtype=1))
    act = orc.swiglu2(outs[0], outs[1])
    L = sh[2]
    tw = 4 * L["k2"]
    xh = orc.exl3_rot_in(act, L["suh"], R, L["k"], bf16=True)
    return orc.exl3_linear(xh, L["words"], 8 * tw, (L["k"] // 16) * 8 * tw, L["svh"], R, L["k"], L["n"], L["k2"],
                           L["cb"], L["sk"], L["wk"], y_dtype=2)


def decode_check_data(bench, j: int, rows: list[int]) -> dict:
    """Layer launch j once more, eagerly and outside every timed region, then its outputs and the host copies of
    everything the oracle needs to recompute the listed rows (a row's output depends on its own activations and
    logits only)."""
    import numpy as np

    torch = bench.torch
    bench.launch(j)
    torch.cuda.synchronize()
    l = bench.layer_of(j)
    d = {"j": j, "rows": rows, "R": bench.R,
         "x": bench.x.view(torch.int16).cpu().numpy().view(np.uint16)[rows].copy(),
         "logits": bench.logits[j].cpu().numpy()[rows].copy(), "bias": bench.bias.cpu().numpy().copy(),
         "out": bench.out.cpu().numpy()[rows].copy(), "pick": bench.pick[j].cpu().numpy()[rows].copy(),
         "wts": bench.wts[j].cpu().numpy()[rows].copy(), "sequence": bench.path != "fused"}
    d["layer"] = bench.layers[l].host_copy(np.unique(d["pick"]))
    d["shared"] = bench.shared[l].host_copy()
    if bench.router:
        d["router_w"] = bench.router_w[l].view(torch.int16).cpu().numpy().view(np.uint16).copy()
    return d


def decode_check(orc, d: dict) -> dict:
    """The oracle's ops.topk -> moe.routed -> forward.mlp -> add on the checked rows against the GPU's layer."""
    import numpy as np

    R = len(d["rows"])
    res = {"launch": d["j"], "rows_checked": R, "of_rows": d["R"], "bar": CHECK_BAR}
    logits = d["logits"]
    if "router_w" in d:
        want_logits = orc.router(d["x"], d["router_w"], 0)
        res["logits_bit_exact"] = bool(np.array_equal(want_logits.view(np.uint32), logits.view(np.uint32)))
    pick, wts = orc.topk8(logits, d["bias"], ROUTED_SCALE)
    res["picks_bit_exact"] = bool(np.array_equal(pick, d["pick"]) and
                                  np.array_equal(wts.view(np.uint32), d["wts"].view(np.uint32)))
    if not set(np.unique(pick)) <= set(d["layer"]["trellis"][0]):
        res.update(max_diff_over_rms=None, ok=False)
        return res
    want = orc.moe_routed(d["x"], pick, wts, _host_routed(orc, d["layer"]), R, SLOTS)
    want = want + _shared_oracle(orc, d["shared"], d["x"], R)
    r, finite = _ratio(d["out"], want)
    res["max_diff_over_rms"] = float(f"{r:.3e}")
    res["ok"] = bool(finite and r <= CHECK_BAR and res["picks_bit_exact"] and res.get("logits_bit_exact", True))
    return res


def prefill_check(orc, d: dict) -> dict:
    """The oracle's prompt_experts.run (fp32 sums, no bf16 rounding) on sampled rows against the GPU's output."""
    R = len(d["rows"])
    want = orc.prompt_experts(d["x"], d["pick"], d["wts"], _host_routed(orc, d["layer"]), R, SLOTS)
    r, finite = _ratio(d["out"], want)
    return {"rows_checked": R, "of_rows": d["R"], "bar": CHECK_BAR, "max_diff_over_rms": float(f"{r:.3e}"),
            "ok": bool(finite and r <= CHECK_BAR)}


def linear_check(orc, d: dict) -> dict:
    """The oracle's exl3 rotIn -> linear (fp32 out) against the GPU's linear.call."""
    L = d["lin"]
    tw = 4 * L["k2"]
    xh = orc.exl3_rot_in(d["x"], L["suh"], 1, L["k"])
    want = orc.exl3_linear(xh, L["words"], 8 * tw, (L["k"] // 16) * 8 * tw, L["svh"], 1, L["k"], L["n"], L["k2"],
                           L["cb"], L["sk"], L["wk"], y_dtype=2)
    r, finite = _ratio(d["out"], want)
    return {"rows_checked": 1, "bar": 1e-4, "max_diff_over_rms": float(f"{r:.3e}"), "ok": bool(finite and r <= 1e-4)}


# ---- the workloads' lines ------------------------------------------------------------------------------------------

DATA = ("synthetic: seeded random EXL3 trellis words generated on the GPU (any bit stream is a valid tile), "
        "random-sign fp16 scales sized for N(0, 0.02) weights, N(0,1) fp16 activations, N(0,1) router logits "
        "fresh every layer")

WORKLOADS = {  # name -> (workload, rows, mixed widths, layers a step, unit)
    "decode": ("config 2: one GLM-5.3 MoE layer at batch-1 decode, one TP=8 rank's shard (D 6144, 256 routed "
               "experts x I 256 + shared expert, EXL3 4-bit mcg), router top-8 from logits", 1, False, 1, "us/layer"),
    "multi": ("config 3: the same layer at 16 rows (4 conversations x 4 draft rows), uniform top-8 routing, 70 % of "
              "the routed experts at 3 bits", 16, True, 1, "us/layer"),
    "stack": ("config 5: 75 resident MoE layers of one TP=8 rank (3-bit for 70 % of the routed experts, 4-bit "
              "shared experts), one token through all of them", 1, True, 75, "us/token"),
    "window64": ("a 64-row decode window (the reference's moe.routed takes up to 128, forward.zig:21) of the config-3 "
                 "layer: uniform top-8, 70 % of the routed experts at 3 bits; ops.topk, moe.routed, the shared expert, "
                 "add", 64, True, 1, "us/layer"),
    "window128": ("a 128-row decode window of the config-3 layer: uniform top-8, 70 % of the routed experts at 3 "
                  "bits; ops.topk, moe.routed, the shared expert, add", 128, True, 1, "us/layer"),
}

def _line(args, value, unit, ms, config, roofline, steps=None, warmup=None) -> dict:
    return {"metric": baseline_metric(), "value": round(value, 3), "unit": unit, "n_gpus": 1,
            "steps": args.steps if steps is None else steps, "warmup": args.warmup if warmup is None else warmup,
            "ms_per_step": round(ms, 6), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
            "dtype": "fp16", "data": DATA, "config": config, "roofline": roofline, "cpu_baseline": None}


def recorded_figure(profile: str, key: str) -> float | None:
    """A figure from a committed rocprofv3 summary under profiles/: the line `key = value`, or None."""
    try:
        with open(os.path.join(ROOT, "profiles", profile)) as f:
            for line in f:
                if line.startswith(key + " ="):
                    return float(line.split("=")[1])
    except (OSError, ValueError):
        pass
    return None


class Leg:
    """One workload's GPU measurement (its line without cpu_baseline / parity) and the CPU work it leaves for after
    every GPU leg: the oracle check of the output it kept, and the CPU baseline."""

    def __init__(self, name: str, line: dict, check, cpu):
        self.name, self.line, self.check, self.cpu = name, line, check, cpu


def run_decode(args, torch, np, name: str) -> Leg:
    from ea_exl3 import device
    from ea_exl3._lib import check, lib

    workload, R, mixed, per_step, unit = WORKLOADS[name]
    n_layers = 75 if name == "stack" else args.layers
    total = args.warmup + args.steps
    bench = DecodeBench(R, n_layers, per_step, mixed, args.seed, 3 * total + 2, args.path,
                        uniform=name == "multi" or name.startswith("window"), router=args.router)
    device.device_status()  # clear the status word before this leg
    # the layer whose output the oracle checks: launch 3 total (none of the timed ones), rows 0 and R - 1 (and two
    # between at 16 rows)
    rows = sorted({0, R // 3, (2 * R) // 3, R - 1})
    chk = decode_check_data(bench, 3 * total * per_step, rows)
    spun = []

    def spin():
        spun.append(spin_up(bench.launch, torch, args.spin_up, max(args.warmup * per_step, 1)))

    # the timed region: K steps launched one by one between synchronized events, as a host issues layers; the same
    # steps replayed from a HIP graph are reported beside it
    eager_ms = time_steps(bench.step, args.steps, args.warmup, torch, first=total, spin=spin)
    graph_ms = time_graph(bench.step, args.steps, args.warmup, torch, spin=spin) if args.path == "fused" else None
    ms = eager_ms
    # the same number of steps again, timing each launch of the dominant kernel on the stream it runs on
    ev = []
    spin()
    for i in range(args.warmup):
        bench.step(2 * total + i)
    torch.cuda.synchronize()
    if args.path == "fused":
        check(lib().ea_profile_enable(1), "profile_enable")
    for i in range(args.steps):
        bench.step_events(2 * total + args.warmup + i, ev)
    torch.cuda.synchronize()
    if args.path == "fused":
        check(lib().ea_profile_enable(0), "profile_enable")
    status = _status_after(device)
    picks = bench.pick.cpu().numpy()
    stages = None
    one_launch = args.path == "fused" and R == 1
    if R > 16 or args.path != "fused":
        routed = [(j, a_, b_) for j, a_, b_, w in ev if w == "routed"]
        durs = [a_.elapsed_time(b_) for _, a_, b_ in routed]
        nbytes = [bench.launch_bytes(j, picks)[0] - bench.shared[bench.layer_of(j)].bytes() for j, _, _ in routed]
        kernel = ("moe.routed (ea_moe_routed: " + ("route, rot_in, the two item lists' gate|up, epilogue and down "
                  "GEMMs, the slot-ordered combine; the prefill path in the scratch's prompt region"
                  if args.path == "fused" else "the reference's six-launch sequence: group, rot_in, grouped gate|up, "
                  "epilogue, grouped down, down_combine") + "), timed with HIP events on its stream")
    elif one_launch:
        # one row routed from logits: the layer is one launch, so the dominant kernel is the whole layer
        durs = [ms_[0] for _, ms_ in ev]
        nbytes = [bench.launch_bytes(j, picks)[0] for j, _ in ev]
        kernel = ("layer1_kernel (ea_ffn_moe_decode at one row routed from logits, the whole layer in one launch: "
                  "top-8, gate|up of the 8 picks and the shared expert, SwiGLU, down, slot-ordered combine)")
    else:
        durs = [ms_[0] for _, ms_ in ev]
        nbytes = [bench.gateup_bytes(j, picks) for j, _ in ev]
        kernel = ("route_kernel + gateup_wide_kernel (ea_ffn_moe_decode's first two launches, timed together: the "
                  "window's top-8 and grouping once, then the gate and up EXL3 GEMV of every touched routed expert and "
                  "of the shared expert)")
        stages = {nm: round(sum(ms_[k] for _, ms_ in ev) / len(ev) * 1e3, 3)
                  for k, nm in enumerate(("gateup_us", "epilogue_us", "down_us", "combine_us"))}
    avg_ms = sum(durs) / len(durs)
    avg_b = sum(nbytes) / len(nbytes)
    timing = "HIP events recorded on the launch stream around each launch (dispatch included)"
    event_us = None
    if one_launch:
        # one launch a layer: the timed region's average is the kernel's average launch duration, back to back as a
        # model runs it; each launch timed between its own events (which adds their dispatch) is reported beside it
        event_us = round(avg_ms * 1e3, 3)
        avg_ms = ms / per_step
        timing = ("HIP events around the timed layers on the launch stream: one launch a layer, so the per-layer "
                  "time is the kernel's average launch duration (gaps between launches included)")
    achieved = avg_b / (avg_ms * 1e-3) / 1e9
    # the step's own roofline, from the timed steps' launches
    first = (total + args.warmup) * per_step
    lb = [bench.launch_bytes(first + j, picks) for j in range(args.steps * per_step)]
    step_b = sum(b for b, _ in lb) / args.steps
    step_f = sum(f for _, f in lb) / args.steps
    us = ms * 1e3
    t_roof_us = max(step_b / (HBM_PEAK_GBS * 1e9), step_f / (FP16_PEAK_TFLOPS * 1e12)) * 1e6
    distinct = float(np.mean([len(set(int(e) for e in picks[first + j].reshape(-1)))
                              for j in range(args.steps * per_step)]))
    if args.router:
        workload += "; logits computed from x by a bf16 router weight [256, 6144] (ea_ffn_moe_decode_router)"
    config = {"workload": workload, "path": args.path,
              "timing": "eager: the K steps launched one by one between synchronized events on the launch stream"
                        + HOLD_NOTE,
              "graph_us": None if graph_ms is None else round(graph_ms * 1e3, 3),
              "graph_note": "the same K steps replayed from one HIP graph between synchronized events, the replay "
                            "behind the same kind of hold",
              "spin_up_calls": spun, "layers_resident": n_layers, "distinct_experts_per_layer": round(distinct, 2),
              "step_bytes": int(step_b), "step_flops": int(step_f), "step_roofline_us": round(t_roof_us, 3),
              "step_hbm_frac": round(t_roof_us / us, 4), "step_gbs": round(step_b / (us * 1e-6) / 1e9, 1),
              "device_status": status}
    roofline = {"kernel": kernel, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "avg_launch_us": round(avg_ms * 1e3, 3),
                "bytes_per_launch": int(avg_b), "launches_timed": len(durs), "timing": timing}
    if event_us is not None:
        roofline["event_us_per_launch"] = event_us
    if stages:
        roofline["layer_stages"] = stages
    prof = {"decode": "layer1_kernel_config2.md", "multi": "decode_layer_config3.md"}.get(name)
    if prof and args.path == "fused" and not args.router:
        key = "layer1_kernel" if one_launch else "gateup_wide_kernel"
        rp = recorded_figure(prof, f"{key}_avg_us")
        if rp and one_launch:
            roofline["rocprof_avg_us"] = rp
            roofline["rocprof_frac"] = round(avg_b / (rp * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
            roofline["rocprof_source"] = f"profiles/{prof} (rocprofv3 --kernel-trace --stats)"
        tr = recorded_figure(prof, "traffic_bytes_per_launch")
        if tr:
            roofline["traffic"] = int(tr)
            roofline["traffic_source"] = f"profiles/{prof} (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; copy-calibrated)"
    line = _line(args, us, unit, ms, config, roofline)
    del bench
    torch.cuda.empty_cache()

    def cpu():
        return cpu_baseline_decode(args.seed, R, mixed, budget_s=args.cpu_budget, layers_per_unit=per_step, unit=unit)

    return Leg(name, line, lambda orc: decode_check(orc, chk), cpu)


def run_linear(args, torch, np) -> Leg:
    """Config 1: linear.call of one 4-bit EXL3 linear 6144 x 2048 at one row (one launch of the small-row kernel)."""
    from ea_exl3 import device, linear
    from ea_exl3._lib import Linear as _Linear, check, lib
    from ea_exl3.resident import DeviceLinear

    K, N = 6144, 2048
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed)
    lins = [DeviceLinear(gen, K, N, 8, 1) for _ in range(args.layers)]
    x = torch.randn((1, K), device="cuda", generator=gen).to(torch.float16)
    y = torch.zeros((1, N), dtype=torch.float32, device="cuda")
    sc = linear.Scratch(1, K, lins[0].sk * N)
    s = device.stream()
    fn = lib().ea_linear_call
    arrs = [(C.POINTER(_Linear) * 1)(C.pointer(l.c)) for l in lins]
    outs = (C.c_uint64 * 1)(y.data_ptr())
    dts = (C.c_int * 1)(2)
    scr = C.byref(sc.c)
    xp = x.data_ptr()

    def step(i, stream=None):
        r = fn(s if stream is None else stream, scr, arrs[i % len(arrs)], 1, xp, 0, 1, outs, dts)
        if r:
            check(r, "linear.call")

    device.device_status()
    step(0)
    torch.cuda.synchronize()
    chk = {"x": x.view(torch.int16).cpu().numpy().view(np.uint16).copy(), "out": y.cpu().numpy().copy(),
           "lin": lins[0].host_copy()}
    spun = []

    def spin():
        spun.append(spin_up(step, torch, args.spin_up, len(lins)))

    ms = time_steps(step, args.steps, args.warmup, torch, spin=spin)
    graph_ms = time_graph(step, args.steps, args.warmup, torch, spin=spin)
    status = _status_after(device)
    b = lins[0].bytes() + K * 2 + N * 4
    f = 2 * K * N
    us = ms * 1e3
    t_roof = max(b / (HBM_PEAK_GBS * 1e9), f / (FP16_PEAK_TFLOPS * 1e12)) * 1e6
    gbs = b / (us * 1e-6) / 1e9
    config = {"workload": "config 1: one EXL3 4-bit linear K 6144 x N 2048 at one fp16 row, fp32 out (linear.call: "
                          "one launch of the small-row kernel, rotation in the kernel)", "linears_resident": args.layers,
              "step_bytes": b, "step_roofline_us": round(t_roof, 3), "step_hbm_frac": round(t_roof / us, 4),
              "timing": "eager: the K calls launched one by one between synchronized events on the launch stream"
                        + HOLD_NOTE,
              "graph_us": round(graph_ms * 1e3, 3), "spin_up_calls": spun, "device_status": status}
    roofline = {"kernel": "lin_small_kernel (the whole call: one launch)", "bound": "hbm", "achieved": round(gbs, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                "avg_launch_us": round(us, 3), "bytes_per_launch": b,
                "timing": "HIP events around the timed calls on the launch stream: one launch a call"}
    prof = "lin_small_kernel_config1.md"
    rp = recorded_figure(prof, "lin_small_kernel_avg_us")
    if rp:
        roofline["rocprof_avg_us"] = rp
        roofline["rocprof_frac"] = round(b / (rp * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
        roofline["rocprof_source"] = f"profiles/{prof} (rocprofv3 --kernel-trace --stats)"
    tr = recorded_figure(prof, "traffic_bytes_per_launch")
    if tr:
        roofline["traffic"] = int(tr)
        roofline["traffic_source"] = f"profiles/{prof} (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; copy-calibrated)"
    line = _line(args, us, "us/linear", ms, config, roofline)
    del lins
    torch.cuda.empty_cache()
    return Leg("linear", line, lambda orc: linear_check(orc, chk),
               lambda: cpu_baseline_linear(args.seed, budget_s=args.cpu_budget))


def run_prefill(args, torch, np, R: int, planes: int = 1) -> Leg:
    """Config 4: prompt_experts.run over R rows, Zipf(1.1) routing, 4-bit experts. Its binding roof is HBM (about 68
    flops a byte at 512 rows, below the ~312 ridge); the MFMA fraction is reported beside it."""
    from ea_exl3 import device, prompt_experts, synth
    from ea_exl3.resident import DeviceRouted

    steps, warmup = args.steps, args.warmup
    lay = DeviceRouted(args.seed, E, D, I, k2=8, cb=1)

    class _Ex:
        def __init__(s, dr):
            s.c = dr.c

    ex = _Ex(lay)
    pick = synth.picks_zipf(args.seed + 1, R, 1.1, E, SLOTS)
    wts = synth.routing_weights(args.seed + 2, R, SLOTS)
    dp, dw = device.upload(pick), device.upload(wts)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed + 3)
    x = torch.randn((R, D), device="cuda", generator=gen).to(torch.float16)
    out = torch.zeros((R, D), dtype=torch.float32, device="cuda")
    sc = prompt_experts.Scratch(ex, R, SLOTS, planes=bool(planes))
    s = device.stream()

    def step(i, stream=None):
        prompt_experts.run(s if stream is None else stream, x.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc,
                           out.data_ptr(), R, do_round=False, x_dtype=0)

    device.device_status()
    step(0)
    torch.cuda.synchronize()
    rows = sorted(set(np.linspace(0, R - 1, 8).astype(int).tolist()))
    chk = {"R": R, "rows": rows, "x": x.view(torch.int16).cpu().numpy().view(np.uint16)[rows].copy(),
           "pick": pick[rows].copy(), "wts": wts[rows].copy(), "out": out.cpu().numpy()[rows].copy()}
    chk["layer"] = lay.host_copy(np.unique(chk["pick"]))
    spun = []

    def spin():
        spun.append(spin_up(step, torch, args.spin_up, 1))

    ms = time_steps(step, steps, warmup, torch, spin=spin)
    graph_ms = time_graph(step, steps, warmup, torch, spin=spin)
    status = _status_after(device)
    distinct = sorted(set(int(e) for e in pick.reshape(-1)))
    b = sum(lay.expert_bytes(e) for e in distinct) + R * D * 2 + R * D * 4 + R * SLOTS * 8
    f = 2 * R * SLOTS * 3 * D * I
    us = ms * 1e3
    t_hbm, t_mfma = b / (HBM_PEAK_GBS * 1e9) * 1e6, f / (FP16_PEAK_TFLOPS * 1e12) * 1e6
    gbs, tfs = b / (us * 1e-6) / 1e9, f / (us * 1e-6) / 1e12
    mode = ("planes 1: the pair plane and the slot-ordered combine (the same bits every run)" if planes else
            "planes 0: down items add into out with fp32 atomics in arrival order (the reference's default mode 0)")
    config = {"workload": f"config 4: prefill chunk of {R} tokens x 6144 through prompt_experts.run, Zipf(1.1) top-8 "
                          "routing over 256 4-bit experts", "mode": mode, "distinct_experts": len(distinct),
              "step_bytes": b, "step_flops": f, "step_roofline_us": round(max(t_hbm, t_mfma), 3),
              "step_roof_frac": round(max(t_hbm, t_mfma) / us, 4), "step_gbs": round(gbs, 1),
              "step_tflops": round(tfs, 2), "mfma_frac": round(tfs / FP16_PEAK_TFLOPS, 4),
              "timing": "eager: the K layers launched one by one between synchronized events (the two item lists "
                        "on two streams run side by side)" + HOLD_NOTE, "graph_us": round(graph_ms * 1e3, 3),
              "graph_note": "the same layers replayed from a HIP graph: the runtime runs the side stream's branch after "
                            "the main one, not beside it", "spin_up_calls": spun, "device_status": status}
    roofline = {"kernel": "prompt_experts.run (whole call: route, rot_in, gate|up item GEMMs, epilogue, down item "
                          "GEMMs, combine)", "bound": "hbm" if t_hbm >= t_mfma else "mfma",
                "achieved": round(gbs, 1) if t_hbm >= t_mfma else round(tfs, 2),
                "peak": HBM_PEAK_GBS if t_hbm >= t_mfma else FP16_PEAK_TFLOPS,
                "unit": "GB/s" if t_hbm >= t_mfma else "TFLOP/s",
                "frac": round(max(t_hbm, t_mfma) / us, 4), "traffic": None,
                "mfma": {"achieved": round(tfs, 2), "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tfs / FP16_PEAK_TFLOPS, 4)}}
    prof = "prefill_config4.md"
    key = "traffic_bytes_per_layer" + ("" if R == 512 else f"_{R}") + ("" if planes else "_planes0")
    tr = recorded_figure(prof, key)
    if tr is not None:  # HBM bytes of the whole layer (every kernel's FETCH_SIZE + WRITE_SIZE, copy-calibrated)
        roofline["traffic"] = int(tr)
        roofline["traffic_source"] = f"profiles/{prof} (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; copy-calibrated)"
    line = _line(args, us, "us/layer", ms, config, roofline, steps, warmup)
    del lay, sc
    torch.cuda.empty_cache()
    return Leg(f"prefill{R}" + ("" if planes else "_planes0"), line, lambda orc: prefill_check(orc, chk),
               lambda: cpu_baseline_prefill(args.seed, R, budget_s=args.cpu_budget))


def run_leg(args, torch, np, name: str) -> Leg:
    if name in WORKLOADS:
        return run_decode(args, torch, np, name)
    if name == "linear":
        return run_linear(args, torch, np)
    if name.startswith("prefill"):
        return run_prefill(args, torch, np, int(name[len("prefill"):].split("_")[0]),
                           planes=0 if name.endswith("_planes0") else args.planes)
    raise ValueError(name)


def main() -> int:
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build runs one TP=8 rank's expert shard on one MI355X and has no "
              "multi-GPU path; run it with --gpus 1", file=sys.stderr)
        return 2
    import numpy as np
    import torch
    from ea_exl3 import device

    device.init(0)
    if args.copy_calibration:
        copy_calibration(torch)
    names = [args.config]
    if args.config == "decode" and not args.no_extra:
        names += [n for n in args.legs.split(",") if n and n != args.config]
    # every GPU leg first, each with its own spin-up, oracle-checked launch and status word; then the CPU work
    legs = []
    for n in names:
        t0 = time.perf_counter()
        legs.append(run_leg(args, torch, np, n))
        print(f"# {n}: {legs[-1].line['value']} {legs[-1].line['unit']} ({time.perf_counter() - t0:.1f} s)",
              file=sys.stderr, flush=True)
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc  # the checker and the CPU baseline: test infrastructure, never on the timed path

    ok = True
    for leg in legs:
        t0 = time.perf_counter()
        leg.line["parity"] = leg.check(orc)
        ok = ok and leg.line["parity"]["ok"] and leg.line["config"]["device_status"] == 0
        if not args.no_cpu_baseline:
            leg.line["cpu_baseline"] = leg.cpu()
        print(f"# {leg.name}: oracle check {leg.line['parity']} ({time.perf_counter() - t0:.1f} s)", file=sys.stderr,
              flush=True)
    result = legs[0].line
    keep = ("value", "unit", "steps", "warmup", "ms_per_step", "config", "roofline", "cpu_baseline", "parity")
    for leg in legs[1:]:
        result[leg.name] = {k: leg.line[k] for k in keep}
    result["library"] = library_identity()
    result["device"] = device_identity(torch)
    print(json.dumps(result))
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
