#!/usr/bin/env python3
"""Benchmark of the EXL3 routed-expert path on one MI355X (gfx950).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config decode|multi|stack|linear|prefill512|prefill2048]

A step is one pass of the hot path over one batch of synthetic input, with every input already in HBM:
  decode (default): one GLM-5.3 MoE layer of a TP=8 rank at batch 1 -- router top-8 from logits,
      the routed experts (moe.routed), the shared expert (EXL3 linears + SwiGLU) and their sum: ea_ffn_moe_decode,
      one launch at one row, five above (route, gate|up, epilogue, down, combine); the default line also carries
      the metric's second half, the 512-token prefill chunk (config 4), as the object "prefill512";
  multi (config 3): the same layer at 16 rows, uniform top-8 (no router bias), 70 % of the experts at 3 bits;
  stack (config 5): 75 resident layers (3-bit for 70 % of the experts), one token through all of them (us / token);
  linear (config 1): one 4-bit EXL3 linear 6144 x 2048 at one row (linear.call);
  prefill512 / prefill2048 (config 4): prompt_experts.run over 512 / 2048 rows with Zipf(1.1) routing.
The decode configs cycle through several distinct resident layers and draw fresh router logits every layer, so the
touched experts are not sitting in the 256 MB Infinity Cache. Their timed region replays the K steps from a HIP
graph (as the reference runs decode); the same steps launched one by one are reported beside it. Prints one JSON
line, with the library's path and hash and the device it ran on.

The dominant kernel's roofline is measured live: HIP events around each of its launches (on the stream the launches
go to) over a further pass identical to the timed one; its algorithmic bytes per launch are the trellis + scales of
every distinct expert the launch touches, the shared expert, the activations, logits and outputs. Its rocprof kernel
duration and HBM traffic a launch come from the committed counter summary (profiles/layer1_kernel_config2.md).
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


def baseline_metric() -> str:
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        return json.load(f)["metric"]


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="decode",
                    choices=["decode", "multi", "stack", "linear", "prefill512", "prefill2048"])
    ap.add_argument("--layers", type=int, default=8, help="distinct resident layers the decode configs cycle through")
    ap.add_argument("--path", default="fused", choices=["fused", "sequence"],
                    help="decode configs: ea_ffn_moe_decode, or the reference's launch sequence (topk, "
                         "moe.routed's six launches, the shared expert's linears, swiglu2, add)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="decode: leave out the 512-token prefill object")
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

    def step_events(self, i: int, ev: list) -> None:
        """Step i again, timing its launches: the fused path's launches from the library's stage events
        (recorded on the launch stream), the sequence path's grouped launches from torch events on the same stream."""
        for q in range(self.per_step):
            j = i * self.per_step + q
            if self.path == "fused":
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
        k.down_combine(s, sc.z, pick, ex.svh_d, sc.y, wts, self._out, R, P, D, 1, SLOTS, E)
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


def time_steps(fn, steps: int, warmup: int, torch, first: int = 0) -> float:
    """Milliseconds a step over `steps` steps after `warmup` untimed ones, between two synchronised events."""
    for i in range(warmup):
        fn(first + i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
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


def time_graph(step, steps: int, warmup: int, torch, first: int = 0) -> float:
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
    graphs[0].replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
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


def cpu_baseline_prefill(seed: int, R: int, budget_s: float = 10.0) -> dict:
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
}


def _line(args, value, unit, ms, config, roofline, cpu) -> dict:
    return {"metric": baseline_metric(), "value": round(value, 3), "unit": unit, "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": False, "scaling": "weak",
            "vs_baseline": None, "dtype": "fp16", "data": DATA, "config": config, "roofline": roofline,
            "cpu_baseline": cpu}


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


def run_decode(args, torch, np) -> dict:
    workload, R, mixed, per_step, unit = WORKLOADS[args.config]
    n_layers = 75 if args.config == "stack" else args.layers
    total = args.warmup + args.steps
    bench = DecodeBench(R, n_layers, per_step, mixed, args.seed, 3 * total + 2, args.path,
                        uniform=args.config == "multi", router=args.router)
    # the timed region: K whole steps replayed from a HIP graph (how the reference runs decode); the same steps
    # launched one by one from the host are timed beside it
    graph_ms = time_graph(bench.step, args.steps, args.warmup, torch) if args.path == "fused" else None
    eager_ms = time_steps(bench.step, args.steps, args.warmup, torch, first=total)
    ms = graph_ms if graph_ms is not None else eager_ms
    # the same number of steps again, timing each launch of the dominant kernel on the stream it runs on
    ev = []
    for i in range(args.warmup):
        bench.step(2 * total + i)
    torch.cuda.synchronize()
    from ea_exl3._lib import check, lib

    if args.path == "fused":
        check(lib().ea_profile_enable(1), "profile_enable")
    for i in range(args.steps):
        bench.step_events(2 * total + args.warmup + i, ev)
    torch.cuda.synchronize()
    if args.path == "fused":
        check(lib().ea_profile_enable(0), "profile_enable")
    picks = bench.pick.cpu().numpy()
    stages = None
    one_launch = args.path == "fused" and R == 1
    if one_launch:
        # one row routed from logits: the layer is one launch, so the dominant kernel is the whole layer
        durs = [ms_[0] for _, ms_ in ev]
        nbytes = [bench.launch_bytes(j, picks)[0] for j, _ in ev]
        kernel = ("layer1_kernel (ea_ffn_moe_decode at one row routed from logits, the whole layer in one launch: "
                  "top-8, gate|up of the 8 picks and the shared expert, SwiGLU, down, slot-ordered combine)")
    elif args.path == "fused":
        durs = [ms_[0] for _, ms_ in ev]
        nbytes = [bench.gateup_bytes(j, picks) for j, _ in ev]
        kernel = ("route_kernel + gateup_wide_kernel (ea_ffn_moe_decode's first two launches, timed together: the "
                  "window's top-8 and grouping once, then the gate and up EXL3 GEMV of every touched routed expert and "
                  "of the shared expert)")
        stages = {name: round(sum(ms_[k] for _, ms_ in ev) / len(ev) * 1e3, 3)
                  for k, name in enumerate(("gateup_us", "epilogue_us", "down_us", "combine_us"))}
    else:
        durs = [a.elapsed_time(b) for _, a, b, _ in ev]
        nbytes = [bench.grouped_bytes(j, picks, w) for j, _, _, w in ev]
        kernel = "grouped_kernel (the routed experts' EXL3 grouped GEMV: gate|up and down launches)"
    avg_ms = sum(durs) / len(durs)
    avg_b = sum(nbytes) / len(nbytes)
    timing = "HIP events recorded on the launch stream around each launch (dispatch included)"
    event_us = None
    if one_launch and graph_ms is not None:
        # one launch a layer: the timed region's average (HIP events around the graph replay on the launch stream) is
        # the kernel's average launch duration, back to back as a model runs it; each launch timed between its own
        # events (which adds their dispatch) is reported beside it
        event_us = round(avg_ms * 1e3, 3)
        avg_ms = graph_ms
        timing = ("HIP events around the graph replay of the timed layers, on the launch stream: one launch a layer, "
                  "so the per-layer time is the kernel's average launch duration (gaps between launches included)")
    achieved = avg_b / (avg_ms * 1e-3) / 1e9
    # the step's own roofline, from the timed steps' launches
    first = (args.warmup if graph_ms is not None else total + args.warmup) * per_step
    lb = [bench.launch_bytes(first + j, picks) for j in range(args.steps * per_step)]
    step_b = sum(b for b, _ in lb) / args.steps
    step_f = sum(f for _, f in lb) / args.steps
    us = ms * 1e3
    t_roof_us = max(step_b / (HBM_PEAK_GBS * 1e9), step_f / (FP16_PEAK_TFLOPS * 1e12)) * 1e6
    distinct = float(np.mean([len(set(int(e) for e in picks[first + j].reshape(-1)))
                              for j in range(args.steps * per_step)]))
    if args.router:
        workload += "; logits computed from x by a bf16 router weight [256, 6144] (ea_ffn_moe_decode_router)"
    config = {"workload": workload, "path": args.path, "timing": "hip graph" if graph_ms is not None else "eager",
              "eager_us": round(eager_ms * 1e3, 3), "layers_resident": n_layers, "distinct_experts_per_layer":
              round(distinct, 2), "step_bytes": int(step_b), "step_flops": int(step_f),
              "step_roofline_us": round(t_roof_us, 3), "step_hbm_frac": round(t_roof_us / us, 4),
              "step_gbs": round(step_b / (us * 1e-6) / 1e9, 1)}
    roofline = {"kernel": kernel, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "avg_launch_us": round(avg_ms * 1e3, 3),
                "bytes_per_launch": int(avg_b), "launches_timed": len(durs), "timing": timing}
    if event_us is not None:
        roofline["event_us_per_launch"] = event_us
    if stages:
        roofline["layer_stages"] = stages
    if args.config == "decode" and one_launch:
        prof = "layer1_kernel_config2.md"
        rp = recorded_figure(prof, "layer1_kernel_avg_us")
        if rp:
            roofline["rocprof_avg_us"] = rp
            roofline["rocprof_frac"] = round(avg_b / (rp * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
            roofline["rocprof_source"] = f"profiles/{prof} (rocprofv3 --kernel-trace --stats)"
        tr = recorded_figure(prof, "traffic_bytes_per_launch")
        if tr:
            roofline["traffic"] = int(tr)
            roofline["traffic_source"] = f"profiles/{prof} (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; copy-calibrated)"
    cpu = None if args.no_cpu_baseline else cpu_baseline_decode(args.seed, R, mixed, layers_per_unit=per_step,
                                                                unit=unit)
    return _line(args, us, unit, ms, config, roofline, cpu)


def run_linear(args, torch, np) -> dict:
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

    eager_ms = time_steps(step, args.steps, args.warmup, torch)
    ms = time_graph(step, args.steps, args.warmup, torch)
    b = lins[0].bytes() + K * 2 + N * 4
    f = 2 * K * N
    us = ms * 1e3
    t_roof = max(b / (HBM_PEAK_GBS * 1e9), f / (FP16_PEAK_TFLOPS * 1e12)) * 1e6
    gbs = b / (us * 1e-6) / 1e9
    config = {"workload": "config 1: one EXL3 4-bit linear K 6144 x N 2048 at one fp16 row, fp32 out (linear.call: "
                          "one launch of the small-row kernel, rotation in the kernel)", "linears_resident": args.layers,
              "step_bytes": b, "step_roofline_us": round(t_roof, 3), "step_hbm_frac": round(t_roof / us, 4),
              "timing": "HIP graph of the timed calls, replayed once between synchronized events",
              "eager_us": round(eager_ms * 1e3, 3)}
    roofline = {"kernel": "lin_small_kernel (the whole call)", "bound": "hbm", "achieved": round(gbs, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None}
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
    cpu = None if args.no_cpu_baseline else cpu_baseline_linear(args.seed)
    return _line(args, us, "us/linear", ms, config, roofline, cpu)


def run_prefill(args, torch, np, R: int, steps: int | None = None, warmup: int | None = None) -> dict:
    """Config 4: prompt_experts.run over R rows, Zipf(1.1) routing, 4-bit experts. Its binding roof is HBM (about 68
    flops a byte at 512 rows, below the ~312 ridge); the MFMA fraction is reported beside it."""
    from ea_exl3 import device, prompt_experts, synth
    from ea_exl3.resident import DeviceRouted

    steps = args.steps if steps is None else steps
    warmup = args.warmup if warmup is None else warmup
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
    sc = prompt_experts.Scratch(ex, R, SLOTS)
    s = device.stream()

    def step(i, stream=None):
        prompt_experts.run(s if stream is None else stream, x.data_ptr(), D, dp.data_ptr(), dw.data_ptr(), ex, sc,
                           out.data_ptr(), R, do_round=False, x_dtype=0)

    ms = time_steps(step, steps, warmup, torch)
    graph_ms = time_graph(step, steps, warmup, torch)
    distinct = sorted(set(int(e) for e in pick.reshape(-1)))
    b = sum(lay.expert_bytes(e) for e in distinct) + R * D * 2 + R * D * 4 + R * SLOTS * 8
    f = 2 * R * SLOTS * 3 * D * I
    us = ms * 1e3
    t_hbm, t_mfma = b / (HBM_PEAK_GBS * 1e9) * 1e6, f / (FP16_PEAK_TFLOPS * 1e12) * 1e6
    gbs, tfs = b / (us * 1e-6) / 1e9, f / (us * 1e-6) / 1e12
    config = {"workload": f"config 4: prefill chunk of {R} tokens x 6144 through prompt_experts.run, Zipf(1.1) top-8 "
                          "routing over 256 4-bit experts", "distinct_experts": len(distinct), "step_bytes": b,
              "step_flops": f, "step_roofline_us": round(max(t_hbm, t_mfma), 3),
              "step_roof_frac": round(max(t_hbm, t_mfma) / us, 4), "step_gbs": round(gbs, 1),
              "step_tflops": round(tfs, 2), "mfma_frac": round(tfs / FP16_PEAK_TFLOPS, 4),
              "timing": "launched one by one between synchronized events (the two item lists on two streams run "
                        "side by side)", "graph_us": round(graph_ms * 1e3, 3),
              "graph_note": "the same layers replayed from a HIP graph: the runtime runs the side stream's branch after "
                            "the main one, not beside it"}
    roofline = {"kernel": "prompt_experts.run (whole call: route, rot_in, gate|up item GEMMs, epilogue, down item "
                          "GEMMs, combine)", "bound": "hbm" if t_hbm >= t_mfma else "mfma",
                "achieved": round(gbs, 1) if t_hbm >= t_mfma else round(tfs, 2),
                "peak": HBM_PEAK_GBS if t_hbm >= t_mfma else FP16_PEAK_TFLOPS,
                "unit": "GB/s" if t_hbm >= t_mfma else "TFLOP/s",
                "frac": round(max(t_hbm, t_mfma) / us, 4), "traffic": None,
                "mfma": {"achieved": round(tfs, 2), "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tfs / FP16_PEAK_TFLOPS, 4)}}
    prof = "prefill_config4.md"
    tr = recorded_figure(prof, "traffic_bytes_per_layer" + ("" if R == 512 else f"_{R}"))
    if tr is not None:  # HBM bytes of the whole layer (every kernel's FETCH_SIZE + WRITE_SIZE, copy-calibrated)
        roofline["traffic"] = int(tr)
        roofline["traffic_source"] = f"profiles/{prof} (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; copy-calibrated)"
    cpu = None if args.no_cpu_baseline else cpu_baseline_prefill(args.seed, R)
    return _line(args, us, "us/layer", ms, config, roofline, cpu) | {"steps": steps, "warmup": warmup}


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
    if args.config in WORKLOADS:
        result = run_decode(args, torch, np)
    elif args.config == "linear":
        result = run_linear(args, torch, np)
    else:
        result = run_prefill(args, torch, np, 512 if args.config == "prefill512" else 2048)
    if args.config == "decode" and not args.no_prefill:
        # the metric's second half: the 512-token prefill chunk (config 4), timed over the line's own steps and
        # warm-up (a layer is ~0.33 ms, so the timed region stays well under a second)
        pf = run_prefill(args, torch, np, 512)
        result["prefill512"] = {k: pf[k] for k in ("value", "unit", "steps", "warmup", "ms_per_step", "config",
                                                   "roofline", "cpu_baseline")}
    result["library"] = library_identity()
    result["device"] = device_identity(torch)
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
