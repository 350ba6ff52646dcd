#!/usr/bin/env python3
"""Benchmark of the EXL3 routed-expert path on one MI355X (gfx950).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config decode|multi|prefill512|prefill2048|linear|stack]

A step is one pass of the hot path over one batch of synthetic input:
  decode (default): one GLM-5.3 MoE layer of a TP=8 rank at batch 1 -- router top-8 from logits,
      the routed experts (moe.routed), the shared expert (EXL3 linears + SwiGLU) and their sum;
  multi (config 3): the same layer at 16 rows, uniform top-8, 70 % of experts at 3 bits;
  prefill512 / prefill2048 (config 4): prompt_experts.run over 512 / 2048 rows with Zipf(1.1) routing;
  linear (config 1): one 4-bit EXL3 linear 6144 x 2048 at one row;
  stack (config 5): 75 resident decode layers, one token through all of them.
Expert shards live in HBM; the decode configs cycle through several distinct layers and draw fresh routing each step,
so the touched experts are not resident in the 256 MB Infinity Cache. Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "expertatlas-glm5.3_amd"))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
FP16_PEAK_TFLOPS = 2500.0    # MI355X dense fp16 MFMA, TFLOP/s
D, I, E, SLOTS = 6144, 256, 256, 8


def baseline_metric() -> str:
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        return json.load(f)["metric"]


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="decode",
                    choices=["decode", "multi", "prefill512", "prefill2048", "linear", "stack"])
    ap.add_argument("--layers", type=int, default=8, help="distinct resident layers the decode configs cycle through")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain device copy of known size (for HBM counter calibration)")
    ap.add_argument("--seed", type=int, default=1234)
    return ap.parse_args()


# ---- the workloads ---------------------------------------------------------------------------------------------------

class DecodeLayerBench:
    """Router top-8 + routed experts + shared expert + sum, R rows, cycling `layers` resident layers."""

    def __init__(self, R: int, layers: int, mixed: bool, seed: int, steps_total: int):
        import numpy as np
        import torch
        from ea_exl3 import device, experts, linear, moe, ops, synth
        from ea_exl3.resident import DeviceRouted, DeviceShared

        self.torch, self.np = torch, np
        self.device, self.experts, self.linear, self.moe, self.ops = device, experts, linear, moe, ops
        self.R = R
        k2 = synth.mixed_widths(seed, E) if mixed else 8
        self.layers = [DeviceRouted(seed + 17 * l, E, D, I, k2=k2, cb=1) for l in range(layers)]
        self.shared = [DeviceShared(seed + 1000 + l, D, I, 8, 1) for l in range(layers)]
        gen = torch.Generator(device="cuda")
        gen.manual_seed(seed + 7)
        self.x = torch.randn((R, D), device="cuda", generator=gen).to(torch.float16)
        self.logits = torch.randn((steps_total, R, E), device="cuda", generator=gen)
        self.bias = 0.1 * torch.randn(E, device="cuda", generator=gen)
        self.pick = torch.zeros((R, SLOTS), dtype=torch.int32, device="cuda")
        self.wts = torch.zeros((R, SLOTS), dtype=torch.float32, device="cuda")
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

    def step(self, i: int) -> None:
        l = i % len(self.layers)
        s, R = self.s, self.R
        self.ops.topk(s, self.logits[i].data_ptr(), self.bias.data_ptr(), self.pick.data_ptr(), self.wts.data_ptr(), R)
        self.moe.routed(s, self.x.data_ptr(), D, self.pick.data_ptr(), self.wts.data_ptr(), self.ex[l], self.scratch,
                        self.out.data_ptr(), R, x_dtype=0)
        self.shared_expert(l)
        self.ops.add_f32(s, self.out.data_ptr(), self.sy.data_ptr(), R * D)

    def shared_expert(self, l: int) -> None:
        # forward.zig:2328-2341 mlp: gate and up (bf16 out), SwiGLU, down (fp32 out)
        sh, s, R = self.shared[l], self.s, self.R
        self.linear.call(s, self.lscratch, [sh.gate, sh.up], self.x.data_ptr(), 0, R,
                         [self.g.data_ptr(), self.u.data_ptr()], [1, 1])
        self.ops.swiglu2(s, self.g.data_ptr(), self.u.data_ptr(), self.act.data_ptr(), R, I)
        self.linear.call(s, self.lscratch, [sh.down], self.act.data_ptr(), 1, R, [self.sy.data_ptr()], [2])

    # the routed sequence of moe.routed issued launch by launch, with events around the grouped launches
    def step_instrumented(self, i: int, ev: list) -> None:
        torch = self.torch
        l = i % len(self.layers)
        s, R = self.s, self.R
        sc, ex = self.scratch.c, self.ex[l].c
        P = R * SLOTS
        maxu = min(P, E)
        self.ops.topk(s, self.logits[i].data_ptr(), self.bias.data_ptr(), self.pick.data_ptr(), self.wts.data_ptr(), R)
        k = self.k
        k.group(s, self.pick.data_ptr(), sc.ids, sc.count, sc.members, R, SLOTS, E, R)
        k.rot_in(s, self.x.data_ptr(), D, self.pick.data_ptr(), ex.suh_g, ex.suh_u, sc.xg, sc.xu, R, D, SLOTS, E,
                 x_dtype=0)
        a = self.experts.grouped_args(x0=sc.xg, x1=sc.xu, tp0=ex.ptr[0], tp1=ex.ptr[1], k2_0=ex.k2[0], k2_1=ex.k2[1],
                                      uids=sc.ids, ucount=sc.count, members=sc.members, z=sc.z, K=D, N=I, P=P, SK=4,
                                      maxm=R, slots=SLOTS, nexp_max=maxu, mats=2, cb=1, nt=8, warps=4, pf=1,
                                      lo=ex.k2_gu[0], hi=ex.k2_gu[1])
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        k.grouped(s, a)
        e1.record()
        ev.append(("gateup", e0, e1))
        k.gateup_epilogue(s, sc.z, self.pick.data_ptr(), ex.svh_g, ex.svh_u, ex.suh_d, sc.xd, R, P, I, 4, SLOTS, E,
                          float("inf"), 1)
        d = self.experts.grouped_args(x0=sc.xd, x1=sc.xd, tp0=ex.ptr[2], tp1=ex.ptr[2], k2_0=ex.k2[2], k2_1=ex.k2[2],
                                      uids=sc.ids, ucount=sc.count, members=sc.members, z=sc.z, K=I, N=D, P=P, SK=1,
                                      maxm=R, slots=SLOTS, nexp_max=maxu, mats=1, cb=1, nt=8, warps=4, pf=1,
                                      lo=ex.k2_d[0], hi=ex.k2_d[1])
        e2, e3 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e2.record()
        k.grouped(s, d)
        e3.record()
        ev.append(("down", e2, e3))
        k.down_combine(s, sc.z, self.pick.data_ptr(), ex.svh_d, sc.y, self.wts.data_ptr(), self.out.data_ptr(), R, P, D,
                       1, SLOTS, E)
        self.shared_expert(l)
        self.ops.add_f32(s, self.out.data_ptr(), self.sy.data_ptr(), R * D)

    def layer_bytes(self, i: int) -> tuple[int, int]:
        """Algorithmic bytes and flops of step i: the trellis + scales of every distinct expert it touches, the
        shared expert, the activations in and out and the logits."""
        pick = self.np.asarray(self.pick.cpu())
        return self._bytes_of(i, pick)

    def _bytes_of(self, i, pick):
        l = i % len(self.layers)
        distinct = sorted(set(int(e) for e in pick.reshape(-1)))
        b = sum(self.layers[l].expert_bytes(e) for e in distinct) + self.shared[l].bytes()
        b += self.R * D * 2 + self.R * E * 4 + self.R * D * 4
        f = 2 * (self.R * SLOTS + self.R) * 3 * D * I
        return b, f, distinct

    def grouped_bytes(self, distinct: list, l: int) -> tuple[int, int]:
        """Algorithmic bytes of the gate|up and the down grouped launches: the touched experts' trellis, the
        rotated inputs read and the partial sums written."""
        lay = self.layers[l]
        P = self.R * SLOTS
        gu = sum(int(lay.bytes[0][e] + lay.bytes[1][e]) for e in distinct) + 2 * P * D * 2 + 2 * 4 * P * I * 4
        dn = sum(int(lay.bytes[2][e]) for e in distinct) + P * I * 2 + P * D * 4
        return gu, dn


def time_steps(fn, steps: int, warmup: int, torch) -> float:
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        fn(warmup + i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


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

def cpu_baseline_decode(seed: int, budget_s: float = 12.0) -> dict:
    """The C oracle (OpenMP) on the host cores, on config 2's work: the layer at batch 1 with 8 routed experts and
    the shared expert, fresh routing per layer. A bounded sample: layers until `budget_s` seconds have passed."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    from ea_exl3 import synth

    rng = np.random.default_rng(seed)
    x = synth.activations(seed, 1, D, "f16")
    sh = [synth.trellis(seed, 99, m, 0, k, n, 8) for m, (k, n) in enumerate(((D, I), (D, I), (I, D)))]
    sh_s = [orc.expert_to_strips(sh[m], k, n, 8) for m, (k, n) in enumerate(((D, I), (D, I), (I, D)))]
    suh = [synth.scales(seed + m, k, 1.0) for m, k in enumerate((D, D, I))]
    svh = [synth.scales(seed + 10 + m, n, 0.02) for m, n in enumerate((I, I, D))]
    tw = 32

    def run(pick, wts, host):
        r = _oracle_routed(orc, host)
        out = orc.moe_routed(x, pick, wts, r, 1, SLOTS)
        xh = [orc.exl3_rot_in(x, suh[m], 1, D) for m in (0, 1)]
        sk, wk = orc.linear_plan(D, I)
        g = orc.exl3_linear(xh[0], sh_s[0], 8 * tw, (D // 16) * 8 * tw, svh[0], 1, D, I, 8, 1, sk, wk, y_dtype=1)
        u = orc.exl3_linear(xh[1], sh_s[1], 8 * tw, (D // 16) * 8 * tw, svh[1], 1, D, I, 8, 1, sk, wk, y_dtype=1)
        act = orc.swiglu2(g, u)
        xd = orc.exl3_rot_in(act, suh[2], 1, I, bf16=True)
        sk, wk = orc.linear_plan(I, D)
        sy = orc.exl3_linear(xd, sh_s[2], 8 * tw, (I // 16) * 8 * tw, svh[2], 1, I, D, 8, 1, sk, wk)
        return out + sy

    # warm the codebook table and the page cache, then time whole layers (host data built outside the clock)
    cases = []
    for i in range(3):
        pick = np.sort(rng.choice(E, SLOTS, replace=False)).astype(np.int32).reshape(1, SLOTS)
        cases.append((pick, synth.routing_weights(seed + i, 1, SLOTS),
                      synth.HostLayer(seed + i, experts=E, dims=D, width=I, k2=8, only=pick.reshape(-1))))
    run(*cases[0])
    n, t_total = 0, 0.0
    while t_total < budget_s and n < 40:
        case = cases[n % len(cases)]
        t0 = time.perf_counter()
        run(*case)
        t_total += time.perf_counter() - t0
        n += 1
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round(t_total / n * 1e6, 1), "unit": "us/layer", "cores": threads, "kind": "port",
            "sample": f"{n} config-2 layers (batch 1: 8 routed 4-bit experts + 4-bit shared expert, D 6144, I 256) "
                      f"through the C oracle with OpenMP, {threads} threads"}


def _oracle_routed(orc, host):
    import numpy as np

    mats = []
    for m in range(3):
        real = [t for t in host.trellis[m] if t is not None]
        ph = np.zeros_like(real[0])
        mats.append([t if t is not None else ph for t in host.trellis[m]])
    return orc.Routed(mats, host.k2, host.suh_g, host.suh_u, host.svh_g, host.svh_u, host.suh_d, host.svh_d,
                      host.dims, host.width, host.cb)


# ---- main ---------------------------------------------------------------------------------------------------------

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

    if args.config not in ("decode",):
        print(f"config {args.config} is not wired into bench.py yet", file=sys.stderr)
        return 2

    total = args.warmup + args.steps
    bench = DecodeLayerBench(1, args.layers, False, args.seed, 2 * total + 8)
    # the timed region: K whole layers
    ms = time_steps(bench.step, args.steps, args.warmup, torch)

    # the dominant kernel, live: events around the grouped launches of the same steps issued launch by launch
    ev = []
    picks = []
    for i in range(args.warmup):
        bench.step_instrumented(total + i, [])
    torch.cuda.synchronize()
    for i in range(args.steps):
        bench.step_instrumented(total + args.warmup + i, ev)
        if i < 16:
            picks.append(np.asarray(bench.pick.cpu()))
    torch.cuda.synchronize()
    gu_ms = [a.elapsed_time(b) for n, a, b in ev if n == "gateup"]
    dn_ms = [a.elapsed_time(b) for n, a, b in ev if n == "down"]
    distinct = sorted(set(int(e) for e in picks[0].reshape(-1)))
    gu_b, dn_b = bench.grouped_bytes(distinct, 0)
    avg_launch_ms = (sum(gu_ms) + sum(dn_ms)) / (len(gu_ms) + len(dn_ms))
    avg_launch_b = (gu_b + dn_b) / 2
    achieved = avg_launch_b / (avg_launch_ms * 1e-3) / 1e9

    layer_b, layer_f, _ = bench._bytes_of(0, picks[0])
    us = ms * 1e3
    t_roof_us = max(layer_b / (HBM_PEAK_GBS * 1e9), layer_f / (FP16_PEAK_TFLOPS * 1e12)) * 1e6
    result = {
        "metric": baseline_metric(),
        "value": round(us, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: seeded random EXL3 trellis words (any bit stream is a valid tile), random-sign fp16 "
                "scales sized for N(0, 0.02) weights, N(0,1) fp16 activations and router logits (fresh each step)",
        "config": {
            "workload": "config 2: one GLM-5.3 MoE layer at batch-1 decode, one TP=8 rank's shard (D 6144, 256 "
                        "routed experts x I 256 + shared expert, EXL3 4-bit mcg), router top-8 from logits",
            "layers_cycled": args.layers,
            "layer_bytes": layer_b,
            "layer_flops": layer_f,
            "layer_roofline_us": round(t_roof_us, 3),
            "layer_hbm_frac": round(t_roof_us / us, 4),
            "layer_gbs": round(layer_b / (us * 1e-6) / 1e9, 1),
        },
        "roofline": {
            "kernel": "grouped_kernel (the routed experts' EXL3 grouped GEMV: gate|up and down launches)",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "avg_launch_us": round(avg_launch_ms * 1e3, 3),
            "bytes_per_launch": int(avg_launch_b),
            "gateup_us": round(sum(gu_ms) / len(gu_ms) * 1e3, 3),
            "down_us": round(sum(dn_ms) / len(dn_ms) * 1e3, 3),
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline_decode(args.seed)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
