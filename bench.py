"""Benchmark: transformer FFN block backward on one MI355X.

Workload: RMSNorm(d=2048) -> SwiGLU (gate/up 2048->5632, down 5632->2048), T = 4096 tokens
(batch 4 x seq 1024), bf16 activations/weights, fp32 accumulation; x ~ N(0,1), weights
N(0, 0.02), dY ~ N(0, 1e-2).  One step = the whole block backward:
    gn_ffn_down_glu_bwd  (down projection with the SwiGLU backward in its epilogue: dG|dU, dWd)
    gn_glu_proj_bwd      (dN = dG Wg + dU Wu, dWg, dWu)
    gn_rmsnorm_bwd       (dx, dw)
with inputs (x, saved rstd / gate / up / activations, weights, dY) resident in HBM.
The metric is layer-backward tokens/s; the dominant kernel's roofline fraction comes from
HIP events around its own launches, and the CPU baseline is the oracle (C, OpenMP) timed on
a bounded token sample of the same workload on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "grilly-next_amd"))

T, DM, HID = 4096, 2048, 5632
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--cpu-tokens", type=int, default=256)
    p.add_argument("--no-cpu", action="store_true")
    return p.parse_args()


def make_inputs(torch, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    bf = torch.bfloat16
    x = torch.randn(T, DM, device=dev, generator=g).to(bf)
    w = torch.ones(DM, device=dev, dtype=bf)
    Wg = (torch.randn(HID, DM, device=dev, generator=g) * 0.02).to(bf)
    Wu = (torch.randn(HID, DM, device=dev, generator=g) * 0.02).to(bf)
    Wd = (torch.randn(DM, HID, device=dev, generator=g) * 0.02).to(bf)
    dY = (torch.randn(T, DM, device=dev, generator=g) * 1e-2).to(bf)
    # forward (untimed) producing the saved tensors of the backward
    xf = x.float()
    rstd = torch.rsqrt((xf * xf).mean(-1) + 1e-6).contiguous()
    n = (xf * rstd[:, None] * w.float()).to(bf)
    gate = (n @ Wg.t()).contiguous()
    up = (n @ Wu.t()).contiguous()
    a = (gate.float() * torch.nn.functional.silu(up.float())).to(bf)
    return dict(x=x, w=w, Wg=Wg, Wu=Wu, Wd=Wd, dY=dY, rstd=rstd, n=n, gate=gate, up=up, a=a)


class Step:
    """The timed backward step; all buffers preallocated (no allocation inside)."""

    def __init__(self, gn, torch, d):
        self.gn, self.d = gn, d
        dev = d["x"].device
        f32, bf = torch.float32, torch.bfloat16
        self.dWd = torch.empty(DM, HID, device=dev, dtype=f32)
        self.dN = torch.empty(T, DM, device=dev, dtype=bf)
        self.dWg = torch.empty(HID, DM, device=dev, dtype=f32)
        self.dWu = torch.empty(HID, DM, device=dev, dtype=f32)
        self.gu = torch.empty(T, 2 * HID, device=dev, dtype=bf)
        self.dx = torch.empty(T, DM, device=dev, dtype=bf)
        self.dw = torch.empty(DM, device=dev, dtype=f32)
        self.ws = gn.workspace(gn.norm_workspace_bytes(T, DM), dev)

    def __call__(self):
        gn, d, P, s = self.gn, self.d, self.gn._ptr, self.gn._stream()
        L = gn.lib()
        gn._check(L.gn_ffn_down_glu_bwd(gn.GLU["swiglu_up"], P(d["dY"]), P(d["a"]), P(d["Wd"]),
                                        P(d["gate"]), P(d["up"]), P(self.gu), P(self.dWd), None,
                                        T, DM, HID, gn.BF16, 0, s), "ffn_down_glu_bwd")
        gn._check(L.gn_glu_proj_bwd(P(self.gu), P(d["n"]), P(d["Wg"]), P(d["Wu"]), P(self.dN),
                                    P(self.dWg), P(self.dWu), None, None, T, DM, HID, gn.BF16, 0,
                                    s), "glu_proj_bwd")
        gn._check(L.gn_rmsnorm_bwd(P(self.dN), P(d["x"]), P(d["w"]), P(d["rstd"]), P(self.dx),
                                   P(self.dw), T, DM, gn.BF16, 0, P(self.ws), self.ws.numel(), s),
                  "rmsnorm_bwd")


def time_dominant(gn, torch, st, reps=20):
    """HIP-event timing of the dominant GEMM launch: dN = dG Wg + dU Wu (K = 2*5632)."""
    d = st.d
    dG = st.gu[:, :HID].contiguous()
    dU = st.gu[:, HID:].contiguous()
    P, L = gn._ptr, gn.lib()
    stream = torch.cuda.current_stream()

    def launch():
        gn._check(L.gn_gemm(P(dG), P(d["Wg"]), HID, P(dU), P(d["Wu"]), HID, P(st.dN), T, DM, 0, 0,
                            gn.BF16, gn.BF16, 0, gn._stream()), "gemm")
    for _ in range(3):
        launch()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        launch()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    flops = 2.0 * T * DM * (2 * HID)
    return ms, flops


def cpu_baseline(tokens):
    """Oracle (C, OpenMP, fp64 accumulation) on `tokens` rows of the same workload."""
    import oracle
    r = np.random.default_rng(2)
    x = r.standard_normal((tokens, DM)).astype(np.float32)
    w = np.ones(DM, np.float32)
    Wg = (r.standard_normal((HID, DM)) * 0.02).astype(np.float32)
    Wu = (r.standard_normal((HID, DM)) * 0.02).astype(np.float32)
    Wd = (r.standard_normal((DM, HID)) * 0.02).astype(np.float32)
    dY = (r.standard_normal((tokens, DM)) * 1e-2).astype(np.float32)
    n, rstd = oracle.rmsnorm_fwd(x, w)
    gate, up = oracle.linear_fwd(n, Wg), oracle.linear_fwd(n, Wu)
    a = oracle.glu_fwd("swiglu_up", gate, up)
    t0 = time.perf_counter()
    dA, _, _ = oracle.linear_bwd(dY, a, Wd, need_db=False)
    dG, dU = oracle.glu_bwd("swiglu_up", dA, gate, up)
    dN1, _, _ = oracle.linear_bwd(dG, n, Wg, need_db=False)
    dN2, _, _ = oracle.linear_bwd(dU, n, Wu, need_db=False)
    oracle.rmsnorm_bwd(dN1 + dN2, x, w, rstd)
    dt = time.perf_counter() - t0
    return tokens / dt, oracle.num_threads(), dt


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the backward "
              "path has no multi-GPU code in this build", file=sys.stderr)
        sys.exit(2)
    import torch
    import gn_bwd as gn
    gn.lib()
    dev = torch.device("cuda:0")
    d = make_inputs(torch, dev)
    st = Step(gn, torch, d)
    for _ in range(args.warmup):
        st()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        st()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    dom_ms, dom_flops = time_dominant(gn, torch, st)
    achieved = dom_flops / (dom_ms * 1e-3) / 1e12
    flops_step = 6 * 2.0 * T * DM * HID
    cpu = None
    if not args.no_cpu:
        v, cores, dt = cpu_baseline(args.cpu_tokens)
        cpu = {"value": round(v, 2), "unit": "tokens/s", "cores": cores, "kind": "port",
               "sample": f"{args.cpu_tokens} of {T} tokens of the same FFN-block backward "
                         f"(oracle C/OpenMP, fp64 accumulation), {dt:.2f} s"}
    out = {
        "metric": "layer backward tokens/s (FFN block: RMSNorm + SwiGLU)",
        "value": round(T / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights, N(0,1e-2) dY)",
        "config": {"workload": "C2 FFN block backward: RMSNorm(2048) + SwiGLU 2048->5632->2048, "
                               "T=4096 (4x1024), bf16 / fp32 accumulate",
                   "tokens": T, "d_model": DM, "hidden": HID, "parallelism": "none (1 GPU)"},
        "step_tflops": round(flops_step / (ms * 1e-3) / 1e12, 2),
        "roofline": {"kernel": "gemm_bf16_mfma (dN = dG Wg + dU Wu, 4096x2048x11264)",
                     "bound": "mfma", "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
                     "launch_ms": round(dom_ms, 4), "traffic": None},
        "cpu_baseline": cpu,
        "wall_s": round(wall, 3),
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
