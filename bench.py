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

Other BASELINE configs (parity-tested, measured with --workload):
    attn  configs[2]: causal attention backward with RoPE, B4 H16 S2048 D128, bf16
    vsa   configs[3]: VSA unpack-project dW (8192 x 10240 bits -> 768, fp32 dY) and the
          surrogate-loss backward (K = 4)
    mlp   configs[0]: MLP 784->256->10 fp32 B=64 through the tape engine (grilly_core)
    decoder configs[4]: 12-layer decoder (d 768, GEGLU, tied embedding 32000, CE), B8 x S1024,
          end-to-end backward through the tape engine
Each prints one JSON line of the same shape; the default (ffn) is the headline metric.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload ffn|attn|vsa|mlp|decoder]
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
    p.add_argument("--cpu-tokens", type=int, default=T)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--workload", default="ffn", choices=["ffn", "attn", "vsa", "mlp", "decoder"])
    p.add_argument("--calib-copy", action="store_true",
                   help="after the timed region, launch one gn_add_inplace over 2^28 floats "
                        "(reads 2 GiB, writes 1 GiB): the reference dispatch that scales the "
                        "FETCH_SIZE / WRITE_SIZE counters of a --pmc run")
    p.add_argument("--ceilings", action="store_true",
                   help="measure this box's MFMA (bf16 32x32x16 loop) and HBM (16-byte copy) "
                        "ceilings with the library's probe kernels and print them as JSON")
    p.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                   help="summarise two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of "
                        "'bench.py --calib-copy' into the HBM traffic of the dominant kernel")
    return p.parse_args()


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "ffn_dn_gemm_hbm_traffic.txt")
CALIB_FLOATS = 1 << 28


def calib_copy(torch, gn):
    x = torch.ones(CALIB_FLOATS, device="cuda:0")
    y = torch.zeros(CALIB_FLOATS, device="cuda:0")
    torch.cuda.synchronize()
    gn.add_inplace(y, x)
    torch.cuda.synchronize()


def pmc_summary(fetch_dir, write_dir):
    """Per-dispatch FETCH_SIZE / WRITE_SIZE (KiB) of the dominant GEMM and of the calibration
    add (known bytes) -> scaled HBM bytes per launch of the dominant GEMM."""
    import csv
    import glob
    import re

    def load(d, counter):
        out = {}
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(path)):
                if r["Counter_Name"] != counter:
                    continue
                key = (r["Kernel_Name"], r["Grid_Size"])
                out.setdefault(key, {}).setdefault(r["Dispatch_Id"], 0.0)
                out[key][r["Dispatch_Id"]] += float(r["Counter_Value"])
        return out

    res = {}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        tab = load(d, counter)
        calib = [v for (k, g), v in tab.items() if "add_kernel" in k]
        # the dN GEMM: gemm_core kernel, plain epilogue, no transposes, grid of 4096 x 2048 tiles
        gemm = {(k, g): v for (k, g), v in tab.items()
                if re.search(r"gemm_core<false, false, unsigned short, \d+, \d+, 0[,>]", k)}
        if not calib or not gemm:
            raise SystemExit(f"{counter}: calibration or GEMM dispatches not found in {d}")
        cvals = [x for v in calib for x in v.values()]
        (gk, gg), gv = max(gemm.items(), key=lambda kv: len(kv[1]))
        gvals = list(gv.values())
        res[counter] = (sum(cvals) / len(cvals), sum(gvals) / len(gvals), len(gvals), gk, gg)
    known = {"FETCH_SIZE": 2.0 * CALIB_FLOATS * 4, "WRITE_SIZE": 1.0 * CALIB_FLOATS * 4}
    total = 0.0
    lines = []
    for counter, (ckib, gkib, n, gk, gg) in res.items():
        factor = known[counter] / (ckib * 1024.0)
        b = gkib * 1024.0 * factor
        total += b
        lines.append(f"{counter}: calibration add {ckib:.0f} KiB/dispatch (expected "
                     f"{known[counter] / 1024:.0f} KiB) -> factor {factor:.4f}; dominant GEMM "
                     f"{gkib:.0f} KiB/dispatch over {n} dispatches -> {b / 1e6:.1f} MB")
    lines.append(f"kernel: {res['FETCH_SIZE'][3][:120]} grid {res['FETCH_SIZE'][4]}")
    lines.append(f"traffic_bytes_per_launch: {total:.0f}")
    print("\n".join(lines))


def ceilings(torch, gn):
    """Measured ceilings: gn_probe_mfma (no memory traffic) and gn_probe_copy (2 GiB)."""
    import ctypes
    lib = gn.lib()
    lib.gn_probe_mfma.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.gn_probe_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    dev = torch.device("cuda:0")
    blocks, iters = 4096, 2000
    out = torch.empty(blocks * 256, device=dev)
    s = gn._stream()
    mf = timed(torch, lambda: gn._check(lib.gn_probe_mfma(out.data_ptr(), blocks, iters, s),
                                        "gn_probe_mfma"), 5, 2)
    flops = blocks * 4.0 * iters * 8 * 32768
    nbytes = 1 << 31
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    cp = timed(torch, lambda: gn._check(lib.gn_probe_copy(dst.data_ptr(), src.data_ptr(), nbytes, s),
                                        "gn_probe_copy"), 10, 3)
    return {"mfma_bf16_tflops": round(flops / (mf * 1e-3) / 1e12, 1),
            "mfma_spec_tflops": BF16_PEAK_TFLOPS,
            "copy_gbs": round(2.0 * nbytes / (cp * 1e-3) / 1e9, 1), "hbm_spec_gbs": HBM_PEAK_GBS,
            "probe": f"gn_probe_mfma {blocks} blocks x {iters} x 8 MFMA per wave; "
                     f"gn_probe_copy {nbytes >> 30} GiB read + written"}


def traffic_from_profile():
    """HBM bytes per launch of the dominant GEMM from the committed counter summary."""
    try:
        for l in open(TRAFFIC_FILE):
            if l.startswith("traffic_bytes_per_launch:"):
                return int(float(l.split(":", 1)[1]))
    except OSError:
        pass
    return None


def timed(torch, fn, steps, warmup):
    """Average ms of fn() over `steps` calls, HIP events on torch's current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def line(metric, value, unit, args, ms, dtype, config, roofline, cpu, higher=True):
    return {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": higher,
            "scaling": "weak", "vs_baseline": None, "dtype": dtype,
            "data": "synthetic (seeded)", "config": config, "roofline": roofline,
            "cpu_baseline": cpu}


def bench_attn(args, torch, gn):
    """causal attention backward with RoPE (theta 1e4), B4 H16 S2048 D128."""
    B, H, S, D = 4, 16, 2048, 128
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    bf = torch.bfloat16
    Q, K, V = (torch.randn(B, H, S, D, device=dev, generator=g).to(bf) for _ in range(3))
    dO = (torch.randn(B, H, S, D, device=dev, generator=g) * 1e-2).to(bf)
    ws = gn.workspace(gn.attn_workspace_bytes(B, H, S, D), dev)
    O, LSE = gn.attn_fwd(Q, K, V, causal=True, rope="interleaved", ws=ws)
    out = (torch.empty_like(Q), torch.empty_like(K), torch.empty_like(V))
    ms = timed(torch, lambda: gn.attn_bwd(Q, K, V, O, dO, LSE, causal=True, rope="interleaved",
                                          ws=ws, out=out), args.steps, args.warmup)
    flops = 5 * 2.0 * S * S * D * 0.5 * B * H  # causal, algorithmic (5 GEMMs)
    tf = flops / (ms * 1e-3) / 1e12
    cpu = None
    if not args.no_cpu:
        import oracle
        r = np.random.default_rng(3)
        Bs, Hs, Ss = B, H, S  # the whole workload
        q, k, v = (r.standard_normal((Bs, Hs, Ss, D)).astype(np.float32) for _ in range(3))
        do = (r.standard_normal((Bs, Hs, Ss, D)) * 1e-2).astype(np.float32)
        o, lse = oracle.attn_fwd(q, k, v)
        t0 = time.perf_counter()
        oracle.attn_bwd(q, k, v, do, lse)
        dt = time.perf_counter() - t0
        cpu = {"value": round(5 * 2.0 * Ss * Ss * D * 0.5 * Bs * Hs / dt / 1e12, 6), "unit": "TFLOP/s",
               "cores": oracle.num_threads(), "kind": "port",
               "sample": f"{Bs} x {Hs} heads x S={Ss}, the whole workload (oracle C/OpenMP fp64), {dt:.2f} s"}
    out = line("causal attention backward with RoPE (algorithmic TFLOP/s)", round(tf, 2),
               "TFLOP/s", args, ms, "bf16",
               {"workload": "C3 causal attention bwd + RoPE(1e4), B4 H16 S2048 D128",
                "batch": B, "heads": H, "seq_len": S, "head_dim": D},
               {"kernel": "gn_attn_bwd (pre-pass + dK/dV + dQ kernels)", "bound": "mfma",
                "achieved": round(tf, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tf / BF16_PEAK_TFLOPS, 4), "traffic": None}, cpu)
    # the forward that produces the saved O and LSE (RoPE rotation + attn_fwd_mfma)
    fo = (torch.empty_like(Q), torch.empty(B, H, S, device=dev))
    def fwd():
        gn._check(gn.lib().gn_attn_fwd(gn._ptr(Q), gn._ptr(K), gn._ptr(V), gn._ptr(fo[0]),
                                       gn._ptr(fo[1]), B, H, S, D, D ** -0.5, 1, gn.ROPE["interleaved"],
                                       1e4, gn.BF16, gn._ptr(ws), ws.numel(), gn._stream()),
                  "gn_attn_fwd")
    ms_f = timed(torch, fwd, args.steps, args.warmup)
    ff = 2 * 2.0 * S * S * D * 0.5 * B * H  # causal: QK^T and PV over half the scores
    out["forward"] = {"kernel": "gn_attn_fwd (RoPE rotation + attn_fwd_mfma)", "ms": round(ms_f, 4),
                      "TFLOP/s": round(ff / (ms_f * 1e-3) / 1e12, 1),
                      "frac": round(ff / (ms_f * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)}
    return out


def bench_vsa(args, torch, gn):
    """VSA unpack-project dW/db (fp32 dY, two-term bf16 split) + surrogate bwd."""
    Bn, D, O, K = 8192, 10240, 768, 4
    words = D // 32
    dev = torch.device("cuda:0")
    r = np.random.default_rng(4)
    bits = gn.u32_tensor(r.integers(0, 2**32, size=(Bn, words), dtype=np.uint64).astype(np.uint32), dev)
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    dY = torch.randn(Bn, O, device=dev, generator=g)
    dW = torch.empty(O, D, device=dev)
    db = torch.empty(O, device=dev)
    ws = gn.workspace(gn.vsa_workspace_bytes(Bn, O), dev)
    ms = timed(torch, lambda: gn.vsa_unpack_project_bwd(dY, bits, D, dW=dW, db=db, ws=ws),
               args.steps, args.warmup)
    flops = 2.0 * O * D * Bn
    tf = flops / (ms * 1e-3) / 1e12
    preds = torch.randn(Bn, K, D, device=dev, generator=g)
    res_np, w_np = np.zeros((Bn, 4), np.uint32), np.full((Bn, K), 1.0 / K, np.float32)
    res_np[:, 1] = 1
    res = gn.u32_tensor(res_np, dev)
    wts = torch.from_numpy(w_np).to(dev)
    dP = torch.empty_like(preds)
    ms_s = timed(torch, lambda: gn.vsa_surrogate_bwd(preds, bits, res, wts, dPreds=dP),
                 args.steps, args.warmup)
    bytes_s = 2.0 * Bn * K * D * 4 + Bn * words * 4
    gbs = bytes_s / (ms_s * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        import oracle
        Bs = 4096  # half the rows: about 8 s of the oracle on the host
        bh = r.integers(0, 2**32, size=(Bs, words), dtype=np.uint64).astype(np.uint32)
        dy = r.standard_normal((Bs, O)).astype(np.float32)
        t0 = time.perf_counter()
        oracle.vsa_unpack_project_bwd(dy, bh, D)
        dt = time.perf_counter() - t0
        cpu = {"value": round(2.0 * O * D * Bs / dt / 1e12, 6), "unit": "TFLOP/s",
               "cores": oracle.num_threads(), "kind": "port",
               "sample": f"{Bs} of {Bn} rows of the dW contraction (oracle C/OpenMP fp64), {dt:.2f} s"}
    out = line("VSA unpack-project dW backward (algorithmic TFLOP/s)", round(tf, 2), "TFLOP/s",
               args, ms, "f32 (bf16x2 split MFMA)",
               {"workload": "C4 VSA unpack-project bwd: 8192 x 10240 bits -> 768, fp32 dY",
                "rows": Bn, "vsa_dim": D, "out_dim": O},
               {"kernel": "gn_vsa_unpack_project_bwd (dY split + vsa_dw_dma + db)", "bound": "mfma",
                "achieved": round(tf, 1),
                "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                "traffic": None}, cpu)
    out["surrogate_bwd"] = {"ms": round(ms_s, 4), "GB/s": round(gbs, 1),
                            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "K": K,
                            "bytes": bytes_s}
    return out


def bench_mlp(args, torch, gn):
    """MLP 784->256->10 fp32, batch 64, ReLU, CE, one backward through the tape."""
    import grilly_core
    import grilly_bridge as gb
    dev = torch.device("cuda:0")
    r = np.random.default_rng(1)
    Bsz = 64
    lim1, lim2 = np.sqrt(6 / (784 + 256)), np.sqrt(6 / (256 + 10))
    t = lambda a, dt=torch.float32: torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dt)
    X = t(r.standard_normal((Bsz, 784)).astype(np.float32))
    y = t(r.integers(0, 10, Bsz).astype(np.int32), torch.int32)
    W1 = t(r.uniform(-lim1, lim1, (256, 784)).astype(np.float32))
    W2 = t(r.uniform(-lim2, lim2, (10, 256)).astype(np.float32))
    b1, b2 = torch.zeros(256, device=dev), torch.zeros(10, device=dev)
    Z = (X @ W1.t() + b1).contiguous()
    Hh = torch.relu(Z).contiguous()
    L = (Hh @ W2.t() + b2).contiguous()
    loss = torch.zeros(1, device=dev)
    device = grilly_core.Device(0)
    gb.attach_torch_stream(device)
    tape = gb.create_tape_context(device)

    def step():
        tape.begin()
        n1 = tape.record_op(grilly_core.OpType.Linear, [gb.tref(X)], [gb.tref(Z)])
        tape.save_for_backward(n1, [W1.data_ptr(), b1.data_ptr()])
        tape.record_op(grilly_core.OpType.ReLU, [gb.tref(Z, True)], [gb.tref(Hh)])
        n3 = tape.record_op(grilly_core.OpType.Linear, [gb.tref(Hh, True)], [gb.tref(L)])
        tape.save_for_backward(n3, [W2.data_ptr(), b2.data_ptr()])
        ce = tape.record_op(grilly_core.OpType.CrossEntropy, [gb.tref(L, True), gb.tref(y)],
                            [gb.tref(loss)], gb.cross_entropy_params(1.0))
        tape.backward(ce, 0)
        tape.end()
    ms = timed(torch, step, args.steps, args.warmup)
    flops = 2.0 * Bsz * (784 * 256 + 256 * 10 + 256 * 10)
    cpu = None
    if not args.no_cpu:
        h = lambda a: a.cpu().numpy()
        cpu = mlp_cpu_baseline(h(X), h(y), h(W1), h(W2), h(Z), h(Hh), h(L))
    return line("MLP tape backward step time (784-256-10, B=64, fp32)", round(ms * 1e3, 2), "us",
                args, ms, "f32",
                {"workload": "C1 MLP 784->256->10 fp32 B=64: CE, 2x linear, ReLU bwd via the tape",
                 "batch": Bsz},
                {"kernel": "whole step (launch-bound)", "bound": "latency",
                 "achieved": round(flops / (ms * 1e-3) / 1e12, 4), "peak": 157.3, "unit": "TFLOP/s",
                 "frac": round(flops / (ms * 1e-3) / 1e12 / 157.3, 6), "traffic": None}, cpu,
                higher=False)


def mlp_cpu_baseline(X, y, W1, W2, Z, H, L):
    """The same C1 backward (CE with scale 1, Linear 2 with dX, ReLU, Linear 1 without dX) on
    the oracle (C, OpenMP), timed on this host: median of 200 steps after 20 warm-up steps."""
    import oracle

    def step():
        dL = oracle.xent_bwd(L, y, 1.0)
        dH, _, _ = oracle.linear_bwd(dL, H, W2)
        dZ = oracle.act_bwd("relu", dH, Z)
        oracle.linear_bwd(dZ, X, W1, need_dx=False)

    for _ in range(20):
        step()
    ts = []
    for _ in range(200):
        t0 = time.perf_counter()
        step()
        ts.append(time.perf_counter() - t0)
    us = float(np.median(ts)) * 1e6
    return {"value": round(us, 2), "unit": "us", "cores": oracle.num_threads(), "kind": "port",
            "sample": "the whole B=64 step (oracle C/OpenMP, fp64 accumulation), median of 200 "
                      "after 20 warm-up steps"}


def bench_decoder(args, torch, gn):
    """12-layer decoder (d 768, 12 heads, GEGLU 3072, tied embedding 32000),
    batch 8 x seq 1024, bf16; one step = tape begin / record / backward / end."""
    import grilly_core
    import grilly_bridge as gb
    from decoder_tape import Decoder
    m = Decoder()
    m.forward()
    device = grilly_core.Device(0)
    gb.attach_torch_stream(device)
    tape = gb.create_tape_context(device)
    ms = timed(torch, lambda: m.backward_step(tape), args.steps, args.warmup)
    tf = m.flops() / (ms * 1e-3) / 1e12
    opt = decoder_optimizer_step(torch, gn, m)
    # the forward that produces the saved tensors (norm/linear/GLU/attention forward kernels)
    fwd_ms = timed(torch, m.forward, 5, 1)
    fwd_tf = m.fwd_flops() / (fwd_ms * 1e-3) / 1e12
    cpu = None
    if not args.no_cpu:
        cpu = decoder_cpu_baseline(m)
    out = line("12-layer decoder backward tokens/s (end-to-end tape backward)",
                round(m.T / (ms * 1e-3), 1), "tokens/s", args, ms, "bf16",
                {"workload": "C5 12-layer decoder bwd: d768 H12 LN, fused QKV, causal attention, "
                             "GEGLU 3072, tied embedding 32000 + CE; B8 x S1024, bf16",
                 "tokens": m.T, "layers": m.L, "d_model": m.d, "heads": m.H, "ff": m.ff,
                 "vocab": m.V, "parallelism": "none (1 GPU)"},
                {"kernel": "whole step (GEMMs, attention, norms, CE, adds)", "bound": "mfma",
                 "achieved": round(tf, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                 "frac": round(tf / BF16_PEAK_TFLOPS, 4), "traffic": None,
                 "flops_per_step": m.flops()}, cpu)
    out["optimizer_step"] = opt
    out["forward"] = {"kernel": "Decoder.forward (gn_layernorm_fwd, gn_linear_fwd, "
                                "gn_glu_linear_fwd, gn_attn_fwd; torch gather and adds)",
                      "ms": round(fwd_ms, 4), "TFLOP/s": round(fwd_tf, 1),
                      "frac": round(fwd_tf / BF16_PEAK_TFLOPS, 4), "flops": m.fwd_flops()}
    return out


def decoder_optimizer_step(torch, gn, m):
    """AdamW after the backward over every decoder weight (fp32 masters, m, v, fp32 gradients,
    bf16 copies written back): one gn_adamw_step call, HIP-event timed, gradients kept (the
    tape releases them at end()).  Bytes per element: read W, g, m, v (16) + write W, m, v
    (12) + bf16 W (2) = 30."""
    ws = [m.E] + [w for p in m.layers for w in p.values()] + [m.lnf_g, m.lnf_b]
    n = sum(w.numel() for w in ws)
    ent = []
    for w in ws:
        f = w.float().contiguous()
        ent.append(dict(W=f, grad=torch.randn_like(f) * 1e-3, state0=torch.zeros_like(f),
                        state1=torch.zeros_like(f), W_bf16=torch.empty_like(w)))
    def step():
        gn.adamw_step(ent, lr=1e-4, weight_decay=0.01, step=1, clear_grad=False)
    ms = timed(torch, step, 10, 3)
    byts = 30.0 * n
    gbs = byts / (ms * 1e-3) / 1e9
    return {"kernel": "adamw_kernel (gn_adamw_step, %d tensors)" % len(ws), "params": n,
            "ms": round(ms, 4), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "bytes": byts}


def decoder_cpu_baseline(m):
    """Oracle (C, OpenMP, fp64 accumulation) on one layer's backward at full size, scaled
    to 12 layers plus the LM head by FLOPs (the head timed as its share of the layer)."""
    import oracle
    T, d, ff, H, B, S = m.T, m.d, m.ff, m.H, m.B, m.S
    D = d // H
    r = np.random.default_rng(5)
    f = lambda *s: r.standard_normal(s).astype(np.float32)
    x, dY = f(T, d), (f(T, d) * 1e-2).astype(np.float32)
    g1 = np.ones(d, np.float32)
    Wqkv, Wo, Wg, Wu, Wd = (f(3 * d, d) * 0.02, f(d, d) * 0.02, f(ff, d) * 0.02, f(ff, d) * 0.02,
                            f(d, ff) * 0.02)
    n1, m1, r1 = oracle.layernorm_fwd(x, g1)
    qkv = oracle.linear_fwd(n1, Wqkv)
    q, k, v = (np.ascontiguousarray(t) for t in qkv.reshape(B, S, 3, H, D).transpose(2, 0, 3, 1, 4))
    o, lse = oracle.attn_fwd(q, k, v, causal=True, rope_mode="none")
    o2 = np.ascontiguousarray(o.transpose(0, 2, 1, 3).reshape(T, d))
    n2, m2, r2 = oracle.layernorm_fwd(x, g1)
    gate, up = oracle.linear_fwd(n2, Wg), oracle.linear_fwd(n2, Wu)
    h = oracle.glu_fwd("geglu_up", gate, up)
    t0 = time.perf_counter()
    dH, _, _ = oracle.linear_bwd(dY, h, Wd)
    dG, dU = oracle.glu_bwd("geglu_up", dH, gate, up)
    dN2 = oracle.linear_bwd(dG, n2, Wg)[0] + oracle.linear_bwd(dU, n2, Wu)[0]
    oracle.layernorm_bwd(dN2, x, g1, m2, r2)
    dO2, _, _ = oracle.linear_bwd(dY, o2, Wo)
    dO4 = np.ascontiguousarray(dO2.reshape(B, S, H, D).transpose(0, 2, 1, 3))
    oracle.attn_bwd(q, k, v, dO4, lse, causal=True, rope_mode="none")
    dQKV = (f(T, 3 * d) * 1e-2).astype(np.float32)  # the layout change back is not timed work
    dN1, _, _ = oracle.linear_bwd(dQKV, n1, Wqkv)
    oracle.layernorm_bwd(dN1, x, g1, m1, r1)
    dt = time.perf_counter() - t0
    layer_flops = (m.flops() - 2 * 2 * T * d * m.V) / m.L
    step_s = dt * (m.L + 2 * 2 * T * d * m.V / layer_flops)
    return {"value": round(T / step_s, 2), "unit": "tokens/s", "cores": oracle.num_threads(),
            "kind": "port",
            "sample": f"one full-size layer backward (T={T}) on the oracle (C/OpenMP, fp64 "
                      f"accumulation), {dt:.1f} s, scaled by FLOPs to {m.L} layers + LM head"}


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
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the backward "
              "path has no multi-GPU code in this build", file=sys.stderr)
        sys.exit(2)
    import torch
    import gn_bwd as gn
    gn.lib()
    if args.ceilings:
        print(json.dumps(ceilings(torch, gn)))
        return
    if args.workload != "ffn":
        fn = {"attn": bench_attn, "vsa": bench_vsa, "mlp": bench_mlp,
              "decoder": bench_decoder}[args.workload]
        print(json.dumps(fn(args, torch, gn)))
        return
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
    if args.calib_copy:
        calib_copy(torch, gn)
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
                     "launch_ms": round(dom_ms, 4), "traffic": traffic_from_profile(),
                     "algorithmic_bytes": 2 * (2 * T * HID + 2 * HID * DM) + 2 * T * DM},
        "cpu_baseline": cpu,
        "wall_s": round(wall, 3),
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
