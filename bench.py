"""Benchmark: transformer FFN block backward on one MI355X.

Workload: RMSNorm(d=2048) -> SwiGLU (gate/up 2048->5632, down 5632->2048), T = 4096 tokens
(batch 4 x seq 1024), bf16 activations/weights, fp32 accumulation; x ~ N(0,1), weights
N(0, 0.02), dY ~ N(0, 1e-2).  One step = the whole block backward:
    gn_ffn_down_glu_bwd  (down projection with the SwiGLU backward in its epilogue: dG|dU, dWd)
    gn_glu_proj_bwd      (dN = dG Wg + dU Wu, dWg, dWu)
    gn_rmsnorm_bwd       (dx, dw)
with inputs (x, saved rstd / gate / up / activations, weights, dY) resident in HBM.
The metric is layer-backward tokens/s; the dominant call's roofline fraction comes from
HIP events around that call inside every timed step (the per-call breakdown from a pass
before the timed region, so the timed steps carry one event pair only), and the CPU
baseline is a numpy fp32 restatement of the reference's CPU path (oracle/cpu_ref.py) timed
on a bounded token sample of the same workload on this host; the C oracle's timing is
reported apart (cpu_oracle).

Other BASELINE configs (parity-tested, measured with --workload):
    attn  configs[2]: causal attention backward with RoPE, B4 H16 S2048 D128, bf16
    attn32 the same shape in fp32 (the reference's dtype) on the generic matrix-core kernels
    vsa   configs[3]: VSA unpack-project dW (8192 x 10240 bits -> 768, fp32 dY) and the
          surrogate-loss backward (K = 4)
    mlp   configs[0]: MLP 784->256->10 fp32 B=64 through the tape engine (grilly_core)
    decoder configs[4]: 12-layer decoder (d 768, GEGLU, tied embedding 32000, CE), B8 x S1024,
          end-to-end backward through the tape engine
    hyper the reference's VSA hypernetwork training step (grilly_core.vsa_training_step) at
          its defaults (K 16, 1.0 GB output layer), batch 1
    linear32 fp32 Linear backward at the hypernetwork's output layer, batch 64
          (1536 -> 163840), on the six-product bf16 MFMA path (fp32-grade)
Each prints one JSON line of the same shape; the default (ffn) is the headline metric.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
                       [--workload ffn|attn|attn32|vsa|mlp|decoder|hyper|linear32]
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
FP32_PEAK_TFLOPS = 157.3  # dense fp32 MFMA (v_mfma_f32_32x32x2_f32)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--cpu-tokens", type=int, default=T)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--workload", default="ffn",
                   choices=["ffn", "attn", "attn32", "vsa", "mlp", "decoder", "hyper", "linear32"])
    p.add_argument("--calib-copy", action="store_true",
                   help="after the timed region, launch one gn_add_inplace over 2^28 floats "
                        "(reads 2 GiB, writes 1 GiB): the reference dispatch that sizes the "
                        "L2 read requests of a --pmc run and checks its write requests")
    p.add_argument("--ceilings", action="store_true",
                   help="measure this box's MFMA (bf16 32x32x16 loop) and HBM (16-byte copy) "
                        "ceilings with the library's probe kernels and print them as JSON")
    p.add_argument("--pmc-summary", nargs=2, metavar=("READ_DIR", "WRITE_DIR"),
                   help="summarise two rocprofv3 --pmc runs of 'bench.py --calib-copy' (read "
                        "requests: TCC_EA0_RDREQ_sum TCC_EA0_RDREQ_32B_sum TCC_BUBBLE_sum; write "
                        "requests: TCC_EA0_WRREQ_sum TCC_EA0_WRREQ_64B_sum) into the HBM traffic "
                        "of the dominant kernel")
    p.add_argument("--pmc-sq", metavar="DIR",
                   help="summarise a rocprofv3 --pmc run of SQ_INSTS_VALU SQ_INSTS_MFMA "
                        "SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE per kernel (VALU instructions "
                        "per MFMA, MFMA busy share of the SIMD cycles)")
    p.add_argument("--pmc-call", default=DOMINANT_CALL, choices=sorted(CALL_KERNELS),
                   help="the FFN step's call whose launches --pmc-summary adds up (default: the "
                        "headline's dominant call, the [dWg;dWu] weight-gradient GEMM)")
    return p.parse_args()


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "ffn_dominant_gemm_hbm_traffic.txt")
# The launches of the FFN step's two largest calls as rocprof names them: (kernel pattern,
# work-items per dispatch).  [dWg;dWu] (transposed A, fp32 C) and dN run one launch each on
# 256 x 128 tiles with three LDS stages and four producer waves (512 threads per block):
# 704 and 256 blocks.
CALL_KERNELS = {
    "[dWg;dWu]": [(r"gemm_core<true, false, float, 256, 128, 0, 3, false, 4>", 704 * 512)],
    "dN": [(r"gemm_core<false, false, unsigned short, 256, 128, 0, 3, false, 4>", 256 * 512)],
}
DOMINANT_CALL = "[dWg;dWu]"
CALIB_FLOATS = 1 << 28


def calib_copy(torch, gn):
    x = torch.ones(CALIB_FLOATS, device="cuda:0")
    y = torch.zeros(CALIB_FLOATS, device="cuda:0")
    torch.cuda.synchronize()
    gn.add_inplace(y, x)
    torch.cuda.synchronize()


def pmc_summary(read_dir, write_dir, call):
    """HBM traffic per call of `call` (CALL_KERNELS) from the L2 -> memory request counters,
    summed over every TCC instance of the 8 XCDs (two --pmc passes of the same command):
      reads:  TCC_EA0_RDREQ_sum (all read requests), TCC_EA0_RDREQ_32B_sum, TCC_BUBBLE_sum (the
              128-byte ones as gfx950 documents them); an ordinary request's size is calibrated
              on the add of --calib-copy, which reads exactly 2 GiB;
      writes: TCC_EA0_WRREQ_sum, TCC_EA0_WRREQ_64B_sum (64-byte ones, the rest 32 bytes),
              scaled by the add's 1 GiB over what the same formula counts for it (1, 1/2 or
              1/3 on the boxes seen: their summed counters read every request once, twice or
              three times, and the read calibration scales the same way).
    Each launch's per-dispatch mean is summed over the call's launches."""
    import csv
    import glob
    import re

    def load(d):
        out = {}
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(path)):
                key = (r["Kernel_Name"], int(float(r["Grid_Size"])), r["Dispatch_Id"])
                out.setdefault(key, {}).setdefault(r["Counter_Name"], 0.0)
                out[key][r["Counter_Name"]] += float(r["Counter_Value"])
        return out

    def mean(tab, pat, grid, counters):
        rows = [v for (k, g, _), v in tab.items() if re.search(pat, k) and (grid is None or g == grid)]
        if not rows:
            raise SystemExit(f"no dispatch of {pat} (grid {grid})")
        return len(rows), {c: sum(r.get(c, 0.0) for r in rows) / len(rows) for c in counters}

    rd = ("TCC_EA0_RDREQ_sum", "TCC_EA0_RDREQ_32B_sum", "TCC_BUBBLE_sum")
    wr = ("TCC_EA0_WRREQ_sum", "TCC_EA0_WRREQ_64B_sum")
    R, W = load(read_dir), load(write_dir)
    _, ca = mean(R, "add_kernel", None, rd)
    plain = ca[rd[0]] - ca[rd[1]] - ca[rd[2]]
    bytes_per_req = (2.0 * CALIB_FLOATS * 4 - 32 * ca[rd[1]] - 128 * ca[rd[2]]) / plain
    rbytes = lambda c: (c[rd[0]] - c[rd[1]] - c[rd[2]]) * bytes_per_req + 32 * c[rd[1]] + 128 * c[rd[2]]
    wcount = lambda c: (c[wr[0]] - c[wr[1]]) * 32 + 64 * c[wr[1]]
    _, cw = mean(W, "add_kernel", None, wr)
    wscale = CALIB_FLOATS * 4 / wcount(cw)
    wbytes = lambda c: wcount(c) * wscale
    lines = [f"call: {call}",
             f"reads: calibration add {ca[rd[0]]:.0f} requests ({ca[rd[1]]:.0f} of 32 B, {ca[rd[2]]:.0f} "
             f"of 128 B) for 2 GiB -> {bytes_per_req:.1f} B per ordinary request",
             f"writes: calibration add {cw[wr[0]]:.0f} requests ({cw[wr[1]]:.0f} of 64 B) count "
             f"{wcount(cw) / 2**30:.4f} GiB for the 1 GiB it writes -> write counts scaled by {wscale:.4f}"]
    total = 0.0
    for pat, grid in CALL_KERNELS[call]:
        n, c = mean(R, pat, grid, rd)
        _, w = mean(W, pat, grid, wr)
        rb, wb = rbytes(c), wbytes(w)
        total += rb + wb
        lines.append(f"  {pat.split('[')[0].rstrip('>')}> grid {grid}: {c[rd[0]]:.0f} read requests "
                     f"({c[rd[1]]:.0f} of 32 B, {c[rd[2]]:.0f} of 128 B) -> {rb / 1e6:.1f} MB read; "
                     f"{w[wr[0]]:.0f} write requests ({w[wr[1]]:.0f} of 64 B) -> {wb / 1e6:.1f} MB "
                     f"written; mean over {n} dispatches")
    lines.append(f"traffic_bytes_per_call: {total:.0f}")
    print("\n".join(lines))


def pmc_sq_summary(d, xcds=8, cus=256, simds=4):
    """Per gn:: kernel, per dispatch means of the four counters and two ratios:
    VALU / MFMA instructions, and MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / XCDs x
    CUs x SIMDs per CU): the share of SIMD cycles the matrix cores are busy while the kernel
    runs.  On gfx950 SQ_VALU_MFMA_BUSY_CYCLES reads 32 cycles per v_mfma_f32_32x32x16_bf16 (its
    issue cost at the dense peak) and GRBM_GUI_ACTIVE is summed over the 8 XCDs."""
    import csv
    import glob
    tab = {}
    for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(path)):
            k = r["Kernel_Name"]
            if "gn::" not in k:
                continue
            ent = tab.setdefault(k, {}).setdefault(r["Dispatch_Id"], {})
            ent[r["Counter_Name"]] = ent.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    rows = []
    for k, disp in tab.items():
        n = len(disp)
        mean = lambda c: sum(v.get(c, 0.0) for v in disp.values()) / n
        valu, mfma = mean("SQ_INSTS_VALU"), mean("SQ_INSTS_MFMA")
        busy, gui = mean("SQ_VALU_MFMA_BUSY_CYCLES"), mean("GRBM_GUI_ACTIVE")
        rows.append((k, n, valu, mfma, valu / mfma if mfma else float("nan"),
                     busy / (gui / xcds * cus * simds) if gui else float("nan")))
    rows.sort(key=lambda r: -r[3])
    print("# dispatches  VALU_insts  MFMA_insts  VALU/MFMA  MFMA_busy  kernel")
    for k, n, valu, mfma, ratio, busy in rows:
        print(f"{n:6d} {valu:14.4g} {mfma:12.4g} {ratio:9.2f} {100 * busy:9.1f}%  {k[:110]}")


def ceilings(torch, gn):
    """Measured ceilings: gn_probe_mfma (no memory traffic) and gn_probe_copy (2 GiB, every
    access mode; the best copy and the read-only stream are reported)."""
    import ctypes
    gn.lib()
    # the probes live in their own library next to libgn_bwd.so (not part of the backward ABI)
    lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.abspath(gn.__file__)), "libgn_probe.so"))
    lib.gn_probe_mfma.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.gn_probe_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                  ctypes.c_void_p]
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
    modes = {}
    for mode, name in ((0, "copy_nt_x4"), (1, "copy_x4"), (2, "copy_x8"), (3, "read_nt_x8")):
        ms = timed(torch, lambda: gn._check(lib.gn_probe_copy(dst.data_ptr(), src.data_ptr(), nbytes,
                                                              mode, s), "gn_probe_copy"), 10, 3)
        moved = (2.0 if mode < 3 else 1.0) * nbytes
        modes[name] = round(moved / (ms * 1e-3) / 1e9, 1)
    best_copy = max(v for k, v in modes.items() if k.startswith("copy"))
    return {"mfma_bf16_tflops": round(flops / (mf * 1e-3) / 1e12, 1),
            "mfma_spec_tflops": BF16_PEAK_TFLOPS, "copy_gbs": best_copy,
            "read_gbs": modes["read_nt_x8"], "copy_modes_gbs": modes, "hbm_spec_gbs": HBM_PEAK_GBS,
            "probe": f"gn_probe_mfma {blocks} blocks x {iters} x 8 MFMA per wave; "
                     f"gn_probe_copy {nbytes >> 30} GiB per mode (copies: read + written)"}


def traffic_from_profile(call):
    """HBM bytes per call of `call` from the committed counter summary (None when the summary
    covers another call or is missing)."""
    try:
        lines = open(TRAFFIC_FILE).read().splitlines()
    except OSError:
        return None
    if f"call: {call}" not in lines:
        return None
    for l in lines:
        if l.startswith("traffic_bytes_per_call:"):
            return int(float(l.split(":", 1)[1]))
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


def attn_cpu_baseline(args, S, D, BH):
    """The reference's CPU attention backward (numpy fp32, P materialised) on 8 heads."""
    if args.no_cpu:
        return None
    from oracle import cpu_ref
    r = np.random.default_rng(3)
    Hs = 8  # 8 of the B*H heads: P is S x S fp32 per head
    q, k, v = (r.standard_normal((Hs, S, D)).astype(np.float32) for _ in range(3))
    do = (r.standard_normal((Hs, S, D)) * 1e-2).astype(np.float32)
    nt = cpu_ref.threads()
    with cpu_ref.limit_threads(nt):
        cpu_ref.attention_step(q[:1], k[:1], v[:1], do[:1], D ** -0.5)
        t0 = time.perf_counter()
        cpu_ref.attention_step(q, k, v, do, D ** -0.5)
        dt = time.perf_counter() - t0
    return {"value": round(5 * 2.0 * S * S * D * 0.5 * Hs / dt / 1e12, 5), "unit": "TFLOP/s",
            "cores": nt, "kind": "port",
            "sample": f"{Hs} of {BH} heads at S={S}, numpy fp32 with P materialised (the "
                      f"reference's CPU path, autograd_core.py:617-654; no RoPE there), "
                      f"{dt:.2f} s; algorithmic causal FLOPs", "cpu_model": cpu_ref.cpu_model()}


def bench_attn32(args, torch, gn):
    """configs[2]'s shape with fp32 tensors (the reference's own dtype): causal attention
    backward with RoPE, B4 H16 S2048 D128, on the generic matrix-core kernels (two-piece bf16
    split, three products per product)."""
    B, H, S, D = 4, 16, 2048, 128
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    Q, K, V = (torch.randn(B, H, S, D, device=dev, generator=g) for _ in range(3))
    dO = torch.randn(B, H, S, D, device=dev, generator=g) * 1e-2
    ws = gn.workspace(gn.attn_workspace_bytes(B, H, S, D, gn.F32), dev)
    O, LSE = gn.attn_fwd(Q, K, V, causal=True, rope="interleaved", ws=ws)
    out = (torch.empty_like(Q), torch.empty_like(K), torch.empty_like(V))
    ms = timed(torch, lambda: gn.attn_bwd(Q, K, V, O, dO, LSE, causal=True, rope="interleaved",
                                          ws=ws, out=out), args.steps, args.warmup)
    flops = 5 * 2.0 * S * S * D * 0.5 * B * H  # causal, algorithmic (5 GEMMs)
    tf = flops / (ms * 1e-3) / 1e12
    out = line("causal attention backward with RoPE, fp32 (algorithmic TFLOP/s)", round(tf, 2),
               "TFLOP/s", args, ms, "f32 (bf16x2 split on MFMA, 3 products)",
               {"workload": "C3 shape in fp32: causal attention bwd + RoPE(1e4), B4 H16 S2048 D128",
                "batch": B, "heads": H, "seq_len": S, "head_dim": D},
               {"kernel": "gn_attn_bwd fp32 (split pre-pass + attn_bwd_gen dK/dV and dQ + "
                          "un-rotating conversion)", "bound": "mfma",
                "achieved": round(tf, 1), "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tf / FP32_PEAK_TFLOPS, 4), "traffic": None,
                "note": "peak = dense fp32 MFMA; the kernels issue 3 bf16 MFMA products per fp32 "
                        "product and 7 products for the algorithmic 5 (the dQ pass recomputes S "
                        f"and dP): {tf * 3 * 7 / 5:.0f} TFLOP/s of bf16 MFMA work issued"},
               attn_cpu_baseline(args, S, D, B * H))
    return out


def bench_attn(args, torch, gn):
    """causal attention backward with RoPE (theta 1e4), B4 H16 S2048 D128."""
    B, H, S, D = 4, 16, 2048, 128
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    bf = torch.bfloat16
    Q, K, V = (torch.randn(B, H, S, D, device=dev, generator=g).to(bf) for _ in range(3))
    dO = (torch.randn(B, H, S, D, device=dev, generator=g) * 1e-2).to(bf)
    ws = gn.workspace(gn.attn_workspace_bytes(B, H, S, D, gn.BF16), dev)
    O, LSE = gn.attn_fwd(Q, K, V, causal=True, rope="interleaved", ws=ws)
    out = (torch.empty_like(Q), torch.empty_like(K), torch.empty_like(V))
    ms = timed(torch, lambda: gn.attn_bwd(Q, K, V, O, dO, LSE, causal=True, rope="interleaved",
                                          ws=ws, out=out), args.steps, args.warmup)
    flops = 5 * 2.0 * S * S * D * 0.5 * B * H  # causal, algorithmic (5 GEMMs)
    tf = flops / (ms * 1e-3) / 1e12
    cpu = attn_cpu_baseline(args, S, D, B * H)
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
        from oracle import cpu_ref
        Bs = 2048  # a quarter of the rows
        bh = r.integers(0, 2**32, size=(Bs, words), dtype=np.uint64).astype(np.uint32)
        dy = r.standard_normal((Bs, O)).astype(np.float32)
        nt = cpu_ref.threads()
        with cpu_ref.limit_threads(nt):
            t0 = time.perf_counter()
            cpu_ref.vsa_unpack_project_backward(dy, bh, D)
            dt = time.perf_counter() - t0
        cpu = {"value": round(2.0 * O * D * Bs / dt / 1e12, 5), "unit": "TFLOP/s", "cores": nt,
               "kind": "port",
               "sample": f"{Bs} of {Bn} rows: unpack to +-1 and dY^T S in numpy fp32 (the shader's "
                         f"formula in the reference's numpy style), {dt:.2f} s",
               "cpu_model": cpu_ref.cpu_model()}
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

    def record():
        n1 = tape.record_op(grilly_core.OpType.Linear, [gb.tref(X)], [gb.tref(Z)])
        tape.save_for_backward(n1, [W1.data_ptr(), b1.data_ptr()])
        tape.record_op(grilly_core.OpType.ReLU, [gb.tref(Z, True)], [gb.tref(Hh)])
        n3 = tape.record_op(grilly_core.OpType.Linear, [gb.tref(Hh, True)], [gb.tref(L)])
        tape.save_for_backward(n3, [W2.data_ptr(), b2.data_ptr()])
        return tape.record_op(grilly_core.OpType.CrossEntropy, [gb.tref(L, True), gb.tref(y)],
                              [gb.tref(loss)], gb.cross_entropy_params(1.0))

    def step():
        tape.begin()
        tape.backward(record(), 0)
        tape.end()
    ms = timed(torch, step, args.steps, args.warmup)
    # the graph comparison: both forms over 200 launch-bound steps
    reps = max(args.steps, 200)
    eager_reps = timed(torch, step, reps, reps // 10)
    graph = graph_replay(torch, grilly_core, device, tape, record, args, eager_reps, reps)
    flops = 2.0 * Bsz * (784 * 256 + 256 * 10 + 256 * 10)
    cpu = None
    if not args.no_cpu:
        h = lambda a: a.cpu().numpy()
        cpu = mlp_cpu_baseline(h(X), h(y), h(W1), h(W2), h(Z), h(Hh), h(L))
    out = line("MLP tape backward step time (784-256-10, B=64, fp32)", round(ms * 1e3, 2), "us",
               args, ms, "f32",
               {"workload": "C1 MLP 784->256->10 fp32 B=64: CE, 2x linear, ReLU bwd via the tape",
                "batch": Bsz},
               {"kernel": "whole step (launch-bound)", "bound": "latency",
                "achieved": round(flops / (ms * 1e-3) / 1e12, 4), "peak": 157.3, "unit": "TFLOP/s",
                "frac": round(flops / (ms * 1e-3) / 1e12 / 157.3, 6), "traffic": None}, cpu,
               higher=False)
    out["with_graph"] = graph
    return out


def graph_replay(torch, grilly_core, device, tape, record, args, eager_ms, reps=None):
    """The same backward captured once into a HIP graph (grilly_core.OpGraph, the replacement
    of the reference's OpGraph) and replayed: one hipGraphLaunch per step in place of the tape
    walk (begin / record / backward / end) and its per-kernel launches.  Same kernels, same
    buffers, same work per step.  reps: replays timed (a launch-bound step needs more than
    --steps for a stable mean; the eager figure it is compared with is then re-timed over the
    same count)."""
    steps = reps or args.steps
    warm = max(args.warmup, steps // 10)
    g = grilly_core.OpGraph()
    tape.begin()
    g.capture_backward(tape, record(), 0)
    tape.end()
    g.optimize(device)
    ms = timed(torch, lambda: g.execute(device), steps, warm)
    counts = g.node_counts()
    g.clear()
    return {"ms_per_step": round(ms, 4), "eager_ms_per_step": round(eager_ms, 4),
            "speedup": round(eager_ms / ms, 3), "kernel_nodes": counts["kernel"],
            "memset_nodes": counts["memset"], "memcpy_nodes": counts["memcpy"], "replays": steps,
            "how": "grilly_core.OpGraph.capture_backward once, then execute() per step, "
                   f"mean over {steps} replays (eager step over the same count)"}


def mlp_cpu_baseline(X, y, W1, W2, Z, H, L):
    """The same C1 backward (CE with scale 1, Linear 2 with dX, ReLU, Linear 1 without dX) in
    numpy fp32 (oracle/cpu_ref.py), timed on this host: median of 200 after 20 warm-up steps."""
    from oracle import cpu_ref
    nt = cpu_ref.threads()
    with cpu_ref.limit_threads(nt):
        for _ in range(20):
            cpu_ref.mlp_step(X, y, W1, W2, Z, H, L)
        ts = []
        for _ in range(200):
            t0 = time.perf_counter()
            cpu_ref.mlp_step(X, y, W1, W2, Z, H, L)
            ts.append(time.perf_counter() - t0)
    us = float(np.median(ts)) * 1e6
    return {"value": round(us, 2), "unit": "us", "cores": nt, "kind": "port",
            "sample": "the whole B=64 step in numpy fp32 (the reference's CPU path, "
                      "autograd_core.py:486-554), median of 200 after 20 warm-up steps",
            "cpu_model": cpu_ref.cpu_model()}


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
    graph = graph_replay(torch, grilly_core, device, tape, lambda: m.record(tape), args, ms)
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
                 "vocab": m.V, "parallelism": "none (1 GPU)",
                 "tape": "set_glu_epilogue(True)" if m.glu_epilogue else "defaults"},
                {"kernel": "whole step (GEMMs, attention, norms, CE, adds)", "bound": "mfma",
                 "achieved": round(tf, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                 "frac": round(tf / BF16_PEAK_TFLOPS, 4), "traffic": None,
                 "flops_per_step": m.flops()}, cpu)
    out["optimizer_step"] = opt
    out["with_graph"] = graph
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
    """One full-size layer's backward in numpy fp32 (oracle/cpu_ref.py: the reference's CPU
    formulas, attention with P materialised), scaled by FLOPs to 12 layers plus the LM head."""
    from oracle import cpu_ref
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
    v1 = (1.0 / r1.astype(np.float64) ** 2 - 1e-5).astype(np.float32)[:, None]
    qkv = oracle.linear_fwd(n1, Wqkv)
    q, k, v = (np.ascontiguousarray(t) for t in qkv.reshape(B, S, 3, H, D).transpose(2, 0, 3, 1, 4))
    q, k, v = (t.reshape(B * H, S, D) for t in (q, k, v))
    gate, up = oracle.linear_fwd(n1, Wg), oracle.linear_fwd(n1, Wu)
    h = oracle.glu_fwd("geglu_up", gate, up)
    o2 = (f(T, d) * 0.1).astype(np.float32)
    nt = cpu_ref.threads()
    with cpu_ref.limit_threads(nt):
        t0 = time.perf_counter()
        dH, _, _ = cpu_ref.linear_backward(dY, h, Wd)
        t = np.tanh(np.float32(np.sqrt(2 / np.pi)) * (up + np.float32(0.044715) * up ** 3))
        gl = 0.5 * up * (1 + t)
        dG = dH * gl
        dU = cpu_ref.gelu_tanh_backward(dH * gate, up)
        dN2 = cpu_ref.linear_backward(dG, n1, Wg)[0] + cpu_ref.linear_backward(dU, n1, Wu)[0]
        cpu_ref.layernorm_backward(dN2, x, g1, m1[:, None], v1)
        dO2, _, _ = cpu_ref.linear_backward(dY, o2, Wo)
        dO4 = np.ascontiguousarray(dO2.reshape(B, S, H, D).transpose(0, 2, 1, 3)).reshape(B * H, S, D)
        cpu_ref.attention_step(q, k, v, dO4, D ** -0.5)
        dQKV = (f(T, 3 * d) * 1e-2).astype(np.float32)  # the layout change back is not timed work
        dN1, _, _ = cpu_ref.linear_backward(dQKV, n1, Wqkv)
        cpu_ref.layernorm_backward(dN1, x, g1, m1[:, None], v1)
        dt = time.perf_counter() - t0
    layer_flops = (m.flops() - 2 * 2 * T * d * m.V) / m.L
    step_s = dt * (m.L + 2 * 2 * T * d * m.V / layer_flops)
    return {"value": round(T / step_s, 2), "unit": "tokens/s", "cores": nt, "kind": "port",
            "sample": f"one full-size layer backward (T={T}) in numpy fp32 (the reference's CPU "
                      f"path, autograd_core.py:486-654, attention with P materialised), {dt:.1f} s, "
                      f"scaled by FLOPs to {m.L} layers + LM head", "cpu_model": cpu_ref.cpu_model()}


def bench_linear32(args, torch, gn):
    """fp32 Linear backward at the hypernetwork's output layer with batch 64: 1536 -> 163840
    (K 16 x vsa 10240), W 1.0 GB.  One step = gn_linear_bwd_ws: dX = dY W (split-K over
    163840), dW = dY^T X (1.0 GB written), db, on the six-product bf16 MFMA path."""
    M, N, K = 64, 163840, 1536
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    dY = torch.randn(M, N, device=dev, generator=g)
    X = torch.randn(M, K, device=dev, generator=g)
    W = torch.randn(N, K, device=dev, generator=g) * 0.02
    dX = torch.empty(M, K, device=dev)
    dW = torch.empty(N, K, device=dev)
    db = torch.empty(N, device=dev)
    ws = gn.workspace(gn.linear_workspace_bytes(M, N, K, 0), dev)
    ms = timed(torch, lambda: gn.linear_bwd(dY, X, W, dX=dX, dW=dW, db=db, ws=ws),
               args.steps, args.warmup)
    byts = 4.0 * (2 * N * K + M * N + 2 * M * K + N)  # W, dW, dY, X, dX, db once each
    gbs = byts / (ms * 1e-3) / 1e9
    flops = 4.0 * M * N * K
    tf = flops / (ms * 1e-3) / 1e12
    out = line("fp32 Linear backward, hypernetwork output layer at batch 64 (GB/s)",
               round(gbs, 1), "GB/s", args, ms, "f32 (bf16x6 split on MFMA)",
               {"workload": "Linear bwd fp32 64 x 1536 -> 163840 (K 16 x vsa 10240): dX, dW, db",
                "M": M, "N": N, "K": K},
               {"kernel": "gn_linear_bwd_ws (dX split-K GEMM + plane sum, dW GEMM, db)",
                "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "bytes": byts}, None)
    out["fp32_work"] = {"flops": flops, "TFLOP/s": round(tf, 1),
                        "vs_fp32_mfma_peak": round(tf / FP32_PEAK_TFLOPS, 3),
                        "fp32_mfma_floor_ms": round(flops / FP32_PEAK_TFLOPS / 1e9, 4),
                        "hbm_floor_ms": round(byts / HBM_PEAK_GBS / 1e6, 4),
                        "note": "a kernel on v_mfma_f32_32x32x2_f32 cannot finish under "
                                "fp32_mfma_floor_ms; the split moves the floor to HBM"}
    return out


def bench_hyper(args, torch, gn):
    """The reference's VSA hypernetwork training step (vsa_training_step, bindings.cpp:
    3140-3286) at its defaults: d_model 768, vsa_dim 10240, K 16, router 32 (W2 = 16 x 10240 x
    1536 fp32 = 1.0 GB), one bitpacked state per step.  One step = upload, forward, loss forward
    (one 64-byte readback, as the reference), backward (the two Linear weights stepped inside
    it), surprise-momentum update of the other parameters, end."""
    import grilly_core as gc
    import grilly_bridge as gb
    dev = gc.Device(0)
    gb.attach_torch_stream(dev)
    d, v, K = 768, 10240, 16
    model = gc.VSAHypernetwork(dev)
    opt = gc.SurpriseMomentumOptimizer(dev, model)
    tape = gc.TapeContext(dev)
    rng = np.random.RandomState(42)
    state = rng.randint(0, 2 ** 32, size=v // 32, dtype=np.uint32)
    delta = rng.randint(0, 2 ** 32, size=v // 32, dtype=np.uint32)
    ms = timed(torch, lambda: gc.vsa_training_step(dev, tape, model, state, delta, opt),
               args.steps, args.warmup)
    # the same step composed call by call with HIP events between the phases.  The two Linear
    # weights take their surprise-momentum step inside their backward pass (read W, s_bar;
    # write W, s_bar; dW never stored); the optimizer pass updates the other four.
    sizes = model.parameter_sizes()
    n_upd = sizes[0] + sizes[1] + sizes[3] + sizes[5]
    phases = [("forward: unpack-project, Linear 768->1536, GELU, Linear 1536->163840 (skinny fp32)",
               4.0 * (sizes[0] + sizes[2] + sizes[4]) + 4.0 * (d + 2 * 1536 + K * v)),
              ("backward: surrogate, Linear 2 (dX, db2, W2 + s_bar stepped in the same pass), GELU, "
               "Linear 1 (likewise), unpack-project",
               16.0 * (sizes[4] + sizes[2]) + 4.0 * (2 * K * v + sizes[0])),
              ("surprise-momentum update of the other four parameters with gradients (read W, g, "
               "s_bar; write W, s_bar)", 20.0 * n_upd)]
    mk = lambda: torch.cuda.Event(enable_timing=True)
    acc = [0.0, 0.0, 0.0]
    reps = max(3, args.steps // 2)
    for it in range(reps + 1):
        ev = [mk() for _ in range(5)]
        tape.begin()
        s = gc.upload_bitpacked(tape, state)
        ev[0].record()
        pred = model.forward(tape, s)
        ev[1].record()
        dl = gc.upload_bitpacked(tape, delta)
        node = gc.record_surrogate_loss(tape, pred, dl)
        gc.vsa_loss_forward(tape, node, model.gumbel_seed, model.gumbel_counter)
        ev[2].record()
        opt.prepare(tape)
        tape.backward(node, 0)
        ev[3].record()
        opt.apply(tape)
        ev[4].record()
        torch.cuda.synchronize()
        tape.end()
        if it:
            for j, (a, b) in enumerate(((0, 1), (2, 3), (3, 4))):
                acc[j] += ev[a].elapsed_time(ev[b]) / reps
    kernels = []
    for (name, byts), t in zip(phases, acc):
        gbs = byts / (t * 1e-3) / 1e9
        kernels.append({"call": name, "bound": "hbm", "ms": round(t, 4), "achieved": round(gbs, 1),
                        "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "work": byts})
    dom = max(kernels, key=lambda k: k["ms"])
    cpu = None
    if not args.no_cpu:
        from oracle import cpu_ref
        W = [gb.download(dev, i, (n,)) for i, n in zip(model.parameter_buffer_ids(), sizes)]
        sb = [np.zeros_like(w) for w in W]
        nt = cpu_ref.threads()
        with cpu_ref.limit_threads(nt):
            t0 = time.perf_counter()
            cpu_ref.hypernet_step(W, state[None], delta[None], d, v, K, sb)
            dt = time.perf_counter() - t0
        cpu = {"value": round(1.0 / dt, 3), "unit": "steps/s", "cores": nt, "kind": "port",
               "sample": f"one full step in numpy fp32 (oracle/cpu_ref.py hypernet_step: the "
                         f"reference's CPU formulas), {dt:.2f} s", "cpu_model": cpu_ref.cpu_model()}
    out = line("VSA hypernetwork training steps/s (vsa_training_step at the reference defaults)",
               round(1e3 / ms, 2), "steps/s", args, ms, "f32",
               {"workload": "H22 vsa_training_step: d_model 768, vsa_dim 10240, K 16, router 32, "
                            "batch 1 (W2 1.0 GB fp32), surprise-momentum optimizer",
                "params": int(sum(sizes)), "parallelism": "none (1 GPU)"},
               {"kernel": dom["call"], "bound": "hbm", "achieved": dom["achieved"],
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": dom["frac"], "launch_ms": dom["ms"],
                "traffic": None,
                "timing": "HIP events around the phase inside the composed step, mean"}, cpu)
    out["kernels"] = kernels
    out["step_bytes"] = sum(p[1] for p in phases)
    return out


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
    """The timed backward step; all buffers preallocated (no allocation inside).  Each GEMM of
    the block is its own C-ABI call (the fused entry points take NULL for the half they skip),
    so HIP events between the calls time every kernel inside the timed steps."""

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

    # (call, kernels, bound, algorithmic work per call: FLOP or bytes)
    CALLS = [
        ("down projection backward: dWd = dY^T A, 2048x5632x4096, beside gu = glu'(dY Wd), "
         "4096x5632x2048 (the SwiGLU backward in the GEMM's epilogue)",
         "gemm_core 256x256 (fp32 C) + gemm_core (epi 1) on the side stream", "mfma",
         2.0 * DM * HID * T + 2.0 * T * HID * DM),
        ("dN = [dG|dU] [Wg;Wu], 4096x2048x11264", "gemm_core 256x128 with producer waves (bf16 C)",
         "mfma", 2.0 * T * DM * 2 * HID),
        ("[dWg;dWu] = [dG|dU]^T N, 11264x2048x4096",
         "gemm_core 256x128 with producer waves (fp32 C; 704 blocks)", "mfma", 2.0 * 2 * HID * DM * T),
        ("RMSNorm backward 4096x2048 (rows + parameter partials)", "norm_bwd_rows + colsum_partials",
         "hbm", 3.0 * T * DM * 2 + 4.0 * T),
    ]

    def __call__(self, ev=None, only=None):
        """ev: events recorded at the call boundaries (all of them, or with `only` = i just the
        two around call i)."""
        gn, d, P, s = self.gn, self.d, self.gn._ptr, self.gn._stream()
        L = gn.lib()
        if not ev:
            rec = lambda i: None
        elif only is None:
            rec = lambda i: ev[i].record()
        else:
            rec = lambda i: ev[i - only].record() if i in (only, only + 1) else None
        rec(0)
        gn._check(L.gn_ffn_down_glu_bwd(gn.GLU["swiglu_up"], P(d["dY"]), P(d["a"]), P(d["Wd"]),
                                        P(d["gate"]), P(d["up"]), P(self.gu), P(self.dWd), None,
                                        T, DM, HID, gn.BF16, 0, s), "ffn_down_glu_bwd")
        rec(1)
        gn._check(L.gn_glu_proj_bwd(P(self.gu), P(d["n"]), P(d["Wg"]), P(d["Wu"]), P(self.dN),
                                    None, None, None, None, T, DM, HID, gn.BF16, 0, s), "glu_proj_bwd (dN)")
        rec(2)
        gn._check(L.gn_glu_proj_bwd(P(self.gu), P(d["n"]), P(d["Wg"]), P(d["Wu"]), None,
                                    P(self.dWg), P(self.dWu), None, None, T, DM, HID, gn.BF16, 0,
                                    s), "glu_proj_bwd (dWg, dWu)")
        rec(3)
        gn._check(L.gn_rmsnorm_bwd(P(self.dN), P(d["x"]), P(d["w"]), P(d["rstd"]), P(self.dx),
                                   P(self.dw), T, DM, gn.BF16, 0, P(self.ws), self.ws.numel(), s),
                  "rmsnorm_bwd")
        rec(4)


def kernel_breakdown(calls, evs):
    """Per-call mean ms over the steps of the breakdown pass from the events recorded between
    the calls."""
    out = []
    for i, (name, kern, bound, work) in enumerate(calls):
        ms = sum(e[i].elapsed_time(e[i + 1]) for e in evs) / len(evs)
        rate = work / (ms * 1e-3) / (1e12 if bound == "mfma" else 1e9)
        peak = BF16_PEAK_TFLOPS if bound == "mfma" else HBM_PEAK_GBS
        out.append({"call": name, "kernels": kern, "bound": bound, "ms": round(ms, 4),
                    "achieved": round(rate, 1), "unit": "TFLOP/s" if bound == "mfma" else "GB/s",
                    "frac": round(rate / peak, 4), "work": work})
    return out


def ffn_inputs_host(tokens):
    r = np.random.default_rng(2)
    x = r.standard_normal((tokens, DM)).astype(np.float32)
    w = np.ones(DM, np.float32)
    Wg = (r.standard_normal((HID, DM)) * 0.02).astype(np.float32)
    Wu = (r.standard_normal((HID, DM)) * 0.02).astype(np.float32)
    Wd = (r.standard_normal((DM, HID)) * 0.02).astype(np.float32)
    dY = (r.standard_normal((tokens, DM)) * 1e-2).astype(np.float32)
    return x, w, Wg, Wu, Wd, dY


def cpu_baseline(tokens):
    """The reference's CPU path (numpy fp32 restatement of autograd_core.py:486-654 with the
    SwiGLU / RMSNorm formulas, oracle/cpu_ref.py) on the whole FFN-block backward: median of 5
    after one warm-up, BLAS threads = the host's CPU share."""
    from oracle import cpu_ref
    import oracle
    x, w, Wg, Wu, Wd, dY = ffn_inputs_host(tokens)
    n, rstd = oracle.rmsnorm_fwd(x, w)
    gate, up = oracle.linear_fwd(n, Wg), oracle.linear_fwd(n, Wu)
    a = oracle.glu_fwd("swiglu_up", gate, up)
    nt = cpu_ref.threads()
    with cpu_ref.limit_threads(nt):
        cpu_ref.ffn_block_step(x, w, rstd, n, gate, up, a, Wg, Wu, Wd, dY)
        ts = []
        for _ in range(5):
            t0 = time.perf_counter()
            cpu_ref.ffn_block_step(x, w, rstd, n, gate, up, a, Wg, Wu, Wd, dY)
            ts.append(time.perf_counter() - t0)
    dt = float(np.median(ts))
    return {"value": round(tokens / dt, 1), "unit": "tokens/s", "cores": nt, "kind": "port",
            "sample": f"the whole {tokens}-token FFN-block backward in numpy fp32 (the reference's "
                      f"CPU path, autograd_core.py:486-654 restated in oracle/cpu_ref.py), median "
                      f"of 5: {dt:.3f} s", "cpu_model": cpu_ref.cpu_model()}


def oracle_timing(tokens):
    """The C oracle (fp64 accumulation, OpenMP) on `tokens` rows: the checker, timed apart."""
    import oracle
    x, w, Wg, Wu, Wd, dY = ffn_inputs_host(tokens)
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
    return {"value": round(tokens / dt, 2), "unit": "tokens/s", "threads": oracle.num_threads(),
            "sample": f"{tokens} tokens on the C oracle (fp64 accumulation), {dt:.2f} s"}


def main():
    args = parse()
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary, args.pmc_call)
        return
    if args.pmc_sq:
        pmc_sq_summary(args.pmc_sq)
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
        fn = {"attn": bench_attn, "attn32": bench_attn32, "vsa": bench_vsa, "mlp": bench_mlp,
              "decoder": bench_decoder, "hyper": bench_hyper, "linear32": bench_linear32}[args.workload]
        print(json.dumps(fn(args, torch, gn)))
        return
    dev = torch.device("cuda:0")
    d = make_inputs(torch, dev)
    st = Step(gn, torch, d)
    for _ in range(args.warmup):
        st()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    mk = lambda: torch.cuda.Event(enable_timing=True)
    # breakdown pass (before the timed region): events at every call boundary.  An event
    # between two calls costs a few microseconds, so the timed steps carry only the two
    # around the dominant call.
    nb = max(5, min(args.steps, 20))
    evs = [[mk() for _ in range(len(Step.CALLS) + 1)] for _ in range(nb)]
    for i in range(nb):
        st(evs[i])
    torch.cuda.synchronize()
    kernels = kernel_breakdown(Step.CALLS, evs)
    # the roofline's kernel: the longest call that is one product (the down projection call
    # runs two products side by side)
    di = max((i for i in range(len(kernels)) if " + " not in Step.CALLS[i][1]),
             key=lambda i: kernels[i]["ms"])
    dev_ = [[mk(), mk()] for _ in range(args.steps)]
    e0, e1 = mk(), mk()
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(args.steps):
        st(dev_[i], only=di)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    dom = dict(kernels[di])
    name, kern, bound, work = Step.CALLS[di]
    dom["ms"] = round(sum(e[0].elapsed_time(e[1]) for e in dev_) / args.steps, 4)
    rate = work / (dom["ms"] * 1e-3) / (1e12 if bound == "mfma" else 1e9)
    dom["achieved"] = round(rate, 1)
    dom["frac"] = round(rate / (BF16_PEAK_TFLOPS if bound == "mfma" else HBM_PEAK_GBS), 4)
    if args.calib_copy:
        calib_copy(torch, gn)
    flops_step = 6 * 2.0 * T * DM * HID
    cpu = None
    extra = {}
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_tokens)
        extra["cpu_oracle"] = oracle_timing(args.cpu_tokens)
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
        "roofline": {"kernel": dom["call"], "launches": dom["kernels"], "bound": dom["bound"],
                     "achieved": dom["achieved"],
                     "peak": BF16_PEAK_TFLOPS if dom["bound"] == "mfma" else HBM_PEAK_GBS,
                     "unit": dom["unit"], "frac": dom["frac"], "launch_ms": dom["ms"],
                     "traffic": traffic_from_profile(dom["call"].split(" = ")[0]),
                     "timing": "HIP events around the call inside every timed step, mean"},
        "kernels_timing": f"per-call HIP events over {nb} steps of a pass before the timed region; "
                          "an event pair at every call boundary adds ~5-10 % to each call, so the "
                          "calls sum above ms_per_step (the timed steps carry one pair only)",
        "kernels": kernels,
        "cpu_baseline": cpu,
        "wall_s": round(wall, 3),
    }
    out.update(extra)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
