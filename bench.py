#!/usr/bin/env python3
"""GLINT hot-path benchmark on one MI355X. Prints ONE JSON line.

Headline: the decode H-TILE GEMV y = x W^T, M = 1,
W = GLINT pin of [14336 x 4096] (bs 64), f32 accumulate, BF16 out. A step is one GEMV
launch; the timed loop rotates through enough distinct weight pins (>= 1 GiB) that the
256 MB Infinity Cache cannot hold the working set. `value` is the effective HBM rate:
algorithmic bytes per launch (N K (1 + 4/64) + 2 K + 2 N = 62.43 MB) / time per launch.

Also measured in the same run (extra keys): whole-model encode and expand of a synthetic
Llama-3-8B-shaped tensor set, the prefill H-TILE GEMM and the
plain INT8 GEMM; each with its own roofline fraction. The CPU baseline is
the repo's numpy restatement of the reference host path (glint_np), timed on this host.

    python bench.py [--gpus 1] [--steps 100] [--warmup 10] [--quick]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
I8_PEAK_TOPS = 5000.0
METRIC = "H-TILE GEMV/GEMM effective HBM GB/s (% peak) + encode GB/s BF16-in, 1 GPU"
GEMV_N, GEMV_K = 14336, 4096


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def timed(torch, fns, steps: int, warmup: int) -> float:
    """Average ms per call over `steps` calls (cycling through fns), HIP events on the
    current stream bracketing the whole timed loop."""
    for i in range(warmup):
        fns[i % len(fns)]()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        fns[i % len(fns)]()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) / steps


def gemv_bytes(N: int, K: int, out_bytes: int = 2) -> float:
    return N * K * (1 + 4 / 64) + 2 * K + out_bytes * N


def bench_gemv(torch, H, steps, warmup):
    N, K = GEMV_N, GEMV_K
    per = gemv_bytes(N, K)
    copies = max(17, int(1.05 * 2 ** 30 / per) + 1)
    g = torch.Generator(device="cuda").manual_seed(2002)
    pins = []
    for _ in range(copies):
        w = (torch.randn(N * K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        pins.append(H.encode_bf16(w, 64))
        del w
    gx = torch.Generator(device="cuda").manual_seed(2001)
    x = torch.randn(K, device="cuda", generator=gx).to(torch.bfloat16)
    y = torch.empty(N, dtype=torch.bfloat16, device="cuda")
    fns = [lambda p=p: H.htile_bf16(p[0], p[1], p[2], x, N, K, 64, out=y) for p in pins]
    ms = timed(torch, fns, steps, warmup)
    yf = torch.empty(N, dtype=torch.float32, device="cuda")
    fns32 = [lambda p=p: H.htile_f32(p[0], p[1], p[2], x, N, K, 64, out=yf) for p in pins]
    ms32 = timed(torch, fns32, steps, warmup)
    # W_down shape: N=4096, K=14336
    pins_d = []
    gd = torch.Generator(device="cuda").manual_seed(2003)
    for _ in range(copies):
        w = (torch.randn(4096 * 14336, device="cuda", generator=gd) * 0.02).to(torch.bfloat16)
        pins_d.append(H.encode_bf16(w, 64))
        del w
    xd = torch.randn(14336, device="cuda", generator=gx).to(torch.bfloat16)
    yd = torch.empty(4096, dtype=torch.bfloat16, device="cuda")
    fnsd = [lambda p=p: H.htile_bf16(p[0], p[1], p[2], xd, 4096, 14336, 64, out=yd) for p in pins_d]
    msd = timed(torch, fnsd, steps, warmup)
    del pins_d
    return {
        "ms": ms, "bytes": per, "gbs": per / ms / 1e6, "copies": copies, "rotation_bytes": copies * per,
        "f32_out_ms": ms32, "f32_out_gbs": gemv_bytes(N, K, 4) / ms32 / 1e6,
        "down_4096x14336_ms": msd, "down_4096x14336_gbs": gemv_bytes(4096, 14336) / msd / 1e6,
    }, pins, x


def llama3_8b_shapes():
    shapes = []
    for _ in range(32):
        shapes += [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096), (14336, 4096), (4096, 14336)]
    shapes += [(128256, 4096), (128256, 4096)]
    return shapes


def bench_model_encode(torch, H, passes: int):
    shapes = llama3_8b_shapes()
    total = sum(a * b for a, b in shapes)
    ws, pins, outs = [], [], []
    for t, (a, b) in enumerate(shapes):
        g = torch.Generator(device="cuda").manual_seed(4000 + t)
        w = (torch.randn(a * b, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        ws.append(w)
    torch.cuda.synchronize()
    for w in ws:
        n = w.numel()
        pins.append((torch.empty((n + 1) // 2, dtype=torch.uint8, device="cuda"),
                     torch.empty((n + 1) // 2, dtype=torch.uint8, device="cuda"),
                     torch.empty((n + 63) // 64, dtype=torch.float32, device="cuda")))
    enc = lambda: [H.encode_bf16(w, 64, out=p) for w, p in zip(ws, pins)]
    ms_enc = timed(torch, [enc], passes, 1)
    del ws
    torch.cuda.empty_cache()
    outs = [torch.empty(p[0].numel() * 2, dtype=torch.bfloat16, device="cuda") for p in pins]
    ns = [a * b for a, b in shapes]
    exp = lambda: [H.expand_bf16(p[0], p[1], p[2], n, 64, out=o) for p, n, o in zip(pins, ns, outs)]
    ms_exp = timed(torch, [exp], passes, 1)
    del outs, pins
    torch.cuda.empty_cache()
    b = 3.0625 * total
    return {
        "params": total, "tensors": len(shapes), "passes": passes,
        "encode_ms": ms_enc, "encode_bf16_in_gbs": 2 * total / ms_enc / 1e6,
        "encode_hbm_gbs": b / ms_enc / 1e6, "encode_frac": b / ms_enc / 1e6 / HBM_PEAK_GBS,
        "expand_bf16_ms": ms_exp, "expand_hbm_gbs": b / ms_exp / 1e6, "expand_frac": b / ms_exp / 1e6 / HBM_PEAK_GBS,
    }


def bench_prefill(torch, H, steps: int):
    out = {}
    g = torch.Generator(device="cuda").manual_seed(3002)
    wg = (torch.randn(14336 * 4096, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    pin_g = H.encode_bf16(wg, 64)
    wd = (torch.randn(4096 * 14336, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    pin_d = H.encode_bf16(wd, 64)
    del wg, wd
    gx = torch.Generator(device="cuda").manual_seed(3001)
    for M in (64, 512, 2048):
        for name, pin, N, K in (("gate", pin_g, 14336, 4096), ("down", pin_d, 4096, 14336)):
            x = torch.randn(M, K, device="cuda", generator=gx).to(torch.bfloat16)
            y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
            ms = timed(torch, [lambda: H.htile_bf16(pin[0], pin[1], pin[2], x, N, K, 64, out=y)], steps, 2)
            fl = 2.0 * M * N * K
            byt = N * K * (1 + 4 / 64) + 2 * M * K + 2 * M * N
            out[f"M{M}_{name}"] = {"ms": ms, "tflops": fl / ms / 1e9, "mfma_frac": fl / ms / 1e9 / BF16_PEAK_TFLOPS,
                                   "eff_gbs": byt / ms / 1e6}
    return out


def bench_int8(torch, H, steps: int):
    M, N, K = 2048, 8192, 8192
    g = torch.Generator(device="cuda").manual_seed(5001)
    A = torch.randint(-127, 128, (M, K), device="cuda", generator=g, dtype=torch.int8)
    B = torch.randint(-127, 128, (N, K), device="cuda", generator=g, dtype=torch.int8)
    sa = torch.rand(M, device="cuda", generator=g) * 0.019 + 1e-3
    sb = torch.rand(N, device="cuda", generator=g) * 0.019 + 1e-3
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ms = timed(torch, [lambda: H.int8_gemm_scaled_bf16(A, B, sa, sb, out=out)], steps, 2)
    ops = 2.0 * M * N * K
    return {"ms": ms, "tops": ops / ms / 1e9, "mfma_frac": ops / ms / 1e9 / I8_PEAK_TOPS, "shape": [M, N, K]}


def cpu_baseline(seconds_target: float = 10.0):
    """The repo's numpy restatement of the reference host path (glint_np: encode_f32,
    expand, x @ W^T) on a bounded sample of the same workload, single process."""
    import numpy as np
    from oracle import glint_oracle as G
    rng = np.random.default_rng(2002)
    K = GEMV_K
    rows = 256
    w = rng.normal(0, 0.02, rows * K).astype(np.float32)
    u16 = G.f32_to_bf16_bits(w)
    hole, plug, am = G.encode_bf16(u16, 64)
    x = G.bf16_bits_to_f32(G.f32_to_bf16_bits(rng.normal(0, 1, K).astype(np.float32)))
    t0 = time.perf_counter()
    reps = 0
    while time.perf_counter() - t0 < seconds_target / 2:
        W = G.expand(hole, plug, am, rows * K, 64).reshape(rows, K)
        _ = W @ x
        reps += 1
    gemv_s = (time.perf_counter() - t0) / reps
    gemv_gbs = gemv_bytes(rows, K) / gemv_s / 1e9
    t0 = time.perf_counter()
    reps = 0
    while time.perf_counter() - t0 < seconds_target / 2:
        G.encode_bf16(u16, 64)
        reps += 1
    enc_s = (time.perf_counter() - t0) / reps
    return {
        "value": gemv_gbs, "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": f"numpy glint_np restatement: expand + x@W^T of {rows}x{K} rows of the GEMV weight, repeated ~{seconds_target / 2:.0f} s",
        "encode_bf16_in_gbs": 2 * rows * K / enc_s / 1e9,
        "encode_sample": f"numpy encode_f32 of {rows}x{K} BF16 weights, repeated ~{seconds_target / 2:.0f} s",
    }


def load_traffic():
    p = ROOT / "profiles" / "htile_gemv_m1_14336x4096.traffic.json"
    if p.is_file():
        try:
            return json.loads(p.read_text()).get("traffic_bytes")
        except Exception:
            return None
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--quick", action="store_true", help="headline GEMV only")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run 10 plain 256 MiB device copies (the reference kernel for scaling PMC byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the GLINT hot path has no multi-GPU mode in this build "
              "(see DESIGN.md for how it would shard). Run with --gpus 1.", file=sys.stderr)
        return 2
    import torch
    from glint_amd import glint_hip as H
    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    H.encode_lib()
    H.p7_lib()
    log(f"device {torch.cuda.get_device_name(0)}")
    if args.calibrate_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    gemv, pins, x = bench_gemv(torch, H, args.steps, args.warmup)
    log(f"gemv {gemv['ms'] * 1e3:.2f} us {gemv['gbs']:.0f} GB/s")
    del pins
    torch.cuda.empty_cache()
    extra = {}
    if not args.quick:
        extra["model_encode"] = bench_model_encode(torch, H, passes=3)
        log(f"model encode {extra['model_encode']['encode_bf16_in_gbs']:.0f} GB/s bf16-in")
        extra["prefill"] = bench_prefill(torch, H, steps=5)
        log("prefill done")
        extra["int8_gemm"] = bench_int8(torch, H, steps=10)
        log(f"int8 {extra['int8_gemm']['tops']:.0f} TOPS")
    cpu = None if args.no_cpu else cpu_baseline()
    achieved = gemv["gbs"]
    line = {
        "metric": METRIC, "value": round(gemv["gbs"], 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": gemv["ms"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded N(0,0.02^2) weights, N(0,1) x)",
        "config": {"workload": "decode H-TILE GEMV, M=1, W GLINT pin [14336x4096] bs=64, bf16 out (BASELINE configs[1])",
                   "N": GEMV_N, "K": GEMV_K, "blocksize": 64, "weight_copies_rotated": gemv["copies"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": load_traffic()},
        "cpu_baseline": cpu,
        "gemv": gemv,
        **extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
