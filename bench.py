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


def timed(torch, fns, steps: int, warmup: int, lead: int = 4) -> float:
    """Average ms per call over exactly `steps` calls (cycling through fns), HIP events on
    the current stream bracketing them, the device synchronized before and after.

    The warmup calls (at least `lead`) are queued after the first synchronize and the start
    event is recorded behind them, so the timed window opens when the GPU finishes the last
    warmup call and holds the `steps` calls back to back, with the host already ahead of
    the GPU. Recording the start event on an idle GPU instead puts the host's latency for
    the first timed call (a few microseconds of Python, ctypes and launch) inside the
    window, which at 20 steps of a 12 us kernel is 2-4% of the figure."""
    torch.cuda.synchronize()
    n = len(fns)
    w = max(warmup, lead)
    for i in range(w):
        fns[i % n]()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        fns[(w + i) % n]()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) / steps


def timed_sync_first(torch, fns, steps: int, warmup: int) -> float:
    """The same loop with the start event recorded on an idle GPU (synchronize, then
    record, then launch): the host's first-launch latency falls inside the window. Kept
    beside `timed` so both figures are on the line."""
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


def settle(torch, fns, seconds: float = 0.05):
    """Untimed launches for about `seconds` before a timed loop, so the GPU is at its
    steady clock and power state when the warmup steps and the timed steps run."""
    t0 = time.perf_counter()
    i = 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(100):
            fns[i % len(fns)]()
            i += 1
        torch.cuda.synchronize()


def bound(fn, *args):
    """A zero-argument call of the C-ABI function `fn` with its arguments converted once
    (tensors to device pointers, ints to C ints), so the timed loop pays only the ctypes
    call and the launch, not Python tensor bookkeeping. Raises on a non-zero return."""
    import ctypes
    conv = []
    for a in args:
        if hasattr(a, "data_ptr"):
            conv.append(ctypes.c_void_p(a.data_ptr()))
        elif isinstance(a, ctypes.c_void_p):
            conv.append(a)
        else:
            conv.append(a)
    conv = tuple(conv)

    def call():
        rc = fn(*conv)
        if rc != 0:
            raise RuntimeError(f"{fn.__name__} rc={rc}")
    return call


def stream_handle(torch):
    import ctypes
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def gemv_bytes(N: int, K: int, out_bytes: int = 2) -> float:
    return N * K * (1 + 4 / 64) + 2 * K + out_bytes * N


def bench_gemv(torch, H, steps, warmup, headline_only=False):
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
    lib, st = H.encode_lib(), stream_handle(torch)
    fns = [bound(lib.launch_glint_htile_bf16_stream, p[0], p[1], p[2], x, y, 1, N, K, 64, st) for p in pins]
    settle(torch, fns, 0.2)
    ms = timed(torch, fns, steps, warmup)
    ms_sync_first = timed_sync_first(torch, fns, steps, warmup)
    if headline_only:
        return {"ms": ms, "bytes": per, "gbs": per / ms / 1e6, "copies": copies, "rotation_bytes": copies * per,
                "ms_sync_first": ms_sync_first}, pins, x
    yf = torch.empty(N, dtype=torch.float32, device="cuda")
    fns32 = [bound(lib.launch_glint_htile_s3_f32_stream, p[0], p[1], p[2], x, yf, 1, N, K, 64, st) for p in pins]
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
    fnsd = [bound(lib.launch_glint_htile_bf16_stream, p[0], p[1], p[2], xd, yd, 1, 4096, 14336, 64, st) for p in pins_d]
    msd = timed(torch, fnsd, steps, warmup)
    del pins_d
    return {
        "ms": ms, "bytes": per, "gbs": per / ms / 1e6, "copies": copies, "rotation_bytes": copies * per,
        "ms_sync_first": ms_sync_first, "f32_out_ms": ms32, "f32_out_gbs": gemv_bytes(N, K, 4) / ms32 / 1e6,
        "down_4096x14336_ms": msd, "down_4096x14336_gbs": gemv_bytes(4096, 14336) / msd / 1e6,
    }, pins, x


def _gemv_cu_plan(N: int, K: int, cus: int):
    """k_htile_gemv_cu's launch plan (glint_htile.hip htile_launch_gemv_cu): workgroups and
    waves per workgroup for an M = 1 GEMV with K % 2048 == 0."""
    S = K // 2048
    narrow = S <= 2
    G = (8 if narrow else 16) // S
    wgs = cus * (2 if narrow else 1)
    rows = -(-N // wgs)
    return -(-N // rows), S * G, rows


def _timeline_summary(a, N: int, K: int, wpg: int, rows: int, nbytes: float) -> list:
    """Text lines for the per-wave stamps `a` (waves x 8, slots as in glint_htile.hip's
    GLINT_TIMELINE block) of one k_htile_gemv_cu launch."""
    import numpy as np
    a = a.astype(np.int64)
    nw = a.shape[0]
    T0 = a[:, 0].min()
    us = lambda v: (v - T0) / 100.0  # s_memrealtime runs at 100 MHz
    st, rdy, lend, en = us(a[:, 0]), us(a[:, 3]), us(a[:, 4]), us(a[:, 5])
    mhz = np.median((a[:, 7] - a[:, 2]) / ((a[:, 5] - a[:, 0]) / 100.0))
    hw = a[:, 1]
    xcc, se, sh, cu = (hw >> 32) & 0xF, (hw >> 13) & 0x7, (hw >> 12) & 0x1, (hw >> 8) & 0xF
    items = a[:, 6]
    wg = np.arange(nw) // wpg
    nwg = nw // wpg
    wst = np.array([st[wg == g].min() for g in range(nwg)])
    wen = np.array([en[wg == g].max() for g in range(nwg)])
    wit = np.array([items[wg == g].sum() for g in range(nwg)])
    key = (xcc * 64 + se * 16 + sh * 8)[::wpg] * 16 + cu[::wpg]
    gen = np.zeros(nwg, dtype=int)
    for k in np.unique(key):
        idx = np.nonzero(key == k)[0]
        gen[idx[np.argsort(wst[idx], kind="stable")]] = np.arange(idx.size)
    pct = lambda v, q=(0, 10, 50, 90, 100): " ".join(f"{x:6.2f}" for x in np.percentile(v, q))
    span = en.max()
    out = [f"{N}x{K}: {nwg} workgroups x {wpg} waves ({rows} rows each) on {np.unique(key).size} CUs; "
           f"shader clock {mhz:.0f} MHz (s_memtime against s_memrealtime)",
           f"  kernel span (first wave start to last wave end) {span:.2f} us: {nbytes / span / 1e3:.0f} GB/s "
           f"({nbytes / span / 1e3 / HBM_PEAK_GBS:.3f} of 8 TB/s) over the span",
           "  times in us from the first wave's start      p0     p10    p50    p90    p100",
           f"  wave start                                  {pct(st)}",
           f"  first item done (table, x, item 1)          {pct(rdy)}",
           f"  item loop done                              {pct(lend)}",
           f"  wave end (after the row stores)             {pct(en)}",
           f"  workgroup end                               {pct(wen)}",
           f"  per wave: loop (first item done -> loop done) {pct(lend - rdy)}",
           f"  per wave: items                             {pct(items)}",
           ]
    for g in np.unique(gen):
        m = gen == g
        out.append(f"  workgroups dispatched {['first', 'second', 'third', 'fourth'][min(g, 3)]} on their CU "
                   f"({m.sum()}): start p50 {np.median(wst[m]):.2f}, end p10/p50/p90/max "
                   f"{pct(wen[m], (10, 50, 90, 100))}, items per workgroup p50 {np.median(wit[m]):.0f}, "
                   f"{np.mean(np.nonzero(m)[0] < nwg // 2) * 100:.0f}% in the first half of the grid")
    ends = " ".join(f"{np.median(wen[(xcc[::wpg] == x)]):.2f}/{wen[(xcc[::wpg] == x)].max():.2f}"
                    for x in np.unique(xcc))
    out.append(f"  workgroup end median/max per XCD: {ends}")
    return out


def gemv_timeline(torch, H, out_path: str, steps: int) -> None:
    """Per-wave timeline of the decode GEMV (k_htile_gemv_cu) at the headline shape and the
    down shape, from libglint_encode_tl.so (the same kernels with stamps compiled in): the
    same rotated pins and timed loop as the headline; the stamps are the loop's last launch."""
    import ctypes
    import numpy as np
    from glint_amd import glint_hip
    path = glint_hip.LIB_DIR / "libglint_encode_tl.so"
    if not path.is_file():
        raise RuntimeError("libglint_encode_tl.so not built: run `python -m glint_amd.build`")
    tl = ctypes.CDLL(str(path))
    VP, I = ctypes.c_void_p, ctypes.c_int
    tl.launch_glint_htile_bf16_stream.argtypes = [VP, VP, VP, VP, VP, I, I, I, I, VP]
    tl.launch_glint_htile_bf16_stream.restype = I
    tl.glint_timeline_fetch.argtypes = [VP, ctypes.c_size_t]
    tl.glint_timeline_fetch.restype = I
    plain = H.encode_lib()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    st = stream_handle(torch)
    lines = [f"# per-wave timeline of k_htile_gemv_cu (M = 1, bs 64, BF16 out) on {torch.cuda.get_device_name(0)}",
             "", "command (repo root):", f"  python3 bench.py --timeline {out_path} --steps {steps}", "",
             "libglint_encode_tl.so is libglint_encode.so built with -DGLINT_TIMELINE: lane 0 of each wave stores",
             "s_memrealtime (100 MHz) stamps at entry, after its first item (cell table, x and item 1 in),",
             "after its item loop and after the row stores, plus XCC_ID/HW_ID, its item count and",
             "s_memtime. The stamps are those of the last launch of a timed loop of back-to-back launches",
             "over rotated pins (the headline loop's setup). A launch's algorithmic bytes over its span",
             "exclude the gap between launches, which the per-launch HIP-event time includes.", ""]
    for N, K in ((GEMV_N, GEMV_K), (4096, 14336)):
        per = gemv_bytes(N, K)
        copies = max(17, int(1.05 * 2 ** 30 / per) + 1)
        g = torch.Generator(device="cuda").manual_seed(2002)
        pins = []
        for _ in range(copies):
            w = (torch.randn(N * K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
            pins.append(H.encode_bf16(w, 64))
            del w
        x = torch.randn(K, device="cuda", generator=g).to(torch.bfloat16)
        y = torch.empty(N, dtype=torch.bfloat16, device="cuda")
        f_pl = [bound(plain.launch_glint_htile_bf16_stream, p[0], p[1], p[2], x, y, 1, N, K, 64, st) for p in pins]
        f_tl = [bound(tl.launch_glint_htile_bf16_stream, p[0], p[1], p[2], x, y, 1, N, K, 64, st) for p in pins]
        settle(torch, f_pl, 0.2)
        ms_pl = timed(torch, f_pl, steps, 100)
        settle(torch, f_tl, 0.05)
        ms_tl = timed(torch, f_tl, steps, 100)
        grid, wpg, rows = _gemv_cu_plan(N, K, cus)
        buf = np.zeros(grid * wpg * 8, dtype=np.uint64)
        rc = tl.glint_timeline_fetch(buf.ctypes.data_as(VP), buf.nbytes)
        if rc != 0:
            raise RuntimeError(f"glint_timeline_fetch rc={rc}")
        a = buf.reshape(grid * wpg, 8)
        if not (a[:, 0] > 0).all():
            raise RuntimeError("timeline: waves without stamps (launch plan differs)")
        lines.append(f"{N}x{K}: {steps} back-to-back launches, HIP events per launch: plain {ms_pl * 1e3:.2f} us "
                     f"({per / ms_pl / 1e6 / HBM_PEAK_GBS:.3f} of 8 TB/s), instrumented {ms_tl * 1e3:.2f} us")
        lines += _timeline_summary(a, N, K, wpg, rows, per)
        lines.append("")
        del pins
        torch.cuda.empty_cache()
    text = "\n".join(lines)
    Path(out_path).write_text(text)
    print(text)


def bench_gemv_pair(torch, H, steps, warmup):
    """Beside the headline, not instead of it (opt-in: --parts gemvpair, so the default run's
    kernel trace holds only the headline's dispatches of its kernel): a decode step's gate
    and up projections are two independent GEMVs on the same x. On two streams (16 GEMVs a
    pass, alternating) one's tail could overlap the other's start; stacked as one 28672-row
    pin they are one launch."""
    N, K = GEMV_N, GEMV_K
    per = gemv_bytes(N, K)
    copies = max(17, int(1.05 * 2 ** 30 / per) + 1)
    g = torch.Generator(device="cuda").manual_seed(2002)
    pins = []
    for _ in range(copies):
        w = (torch.randn(N * K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        pins.append(H.encode_bf16(w, 64))
        del w
    x = torch.randn(K, device="cuda", generator=g).to(torch.bfloat16)
    lib, st = H.encode_lib(), stream_handle(torch)
    ys = [torch.empty(N, dtype=torch.bfloat16, device="cuda") for _ in range(2)]
    pair = lambda i, s: bound(lib.launch_glint_htile_bf16_stream, pins[i % copies][0], pins[i % copies][1],
                              pins[i % copies][2], x, ys[i % 2], 1, N, K, 64, s)
    ms_pair = timed(torch, [spread_over_streams(torch, pair, 16, 2)], max(steps // 16, 20), 3) / 16
    gs = torch.Generator(device="cuda").manual_seed(2004)
    pins_s = []
    for _ in range(max(5, int(1.05 * 2 ** 30 / (2 * per)) + 1)):
        w = (torch.randn(2 * N * K, device="cuda", generator=gs) * 0.02).to(torch.bfloat16)
        pins_s.append(H.encode_bf16(w, 64))
        del w
    ys2 = torch.empty(2 * N, dtype=torch.bfloat16, device="cuda")
    fnss = [bound(lib.launch_glint_htile_bf16_stream, p[0], p[1], p[2], x, ys2, 1, 2 * N, K, 64, st) for p in pins_s]
    ms_stack = timed(torch, fnss, max(steps // 2, 50), warmup)
    del pins_s
    del pins
    return {"two_streams": {"ms_per_gemv": ms_pair, "gbs": per / ms_pair / 1e6, "frac": per / ms_pair / 1e6 / HBM_PEAK_GBS},
            "stacked_28672x4096": {"ms": ms_stack, "gbs": 2 * per / ms_stack / 1e6,
                                   "frac": 2 * per / ms_stack / 1e6 / HBM_PEAK_GBS}}


def llama3_8b_shapes():
    shapes = []
    for _ in range(32):
        shapes += [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096), (14336, 4096), (4096, 14336)]
    shapes += [(128256, 4096), (128256, 4096)]
    return shapes


MODEL_STREAMS = 4


def spread_over_streams(torch, make_call, count: int, nstreams: int, rounds: int = 1):
    """One pass over `count` independent calls, `rounds` times, call j on stream j % nstreams
    (HIP streams at the default priority), fenced by events so the pass starts and ends on
    the current stream and times like one call. The fence empties the GPU once per pass (the
    next pass's streams wait for this one to end on the current stream), so a pass should
    hold many calls. make_call(i, stream_handle) -> zero-argument call."""
    import ctypes
    main = torch.cuda.current_stream()
    streams = [torch.cuda.Stream() for _ in range(nstreams)]
    calls = [make_call(j % count, ctypes.c_void_p(streams[j % nstreams].cuda_stream)) for j in range(count * rounds)]

    def run():
        start = torch.cuda.Event()
        start.record(main)
        for st in streams:
            st.wait_event(start)
        for c in calls:
            c()
        for st in streams:
            done = torch.cuda.Event()
            done.record(st)
            main.wait_event(done)
    return run


def bench_model_encode(torch, H, passes: int):
    """Encode then expand (to BF16) the Llama-3-8B-shaped tensor set. The tensors are
    independent, so a pass spreads them over MODEL_STREAMS streams as a pin writer would;
    the one-stream pass is reported beside it."""
    shapes = llama3_8b_shapes()
    total = sum(a * b for a, b in shapes)
    ws, pins = [], []
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
    lib = H.encode_lib()
    enc = lambda i, st: bound(lib.glint_encode_bf16_device, ws[i], ws[i].numel(), 64, pins[i][0], pins[i][1],
                              pins[i][2], st)
    nt = len(shapes)
    cur = stream_handle(torch)
    ms_enc = timed(torch, [spread_over_streams(torch, enc, nt, MODEL_STREAMS)], passes, 1)
    ms_enc1 = timed(torch, [enc(i, cur) for i in range(nt)], passes * nt, nt) * nt  # in order on one stream
    del ws
    torch.cuda.empty_cache()
    outs = [torch.empty(p[0].numel() * 2, dtype=torch.bfloat16, device="cuda") for p in pins]
    ns = [a * b for a, b in shapes]
    exp = lambda i, st: bound(lib.glint_expand_packed_to_bf16_device, pins[i][0], pins[i][1], pins[i][2], ns[i], 64,
                              outs[i], st)
    ms_exp = timed(torch, [spread_over_streams(torch, exp, nt, MODEL_STREAMS)], passes, 1)
    ms_exp1 = timed(torch, [exp(i, cur) for i in range(nt)], passes * nt, nt) * nt
    del outs, pins
    torch.cuda.empty_cache()
    b = 3.0625 * total
    return {
        "params": total, "tensors": len(shapes), "passes": passes, "streams": MODEL_STREAMS,
        "encode_ms": ms_enc, "encode_bf16_in_gbs": 2 * total / ms_enc / 1e6,
        "encode_hbm_gbs": b / ms_enc / 1e6, "encode_frac": b / ms_enc / 1e6 / HBM_PEAK_GBS,
        "expand_bf16_ms": ms_exp, "expand_hbm_gbs": b / ms_exp / 1e6, "expand_frac": b / ms_exp / 1e6 / HBM_PEAK_GBS,
        "one_stream": {"encode_ms": ms_enc1, "encode_frac": b / ms_enc1 / 1e6 / HBM_PEAK_GBS,
                       "expand_bf16_ms": ms_exp1, "expand_frac": b / ms_exp1 / 1e6 / HBM_PEAK_GBS},
    }


def bench_encode_4096(torch, H, passes: int = 5):
    """The CPU-reference configuration on the GPU: 4096x4096 BF16 (seed 1001, 0.1% outliers
    x10), bs 64, 20 distinct copies (> 256 MB Infinity Cache) cycled 4 times per pass, spread
    over MODEL_STREAMS streams; also in order on the current stream (no fork and join)."""
    import numpy as np
    rng = np.random.default_rng(1001)
    n = 4096 * 4096
    w = rng.normal(0.0, 0.02, n).astype(np.float32)
    w[rng.choice(n, n // 1000, replace=False)] *= np.float32(10.0)
    u = w.view(np.uint32)
    u16 = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    src = torch.from_numpy(u16.view(np.int16)).cuda()
    copies = 20
    ws = [src.clone() for _ in range(copies)]
    pins = [(torch.empty(n // 2, dtype=torch.uint8, device="cuda"), torch.empty(n // 2, dtype=torch.uint8, device="cuda"),
             torch.empty(n // 64, dtype=torch.float32, device="cuda")) for _ in range(copies)]
    lib = H.encode_lib()
    enc = lambda i, st: bound(lib.glint_encode_bf16_device, ws[i], n, 64, pins[i][0], pins[i][1], pins[i][2], st)
    ms = timed(torch, [spread_over_streams(torch, enc, copies, MODEL_STREAMS, rounds=4)], passes, 1) / (4 * copies)
    # one stream: the calls in order on the current stream, no fork and join per pass
    cur = stream_handle(torch)
    ms1 = timed(torch, [enc(i, cur) for i in range(copies)], passes * copies * 4, copies)
    del ws, pins, src
    torch.cuda.empty_cache()
    return {"config": "4096x4096 BF16, seed 1001, 0.1% outliers x10, bs 64; 20 copies cycled 4 times per pass",
            "streams": MODEL_STREAMS, "ms_per_matrix": ms, "encode_bf16_in_gbs": 2 * n / ms / 1e6,
            "encode_frac": 3.0625 * n / ms / 1e6 / HBM_PEAK_GBS,
            "one_stream_ms_per_matrix": ms1, "one_stream_frac": 3.0625 * n / ms1 / 1e6 / HBM_PEAK_GBS}


def bench_host_abi(H, reps: int = 5):
    """The reference's host-pointer ABI (glint_encode_bf16_host, expand to f32 / BF16 host)
    on the 4096x4096 CPU-reference config: pageable host buffers in and out, so every call
    pays H2D + kernel + D2H over PCIe. Reported apart from the device-resident rates."""
    import ctypes
    import numpy as np
    lib = H.encode_lib()
    rng = np.random.default_rng(1001)
    n = 4096 * 4096
    w = rng.normal(0.0, 0.02, n).astype(np.float32)
    w[rng.choice(n, n // 1000, replace=False)] *= np.float32(10.0)
    u = w.view(np.uint32)
    u16 = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    hole = np.empty((n + 1) // 2, np.uint8)
    plug = np.empty_like(hole)
    am = np.empty((n + 63) // 64, np.float32)
    out32 = np.empty(n, np.float32)
    out16 = np.empty(n, np.uint16)
    P = lambda a: ctypes.c_void_p(a.ctypes.data)

    def per_call(fn):
        assert fn() == 0
        t0 = time.perf_counter()
        for _ in range(reps):
            assert fn() == 0
        return (time.perf_counter() - t0) / reps

    enc = per_call(lambda: lib.glint_encode_bf16_host(P(u16), n, 64, P(hole), P(plug), P(am)))
    e32 = per_call(lambda: lib.glint_expand_packed_to_f32_host(P(hole), P(plug), P(am), n, 64, P(out32)))
    e16 = per_call(lambda: lib.glint_expand_packed_to_bf16_host(P(hole), P(plug), P(am), n, 64, P(out16)))
    return {
        "config": "4096x4096 BF16, seed 1001, 0.1% outliers, bs 64; pageable host buffers",
        "encode_ms": enc * 1e3, "encode_bf16_in_gbs": 2 * n / enc / 1e9,
        "expand_f32_ms": e32 * 1e3, "expand_f32_out_gbs": 4 * n / e32 / 1e9,
        "expand_bf16_ms": e16 * 1e3, "expand_bf16_out_gbs": 2 * n / e16 / 1e9,
    }


def bench_prefill(torch, H, steps: int, copies: int = 6):
    """Prefill GEMMs at M = 64, 512, 2048 for the gate and down shapes, and batched decode at
    M = 2, 4, 8 (the small-M GEMV) on the same shapes. Each shape rotates
    `copies` pins (about 370 MB per shape) so the weights are not served from the
    256 MB last-level cache between calls."""
    out = {}
    g = torch.Generator(device="cuda").manual_seed(3002)
    pins = {}
    for name, N, K in (("gate", 14336, 4096), ("down", 4096, 14336)):
        w = (torch.randn(N * K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        pin = H.encode_bf16(w, 64)
        del w
        pins[name] = ([pin] + [tuple(t.clone() for t in pin) for _ in range(copies - 1)], N, K)
    gx = torch.Generator(device="cuda").manual_seed(3001)
    lib, st = H.encode_lib(), stream_handle(torch)
    # batched decode: M = 2..8 rows run the small-M GEMV (each weight read once for all rows)
    dec = {}
    for M in (2, 4, 8):
        for name, (cps, N, K) in pins.items():
            x = torch.randn(M, K, device="cuda", generator=gx).to(torch.bfloat16)
            y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
            calls = [bound(lib.launch_glint_htile_bf16_stream, p[0], p[1], p[2], x, y, M, N, K, 64, st) for p in cps]
            settle(torch, calls, 0.05)
            ms = timed(torch, calls, steps * 3, copies)
            byt = N * K * (1 + 4 / 64) + 2 * M * K + 2 * M * N
            dec[f"M{M}_{name}"] = {"ms": ms, "eff_gbs": byt / ms / 1e6, "hbm_frac": byt / ms / 1e6 / HBM_PEAK_GBS}
            # the reference ABI's f32 output (the f32 small-M GEMV up to M = 4, the 3-plane tile above)
            yf = torch.empty(M, N, dtype=torch.float32, device="cuda")
            calls32 = [bound(lib.launch_glint_htile_s3_f32_stream, p[0], p[1], p[2], x, yf, M, N, K, 64, st) for p in cps]
            settle(torch, calls32, 0.05)
            ms32 = timed(torch, calls32, steps * 3, copies)
            dec[f"M{M}_{name}"]["f32_out"] = {"ms": ms32, "eff_gbs": (byt + 2 * M * N) / ms32 / 1e6}
            del yf
    out["batched_decode"] = dec
    for M in (64, 512, 2048):
        for name, (cps, N, K) in pins.items():
            x = torch.randn(M, K, device="cuda", generator=gx).to(torch.bfloat16)
            y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
            calls = [bound(lib.launch_glint_htile_bf16_stream, p[0], p[1], p[2], x, y, M, N, K, 64, st) for p in cps]
            settle(torch, calls, 0.05)
            ms = timed(torch, calls, steps * (3 if M <= 64 else 1), copies)
            fl = 2.0 * M * N * K
            byt = N * K * (1 + 4 / 64) + 2 * M * K + 2 * M * N
            # the reference ABI's f32 output (three exact BF16 weight planes on MFMA)
            yf = torch.empty(M, N, dtype=torch.float32, device="cuda")
            calls32 = [bound(lib.launch_glint_htile_s3_f32_stream, p[0], p[1], p[2], x, yf, M, N, K, 64, st) for p in cps]
            settle(torch, calls32, 0.05)
            ms32 = timed(torch, calls32, steps * (3 if M <= 64 else 1), copies)
            byt32 = byt + 2 * M * N
            out[f"M{M}_{name}"] = {"ms": ms, "tflops": fl / ms / 1e9, "mfma_frac": fl / ms / 1e9 / BF16_PEAK_TFLOPS,
                                   "eff_gbs": byt / ms / 1e6, "hbm_frac": byt / ms / 1e6 / HBM_PEAK_GBS,
                                   "f32_out": {"ms": ms32, "tflops": fl / ms32 / 1e9, "over_bf16": ms32 / ms,
                                               "eff_gbs": byt32 / ms32 / 1e6,
                                               "mfma_frac_3planes": 3 * fl / ms32 / 1e9 / BF16_PEAK_TFLOPS}}
            del yf
    del pins
    return out


def bench_int8(torch, H, steps: int):
    M, N, K = 2048, 8192, 8192
    g = torch.Generator(device="cuda").manual_seed(5001)
    A = torch.randint(-127, 128, (M, K), device="cuda", generator=g, dtype=torch.int8)
    B = torch.randint(-127, 128, (N, K), device="cuda", generator=g, dtype=torch.int8)
    sa = torch.rand(M, device="cuda", generator=g) * 0.019 + 1e-3
    sb = torch.rand(N, device="cuda", generator=g) * 0.019 + 1e-3
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    call = lambda: H.int8_gemm_scaled_bf16(A, B, sa, sb, out=out)
    settle(torch, [call], 0.05)
    ms = timed(torch, [call], steps, 2)
    ops = 2.0 * M * N * K
    return {"ms": ms, "tops": ops / ms / 1e9, "mfma_frac": ops / ms / 1e9 / I8_PEAK_TOPS, "shape": [M, N, K]}


def bench_int8_abi(torch, H, steps: int):
    """The attach ABI's int8_mma_gemm (bf16 x quantized per 64-block on the device, per-64
    weight scales, f32 out) at the reference's published shape (M 70, N 4096, K 3072:
    0.1524 ms on an RTX 3060) and at the INT8 config's 2048 x 8192 x 8192. OP = 2 M N K."""
    out = {}
    g = torch.Generator(device="cuda").manual_seed(5004)
    lib = H.p7_lib()
    st = stream_handle(torch)
    for M, N, K in ((70, 4096, 3072), (2048, 8192, 8192)):
        x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
        q = torch.randint(-127, 128, (N * K,), device="cuda", generator=g, dtype=torch.int8)
        sc = torch.rand(N * K // 64, device="cuda", generator=g) * 0.02 + 1e-3
        y = torch.empty(M, N, dtype=torch.float32, device="cuda")
        xq = torch.empty(M * K, dtype=torch.int8, device="cuda")
        sx = torch.empty(M * K // 64, dtype=torch.float32, device="cuda")
        lin = H.Int8MmaLinear(q.data_ptr(), sc.data_ptr(), N, K)
        call = bound(lib.int8_mma_gemm, x, lin, y, M, xq, sx, st)
        settle(torch, [call], 0.05)
        ms = timed(torch, [call], steps * (10 if M < 256 else 1), 2)
        ops = 2.0 * M * N * K
        out[f"M{M}_{N}x{K}"] = {"ms": ms, "tops": ops / ms / 1e9, "mfma_frac": ops / ms / 1e9 / I8_PEAK_TOPS}
        del x, q, sc, y, xq, sx
    return out


def bench_w8a16(torch, H, steps: int, copies: int = 6):
    """int8_tile_gemm_bf16 (W8A16 over an INT8 pin linear): HBM-bound decode shapes and the
    MFMA-bound 2048 x 8192 x 8192 shape of the INT8 config. Each shape rotates `copies`
    weight copies (at least 370 MB) so they are not served from the last-level cache."""
    out = {}
    g = torch.Generator(device="cuda").manual_seed(6001)
    for M, N, K in ((1, 14336, 4096), (64, 14336, 4096), (2048, 8192, 8192)):
        q = torch.randint(-127, 128, (N * K,), device="cuda", generator=g, dtype=torch.int8)
        sc = torch.rand(N * K // 64, device="cuda", generator=g) * 0.02 + 1e-3
        ws = [(q, sc)] + [(q.clone(), sc.clone()) for _ in range(copies - 1)]
        x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
        y = torch.empty(M, N, dtype=torch.float32, device="cuda")
        calls = [lambda w=w: H.int8_tile_gemm(x, w[0], w[1], N, K, y=y) for w in ws]
        settle(torch, calls, 0.05)
        # a few-microsecond call needs many steps before launch jitter averages out
        ms = timed(torch, calls, steps * (30 if M == 1 else 3 if M <= 64 else 1), copies)
        fl = 2.0 * M * N * K
        byt = N * K * (1 + 4 / 64) + 2 * M * K + 4 * M * N
        out[f"M{M}_{N}x{K}"] = {"ms": ms, "tflops": fl / ms / 1e9, "mfma_frac": fl / ms / 1e9 / BF16_PEAK_TFLOPS,
                                "eff_gbs": byt / ms / 1e6, "hbm_frac": byt / ms / 1e6 / HBM_PEAK_GBS}
        del q, sc, ws, x, y
    return out


def kmajor_step_graphs(torch, lib, pins, x, y, part, idx, cnt, N, K, ksg, ks, nsel, reps: int = 20):
    """The K-major decode step over every pin, captured into a HIP graph and replayed
    (per-step ms, HIP events around `reps` replays). Two graphs: the three calls in order on
    one stream, and the selection on a second stream beside the fold (it needs only x),
    joined by events before the correction. The selection of step i + 1 waits for step i's
    correction, which reads idx and cnt. Both capture streams have a split-K workspace, so
    the fold and correction add their slices in-kernel as in the eager loop."""
    import ctypes

    def vp(t):
        return ctypes.c_void_p(t.data_ptr())

    out = []
    for beside in (False, True):
        s, s2 = torch.cuda.Stream(), torch.cuda.Stream()
        hs, hs2 = ctypes.c_void_p(s.cuda_stream), ctypes.c_void_p(s2.cuda_stream)
        if lib.glint_htile_workspace_reserve(hs) != 0:
            raise RuntimeError("glint_htile_workspace_reserve failed")
        s.wait_stream(torch.cuda.current_stream())
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for pk in pins:
                if beside:
                    s2.wait_stream(s)
                    rc = lib.glint_select_topk(vp(x), K, nsel, vp(idx), vp(cnt), hs2)
                    join = torch.cuda.Event()
                    join.record(s2)
                else:
                    rc = lib.glint_select_topk(vp(x), K, nsel, vp(idx), vp(cnt), hs)
                rc |= lib.glint_gemv_km_fold(vp(pk[0]), vp(pk[2]), vp(x), vp(y), N, K, ksg, vp(part), hs)
                if beside:
                    s.wait_event(join)
                rc |= lib.glint_apply_corr_km(vp(pk[0]), vp(pk[1]), vp(pk[2]), vp(x), vp(idx), vp(cnt), vp(y), N, K,
                                              ks, vp(part), hs)
                if rc != 0:
                    raise RuntimeError(f"k-major step capture rc={rc}")
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            for _ in range(3):
                g.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(reps):
                g.replay()
            e1.record(s)
        e1.synchronize()
        out.append(e0.elapsed_time(e1) / (reps * len(pins)))
        del g
        lib.glint_htile_workspace_release(hs)
    return out


def bench_kmajor(torch, H, steps: int = 200, copies: int = 20):
    """The K-major decode step at the decode shape (N 14336, K 4096): fold GEMV (HBM bytes:
    hole_k N K / 2 + scales_k N K / 16 + x + y), device selection of 10% of the channels,
    and the plug correction over them, each timed alone and as one step (three launches
    back to back, C ABI through pre-bound ctypes calls). Pins rotate over `copies` (about
    1.3 GB)."""
    N, K = GEMV_N, GEMV_K
    g = torch.Generator(device="cuda").manual_seed(4242)
    pins = []
    for _ in range(copies):
        w = (torch.randn(N * K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        h, p, a = H.encode_bf16(w, 64)
        pins.append(H.kmajor_pack(h, p, a, N, K))
        del w, h, p, a
    x = torch.randn(K, device="cuda", generator=g).to(torch.bfloat16)
    y = torch.empty(N, dtype=torch.float32, device="cuda")
    part = torch.empty(32 * N, dtype=torch.float32, device="cuda")
    idx = torch.empty(K, dtype=torch.int32, device="cuda")
    cnt = torch.empty(1, dtype=torch.int32, device="cuda")
    lib, st = H.encode_lib(), stream_handle(torch)
    # the fold and the correction add their K slices through the stream's split-K counters
    # when the stream has a workspace (they never allocate one themselves)
    if lib.glint_htile_workspace_reserve(st) != 0:
        raise RuntimeError("glint_htile_workspace_reserve failed")
    ksg, ks, nsel = 16, 8, K // 10
    fold_bytes = N * K / 2 + N * K / 16 + 2 * K + 4 * N
    folds = [bound(lib.glint_gemv_km_fold, pk[0], pk[2], x, y, N, K, ksg, part, st) for pk in pins]
    sel = bound(lib.glint_select_topk, x, K, nsel, idx, cnt, st)
    corrs = [bound(lib.glint_apply_corr_km, pk[0], pk[1], pk[2], x, idx, cnt, y, N, K, ks, part, st) for pk in pins]
    settle(torch, folds, 0.05)
    ms_fold = timed(torch, folds, steps, 10)
    ms_sel = timed(torch, [sel], steps, 10)
    sel()
    ms_corr = timed(torch, corrs, steps, 10)

    def step_of(i):
        def run():
            folds[i]()
            sel()
            corrs[i]()
        return run
    ms_step = timed(torch, [step_of(i) for i in range(copies)], steps, 10)
    try:
        ms_graph, ms_graph2 = kmajor_step_graphs(torch, lib, pins, x, y, part, idx, cnt, N, K, ksg, ks, nsel)
    except RuntimeError as e:  # a capture this runtime refuses costs these two figures, not the line
        log(f"k-major graph step not measured: {e}")
        torch.cuda.synchronize()
        ms_graph = ms_graph2 = None
    # the reference's capacity mode: plug_k stays in mapped pinned host memory and the
    # correction reads only the selected channels' rows over the bus
    import ctypes
    import os
    hip = ctypes.CDLL(os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so"))
    nbytes = pins[0][1].numel()
    hbuf, dptr = ctypes.c_void_p(), ctypes.c_void_p()
    ms_corr_host = None
    if hip.hipHostMalloc(ctypes.byref(hbuf), ctypes.c_size_t(nbytes), ctypes.c_uint(0x2)) == 0:
        try:
            if hip.hipHostGetDevicePointer(ctypes.byref(dptr), hbuf, ctypes.c_uint(0)) == 0 and dptr.value:
                host_plug = pins[0][1].cpu().numpy()
                ctypes.memmove(hbuf, host_plug.ctypes.data, nbytes)
                c = bound(lib.glint_apply_corr_km, pins[0][0], dptr, pins[0][2], x, idx, cnt, y, N, K, ks, part, st)
                ms_corr_host = timed(torch, [c], max(steps // 10, 10), 3)
        finally:
            torch.cuda.synchronize()
            hip.hipHostFree(hbuf)
    del pins
    return {"config": f"N {N} K {K}, fold ksg {ksg}, 10% of channels selected, correction ks {ks}",
            "fold_ms": ms_fold, "fold_gbs": fold_bytes / ms_fold / 1e6, "fold_frac": fold_bytes / ms_fold / 1e6 / HBM_PEAK_GBS,
            "select_ms": ms_sel, "corr_ms": ms_corr, "step_ms": ms_step, "selected": int(cnt.item()),
            "step_graph_ms": ms_graph, "step_graph_select_beside_fold_ms": ms_graph2,
            "corr_host_plug_ms": ms_corr_host,
            "resident_bytes_per_weight": 0.5 + 4 / 64, "full_gemv_resident_bytes_per_weight": 1 + 4 / 64}


def bench_copy_ceiling(torch, mib: int = 1024):
    """A plain device-to-device copy (torch's copy kernel) of `mib` MiB: the mixed
    read+write rate this HBM reaches with the simplest access pattern, the practical
    ceiling next to 8 TB/s for encode and expand (which read and write)."""
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    ms = timed(torch, [lambda: dst.copy_(src)], 20, 3)
    del src, dst
    return {"bytes_moved": 2 * n, "ms": ms, "gbs": 2 * n / ms / 1e6, "frac": 2 * n / ms / 1e6 / HBM_PEAK_GBS}


def bench_read_ceiling(torch, H, steps: int):
    """Read-only HBM ceilings from libglint_probe's grid-stride read (no writes):
    - `stream_1gib`: one 1 GiB buffer per launch, the steady streaming rate;
    - `gemv_sized`: 62.43 MB buffers (the 14336 x 4096 GEMV's bytes) rotated over more than
      1 GiB, the same launch size and rotation as the headline, so launch cost and ramp are
      in it: the practical floor for the headline GEMV, which also computes and writes y."""
    import ctypes
    lib = H.probe_lib().glint_probe_read
    st = stream_handle(torch)
    grid = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.empty(grid * 1024, dtype=torch.int32, device="cuda")
    big = torch.ones(1 << 30, dtype=torch.uint8, device="cuda")
    ms_big = timed(torch, [bound(lib, big, ctypes.c_int64(big.numel()), sink, grid, st)], 20, 3)
    del big
    per = int(gemv_bytes(GEMV_N, GEMV_K)) // 16 * 16
    copies = max(17, int(1.05 * 2 ** 30 / per) + 1)
    bufs = [torch.ones(per, dtype=torch.uint8, device="cuda") for _ in range(copies)]
    fns = [bound(lib, b, ctypes.c_int64(per), sink, grid, st) for b in bufs]
    settle(torch, fns, 0.1)
    ms = timed(torch, fns, steps, 10)
    del bufs
    torch.cuda.empty_cache()
    return {"stream_1gib": {"bytes": 1 << 30, "ms": ms_big, "gbs": (1 << 30) / ms_big / 1e6,
                            "frac": (1 << 30) / ms_big / 1e6 / HBM_PEAK_GBS},
            "gemv_sized": {"bytes": per, "copies": copies, "ms": ms, "gbs": per / ms / 1e6,
                           "frac": per / ms / 1e6 / HBM_PEAK_GBS},
            "grid": f"{grid} x 1024 threads, grid-stride 16-B nontemporal loads"}


def bench_pin_tools(tensors: int = 16):
    """The pin tools' device path end to end: convert a synthetic two-shard BF16 model
    (tensors x 4096 x 4096) from safetensors files to a pin and unpin it back to BF16.
    Includes file reads and writes (page cache), host staging and PCIe both ways."""
    import tempfile
    import time
    import numpy as np
    from glint_amd import pin_tools as P
    from glint_amd.tensorfile import save
    rng = np.random.default_rng(4000)
    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR", "/tmp")) as td:
        src = Path(td) / "src"
        src.mkdir()
        wmap = {}
        for s in range(2):
            shard = f"model-0000{s + 1}-of-00002.safetensors"
            ts = []
            for l in range(tensors // 2):
                w = (rng.standard_normal((4096, 4096), dtype=np.float32) * 0.02).view(np.uint32)
                raw = ((w + (0x7FFF + ((w >> 16) & 1))) >> 16).astype("<u2").tobytes()
                ts.append((f"layers.{s * tensors // 2 + l}.mlp.weight", "BF16", (4096, 4096), raw))
            save(src / shard, ts)
            wmap.update({t[0]: shard for t in ts})
        (src / P.INDEX_NAME).write_text(json.dumps({"metadata": {}, "weight_map": wmap}))
        P.convert(src, Path(td) / "warm", dry_run=True)
        t0 = time.perf_counter()
        P.convert(src, Path(td) / "pin")
        t_conv = time.perf_counter() - t0
        t0 = time.perf_counter()
        P.unpin(Path(td) / "pin", Path(td) / "back")
        t_unpin = time.perf_counter() - t0
    gb = tensors * 4096 * 4096 * 2 / 1e9
    return {"config": f"{tensors} x 4096x4096 BF16 in two shards ({gb:.2f} GB), files in the page cache",
            "convert_s": t_conv, "convert_bf16_in_gbs": gb / t_conv, "unpin_s": t_unpin,
            "unpin_bf16_out_gbs": gb / t_unpin}


def cpu_model() -> str:
    """The host CPU's model name (the lscpu 'Model name' line, read from /proc/cpuinfo)."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(seconds_target: float = 24.0):
    """The CPU path beside the GPU, on this host, each leg repeated for a bounded time:
    the repo's C restatement of the reference host path (oracle/glint_oracle.c, OpenMP over
    the threads it reports) running the headline GEMV (expand-on-the-fly H-TILE, f32
    accumulate) at full size and encoding the CPU-reference configuration (4096x4096, seed
    1001, 0.1% outliers x10); the numpy restatement (one core) of encode, expand and a GEMV
    on row samples; numpy expand + BLAS x @ W^T at the prefill shape (a row sample of W); and
    the C int32 INT8 GEMM on a full-row sample of 2048x8192x8192."""
    import os
    import numpy as np
    from oracle import glint_oracle as G
    orc = G.Oracle()
    N, K = GEMV_N, GEMV_K
    w = np.random.default_rng(2002).normal(0.0, 0.02, N * K).astype(np.float32)
    u16 = G.f32_to_bf16_bits(w)
    del w
    hole, plug, am = orc.encode_bf16(u16, 64)
    x = G.f32_to_bf16_bits(np.random.default_rng(2001).normal(0.0, 1.0, K).astype(np.float32))

    def rate(fn, budget):
        fn()
        t0, reps = time.perf_counter(), 0
        while time.perf_counter() - t0 < budget or reps == 0:
            fn()
            reps += 1
        return (time.perf_counter() - t0) / reps, reps

    T = seconds_target
    gemv_s, gemv_reps = rate(lambda: orc.htile_f32(hole, plug, am, x, 1, N, K, 64), T * 0.3)
    rng = np.random.default_rng(1001)
    n0 = 4096 * 4096
    w0 = rng.normal(0.0, 0.02, n0).astype(np.float32)
    w0[rng.choice(n0, n0 // 1000, replace=False)] *= np.float32(10.0)
    u0 = G.f32_to_bf16_bits(w0)
    enc_s, enc_reps = rate(lambda: orc.encode_bf16(u0, 64), T * 0.2)
    # numpy restatement, one core: encode / expand of 256 rows of the 4096^2 config, GEMV rows
    rows = 256
    ws0 = G.bf16_bits_to_f32(u0[:rows * 4096])
    npe_s, npe_reps = rate(lambda: G.encode_f32(ws0, 64), T * 0.1)
    h0, p0, a0 = G.encode_f32(ws0, 64)
    npx_s, npx_reps = rate(lambda: G.expand(h0, p0, a0, rows * 4096, 64), T * 0.05)
    hs, ps, ams = hole[:rows * K // 2], plug[:rows * K // 2], am[:rows * K // 64]
    xf = G.bf16_bits_to_f32(x)
    np_s, np_reps = rate(lambda: G.expand(hs, ps, ams, rows * K, 64).reshape(rows, K) @ xf, T * 0.05)
    # numpy expand + BLAS GEMM at the prefill shape (M 512 x 4096 against 1024 of W's 14336 rows)
    Mp, rows_p = 512, 1024
    Xp = np.random.default_rng(3001).normal(0.0, 1.0, (Mp, K)).astype(np.float32)
    hp, pp, ap_ = hole[:rows_p * K // 2], plug[:rows_p * K // 2], am[:rows_p * K // 64]
    pf_s, pf_reps = rate(lambda: Xp @ G.expand(hp, pp, ap_, rows_p * K, 64).reshape(rows_p, K).T, T * 0.1)
    try:
        from threadpoolctl import threadpool_info
        blas_threads = max((i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"),
                           default=None)
    except Exception:
        blas_threads = None
    # C int32 INT8 GEMM, rows [0, 32) of the 2048 x 8192 x 8192 config
    M8, N8, K8, r8 = 2048, 8192, 8192, 32
    g8 = np.random.default_rng(5001)
    A = g8.integers(-127, 128, (M8, K8), dtype=np.int8)
    B = np.random.default_rng(5002).integers(-127, 128, (N8, K8), dtype=np.int8)
    i8_s, i8_reps = rate(lambda: orc.int8_gemm_i32(A, B, M8, N8, K8, 0, r8), T * 0.2)
    threads = orc.threads()
    return {
        "value": gemv_bytes(N, K) / gemv_s / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": f"C oracle H-TILE GEMV 14336x4096 (bs 64, bf16 x, f32 accumulate), full size, "
                  f"{gemv_reps} runs in ~{T * 0.3:.0f} s, OpenMP {threads} threads",
        "cpu_model": cpu_model(), "nproc": os.cpu_count(),
        "gemv_us": gemv_s * 1e6,
        "encode_bf16_in_gbs": 2 * n0 / enc_s / 1e9, "encode_threads": threads,
        "encode_sample": f"C oracle encode of the 4096x4096 CPU-reference config (seed 1001, 0.1% outliers), "
                         f"{enc_reps} runs",
        "numpy_encode_gbs": 2 * rows * 4096 / npe_s / 1e9, "numpy_expand_f32_out_gbs": 4 * rows * 4096 / npx_s / 1e9,
        "numpy_gemv_gbs": gemv_bytes(rows, K) / np_s / 1e9, "numpy_cores": 1,
        "numpy_sample": f"numpy restatement (oracle/glint_oracle.py), one core: encode_f32 of 256 rows of the 4096^2 "
                        f"config ({npe_reps} runs), expand of the same ({npx_reps} runs), expand + x @ W^T of "
                        f"{rows}x{K} GEMV rows ({np_reps} runs)",
        "numpy_prefill_tflops": 2.0 * Mp * rows_p * K / pf_s / 1e12, "blas_threads": blas_threads,
        "numpy_prefill_sample": f"numpy expand + BLAS X[{Mp}x{K}] @ W^T over {rows_p} of the 14336 gate rows, "
                                f"{pf_reps} runs",
        "int8_cpu_tops": 2.0 * r8 * N8 * K8 / i8_s / 1e12, "int8_threads": threads,
        "int8_sample": f"C oracle int32 GEMM, rows [0, {r8}) of A[2048x8192] against all of B[8192x8192] "
                       f"(full rows), {i8_reps} runs",
    }


# ---------------------------------------------------------------- profile summaries
GEMV_KERNEL = "k_htile_gemv_cu<true,1,512,"  # headline dispatch (bf16 out, 512-thread form), spaces removed
TRAFFIC_JSON = ROOT / "profiles" / "htile_gemv_m1_14336x4096.traffic.json"
PMC_CMD = ("rocprofv3 --pmc {ctr} -d <dir> -o run -- python3 bench.py --quick --no-cpu --headline-only "
           "--calibrate-copy --steps 20 --warmup 5")


def _pmc_avg(db_path, counter):
    """Per-dispatch average of `counter` by kernel name from a rocprofv3 (rocpd) database."""
    import sqlite3
    import statistics
    cur = sqlite3.connect(db_path).cursor()
    by = {}
    for name, ctr, val in cur.execute("select kernel_name, counter_name, value from counters_collection"):
        if ctr == counter:
            by.setdefault(name, []).append(val)
    return {k: (statistics.mean(v), len(v)) for k, v in by.items()}


def summarize_traffic(fetch_db, write_db) -> dict:
    """HBM bytes per headline GEMV launch from two --pmc runs (FETCH_SIZE, WRITE_SIZE, KiB
    per dispatch). Each counter is scaled by what it reads for the 256 MiB device copy
    (`__amd_rocclr_copyBuffer`, 10 calls made by --calibrate-copy): true bytes / counted."""
    copy_bytes = 256 << 20
    out = {"algorithmic_bytes": gemv_bytes(GEMV_N, GEMV_K)}
    for tag, db, ctr in (("fetch", fetch_db, "FETCH_SIZE"), ("write", write_db, "WRITE_SIZE")):
        avg = _pmc_avg(db, ctr)
        copy = [v for k, v in avg.items() if "copyBuffer" in k]
        gemv = [v for k, v in avg.items() if GEMV_KERNEL in k.replace(" ", "")]
        if not copy or not gemv:
            raise SystemExit(f"{db}: need copyBuffer and {GEMV_KERNEL} dispatches with {ctr}")
        scale = copy_bytes / (copy[0][0] * 1024.0)
        out[f"{tag}_counter_kib"] = gemv[0][0]
        out[f"{tag}_dispatches"] = gemv[0][1]
        out[f"{tag}_copy_counter_kib"] = copy[0][0]
        out[f"{tag}_scale"] = scale
        out[f"{tag}_bytes"] = gemv[0][0] * 1024.0 * scale
    out["traffic_bytes"] = out["fetch_bytes"] + out["write_bytes"]
    out["traffic_over_algorithmic"] = out["traffic_bytes"] / out["algorithmic_bytes"]
    out["commands"] = [PMC_CMD.format(ctr="FETCH_SIZE"), PMC_CMD.format(ctr="WRITE_SIZE"),
                       "python3 bench.py --summarize-traffic <fetch dir>/run_results.db <write dir>/run_results.db"]
    TRAFFIC_JSON.write_text(json.dumps(out, indent=1) + "\n")
    return out


def summarize_trace(kt_db, bench_json=None) -> str:
    """Per-kernel dispatch count and average / min / max duration from a --kernel-trace run,
    written as a text table next to the traffic figures."""
    import sqlite3
    import statistics
    cur = sqlite3.connect(kt_db).cursor()
    by = {}
    for name, start, end, gx, wx in cur.execute("select name, start, end, grid_x, workgroup_x from kernels"):
        by.setdefault((name, gx, wx), []).append((end - start) / 1e3)
    lines = [f"{'kernel':90s} {'grid_x':>9s} {'wg':>5s} {'calls':>6s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s} "
             f"{'total_ms':>9s}"]
    for (name, gx, wx), ds in sorted(by.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"{name[:90]:90s} {gx:9d} {wx:5d} {len(ds):6d} {statistics.mean(ds):9.2f} {min(ds):9.2f} "
                     f"{max(ds):9.2f} {sum(ds) / 1e3:9.3f}")
    text = "\n".join(lines)
    if bench_json:
        j = json.loads(Path(bench_json).read_text().strip().splitlines()[-1])
        text += (f"\n\nbench.py (same run) ms_per_step {j['ms_per_step'] * 1e3:.2f} us -> {j['value']:.0f} GB/s, "
                 f"roofline frac {j['roofline']['frac']}")
    return text


# Counter evidence: one fixed workload run under five rocprofv3 passes (FETCH_SIZE, WRITE_SIZE,
# derived utilisation, raw instruction counts, kernel trace), each dispatch assigned to its phase
# by kernel name and dispatch order. MI355X: 256 CUs, 1024 SIMDs.
COUNTERS_JSON = ROOT / "profiles" / "counters_hot_kernels.json"
CU_NUM, SIMD_NUM = 256, 1024
COUNTER_PASSES = {
    "fetch": "--pmc FETCH_SIZE",
    "write": "--pmc WRITE_SIZE",
    "util": "--pmc VALUBusy MfmaUtil LDSBankConflict",
    "inst": "--pmc SQ_INSTS_VALU SQ_INSTS_LDS SQ_INSTS_MFMA SQ_LDS_IDX_ACTIVE SQ_WAVES GRBM_GUI_ACTIVE",
    "trace": "--kernel-trace --stats",
}


ENCODE_PIECE_CHUNKS = 1 << 17  # the library's most 512-element chunks per encode launch


def encode_launches(n: int) -> int:
    """k_encode_bf16_b64 dispatches of one BF16 bs-64 encode of n elements (n % 512 == 0):
    the library launches tensors above ENCODE_PIECE_CHUNKS chunks in equal pieces."""
    return max(1, -(-(n // 512) // ENCODE_PIECE_CHUNKS))


def counter_workload(torch, H, manifest_path):
    """The hot kernels at their BASELINE shapes, a fixed number of dispatches each, on one
    stream, phases fenced by synchronize. Writes the phase manifest (kernel-name key, how many
    dispatches of that key precede the phase, how many belong to it, algorithmic bytes and
    operations per phase) for --summarize-counters."""
    lib, st = H.encode_lib(), stream_handle(torch)
    launched = {}
    phases = []

    def phase(name, key, count, fn, nbytes=None, ops=None, elements=None, note=""):
        torch.cuda.synchronize()
        phases.append({"name": name, "kernel": key, "skip": launched.get(key, 0), "count": count,
                       "algorithmic_bytes": nbytes, "ops": ops, "elements": elements, "note": note})
        fn()
        torch.cuda.synchronize()
        launched[key] = launched.get(key, 0) + count
        log(f"counter workload: {name} ({count} dispatches)")

    def encode_pin(w):
        launched["k_encode_bf16_b64"] = launched.get("k_encode_bf16_b64", 0) + 1
        return H.encode_bf16(w, 64)

    g = torch.Generator(device="cuda").manual_seed(7001)
    # copy calibration for the byte counters
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    phase("hbm_copy_256mib", "copyBuffer", 10, lambda: [dst.copy_(src) for _ in range(10)], nbytes=10 * 2 * (256 << 20),
          note="torch device copy, the reference for scaling FETCH_SIZE / WRITE_SIZE")
    del src, dst
    # encode at the decode shape: 6 distinct inputs (704 MB, more than the 256 MB last-level cache)
    N, K = GEMV_N, GEMV_K
    ws = [(torch.randn(N * K, device="cuda", generator=g) * 0.02).to(torch.bfloat16) for _ in range(6)]
    outs = [(torch.empty(N * K // 2, dtype=torch.uint8, device="cuda"), torch.empty(N * K // 2, dtype=torch.uint8, device="cuda"),
             torch.empty(N * K // 64, dtype=torch.float32, device="cuda")) for _ in range(6)]
    phase("encode_14336x4096", "k_encode_bf16_b64", 6,
          lambda: [bound(lib.glint_encode_bf16_device, w, N * K, 64, *o, st)() for w, o in zip(ws, outs)],
          nbytes=6 * 3.0625 * N * K, elements=6 * N * K)
    del ws, outs
    # encode over the Llama-3-8B tensor set (every size a multiple of 512; one dispatch per
    # tensor, the two embedding tensors in ENCODE_PIECE_CHUNKS pieces)
    shapes = llama3_8b_shapes()
    total = sum(a * b for a, b in shapes)
    ws = [(torch.randn(a * b, device="cuda", generator=g) * 0.02).to(torch.bfloat16) for a, b in shapes]
    outs = [(torch.empty(w.numel() // 2, dtype=torch.uint8, device="cuda"),
             torch.empty(w.numel() // 2, dtype=torch.uint8, device="cuda"),
             torch.empty(w.numel() // 64, dtype=torch.float32, device="cuda")) for w in ws]
    phase("encode_model_set", "k_encode_bf16_b64", sum(encode_launches(a * b) for a, b in shapes),
          lambda: [bound(lib.glint_encode_bf16_device, w, w.numel(), 64, *o, st)() for w, o in zip(ws, outs)],
          nbytes=3.0625 * total, elements=total, note="226 Llama-3-8B tensors, 8.03e9 weights")
    del ws, outs
    torch.cuda.empty_cache()
    # decode GEMV (headline), 19 rotated pins
    pins = []
    for _ in range(19):
        pins.append(encode_pin((torch.randn(N * K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)))
    x = torch.randn(K, device="cuda", generator=g).to(torch.bfloat16)
    y = torch.empty(N, dtype=torch.bfloat16, device="cuda")
    calls = [bound(lib.launch_glint_htile_bf16_stream, p[0], p[1], p[2], x, y, 1, N, K, 64, st) for p in pins]
    phase("gemv_m1_14336x4096", GEMV_KERNEL, 38, lambda: [c() for c in calls + calls], nbytes=38 * gemv_bytes(N, K))
    # prefill on the gate shape, 6 rotated pins (373 MB)
    pins = pins[:6]
    for M, key, name in ((2048, "k_tile_big<2,GlintTileProducer,TileOutBF16,0>", "prefill_m2048_14336x4096"),
                         (64, "k_htile_rl<4,false>", "prefill_m64_14336x4096")):
        xm = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
        ym = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        calls = [bound(lib.launch_glint_htile_bf16_stream, p[0], p[1], p[2], xm, ym, M, N, K, 64, st) for p in pins]
        phase(name, key, 6, lambda: [c() for c in calls], ops=6 * 2.0 * M * N * K,
              nbytes=6 * (N * K * (1 + 4 / 64) + 2 * M * K + 2 * M * N))
        del xm, ym
    del pins
    # INT8 GEMM at the INT8 config: the raw per-row / per-column GEMM and the attach ABI
    M, N8, K8 = 2048, 8192, 8192
    A = torch.randint(-127, 128, (M, K8), device="cuda", generator=g, dtype=torch.int8)
    B = torch.randint(-127, 128, (N8, K8), device="cuda", generator=g, dtype=torch.int8)
    sa = torch.rand(M, device="cuda", generator=g) * 0.019 + 1e-3
    sb = torch.rand(N8, device="cuda", generator=g) * 0.019 + 1e-3
    o8 = torch.empty(M, N8, dtype=torch.bfloat16, device="cuda")
    phase("int8_gemm_2048x8192x8192", "k_int8_gemm_dma", 4,
          lambda: [H.int8_gemm_scaled_bf16(A, B, sa, sb, out=o8) for _ in range(4)], ops=4 * 2.0 * M * N8 * K8)
    del A, B, sa, sb, o8
    p7 = H.p7_lib()
    xb = torch.randn(M, K8, device="cuda", generator=g).to(torch.bfloat16)
    q = torch.randint(-127, 128, (N8 * K8,), device="cuda", generator=g, dtype=torch.int8)
    sc = torch.rand(N8 * K8 // 64, device="cuda", generator=g) * 0.02 + 1e-3
    yf = torch.empty(M, N8, dtype=torch.float32, device="cuda")
    xq = torch.empty(M * K8, dtype=torch.int8, device="cuda")
    sx = torch.empty(M * K8 // 64, dtype=torch.float32, device="cuda")
    lin = H.Int8MmaLinear(q.data_ptr(), sc.data_ptr(), N8, K8)
    call = bound(p7.int8_mma_gemm, xb, lin, yf, M, xq, sx, st)
    phase("int8_mma_gemm_abi_2048x8192x8192", "k_int8_mma_dma", 4, lambda: [call() for _ in range(4)],
          ops=4 * 2.0 * M * N8 * K8, note="per-64 scales, kb-ordered f32 epilogue, last step fused")
    Path(manifest_path).write_text(json.dumps({"phases": phases, "cu_num": CU_NUM, "simd_num": SIMD_NUM}, indent=1) + "\n")


def _dispatch_rows(db_path, key):
    """{counter: value} per dispatch of kernels whose name (spaces removed) contains key,
    ordered by dispatch id, with the dispatch's start and end."""
    import sqlite3
    cur = sqlite3.connect(db_path).cursor()
    rows = {}
    tables = {r[0] for r in cur.execute("select name from sqlite_master")}
    if "counters_collection" in tables:
        for did, name, ctr, val, start, end in cur.execute(
                "select dispatch_id, kernel_name, counter_name, value, start, end from counters_collection"):
            if key in name.replace(" ", ""):
                r = rows.setdefault(did, {"start": start, "end": end})
                r[ctr] = val
    if not rows:
        for did, name, start, end in cur.execute("select dispatch_id, name, start, end from kernels"):
            if key in name.replace(" ", ""):
                rows[did] = {"start": start, "end": end}
    return [rows[d] for d in sorted(rows)]


def summarize_counters(manifest, dbs, out_path=None) -> dict:
    """Per-phase HBM traffic, utilisation and kernel time from the five passes, written to
    out_path (profiles/counters_hot_kernels.json by default)."""
    import statistics
    man = json.loads(Path(manifest).read_text())
    cu, simd = man["cu_num"], man["simd_num"]
    by_phase = {}
    for tag, db in dbs.items():
        for ph in man["phases"]:
            rows = _dispatch_rows(db, ph["kernel"])[ph["skip"]:ph["skip"] + ph["count"]]
            if len(rows) != ph["count"]:
                raise SystemExit(f"{db}: {ph['name']}: {len(rows)} of {ph['count']} dispatches of {ph['kernel']}")
            by_phase.setdefault(ph["name"], {})[tag] = rows
    copy = by_phase["hbm_copy_256mib"]
    scale = {c: (256 << 20) / (statistics.mean(r[c] for r in copy[t]) * 1024.0)
             for t, c in (("fetch", "FETCH_SIZE"), ("write", "WRITE_SIZE"))}
    out = {"device": "MI355X (gfx950), one GPU", "cu_num": cu, "simd_num": simd,
           "byte_scale": {"FETCH_SIZE": scale["FETCH_SIZE"], "WRITE_SIZE": scale["WRITE_SIZE"],
                          "rule": "true bytes of 10 torch 256 MiB device copies / counter KiB * 1024"},
           "formulas": {
               "hbm_bytes": "sum over the phase of (FETCH_SIZE * fetch scale + WRITE_SIZE * write scale) * 1024",
               "VALUBusy": "100 * SQ_ACTIVE_INST_VALU / CU_NUM / GRBM_GUI_ACTIVE (rocprofv3 derived, per dispatch)",
               "MfmaUtil": "100 * SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE * SIMD_NUM) (rocprofv3 derived)",
               "LDSBankConflict": "100 * SQ_LDS_BANK_CONFLICT / GRBM_GUI_ACTIVE / CU_NUM (rocprofv3 derived)",
               "lds_active_pct": "100 * SQ_LDS_IDX_ACTIVE / GRBM_GUI_ACTIVE / CU_NUM",
               "per-dispatch percentages": "weighted by each dispatch's kernel-trace duration",
               "kernel_us": "kernel-trace durations (begin to end), summed over the phase",
               "hbm_frac": "algorithmic bytes / kernel time / 8 TB/s",
               "mfma_frac": "operations / kernel time / dense peak (bf16 2.5 PFLOP/s, int8 5.0 POP/s)"},
           "phases": {}}
    for ph in man["phases"]:
        d = by_phase[ph["name"]]
        dur = [(r["end"] - r["start"]) / 1e3 for r in d["trace"]]
        wsum = sum(dur)

        def wavg(tag, ctr):
            return sum(r[ctr] * w for r, w in zip(d[tag], dur)) / wsum

        res = {"kernel": ph["kernel"], "dispatches": ph["count"], "note": ph["note"],
               "kernel_us_total": wsum, "kernel_us_avg": wsum / len(dur)}
        fetch = sum(r["FETCH_SIZE"] for r in d["fetch"]) * 1024.0 * scale["FETCH_SIZE"]
        write = sum(r["WRITE_SIZE"] for r in d["write"]) * 1024.0 * scale["WRITE_SIZE"]
        res.update({"hbm_fetch_bytes": fetch, "hbm_write_bytes": write})
        if ph["algorithmic_bytes"]:
            res["algorithmic_bytes"] = ph["algorithmic_bytes"]
            res["traffic_over_algorithmic"] = (fetch + write) / ph["algorithmic_bytes"]
            res["hbm_frac"] = ph["algorithmic_bytes"] / (wsum * 1e-6) / 1e9 / HBM_PEAK_GBS
            res["counted_hbm_gbs"] = (fetch + write) / (wsum * 1e-6) / 1e9
        if ph["ops"]:
            peak = I8_PEAK_TOPS if "int8" in ph["name"] else BF16_PEAK_TFLOPS
            res["tera_ops_per_s"] = ph["ops"] / (wsum * 1e-6) / 1e12
            res["mfma_frac"] = res["tera_ops_per_s"] / peak
        for c in ("VALUBusy", "MfmaUtil", "LDSBankConflict"):
            res[c] = wavg("util", c)
        res["lds_active_pct"] = sum(100.0 * r["SQ_LDS_IDX_ACTIVE"] / r["GRBM_GUI_ACTIVE"] / cu * w
                                    for r, w in zip(d["inst"], dur)) / wsum
        for c in ("SQ_INSTS_VALU", "SQ_INSTS_LDS", "SQ_INSTS_MFMA", "SQ_WAVES"):
            res[c] = sum(r[c] for r in d["inst"])
        if ph["elements"]:
            res["valu_insts_per_512_elements"] = res["SQ_INSTS_VALU"] / (ph["elements"] / 512)
        out["phases"][ph["name"]] = res
    out["commands"] = [f"rocprofv3 {flags} -d <dir_{tag}> -o run -- python3 bench.py --counter-workload <dir_{tag}>/manifest.json"
                       for tag, flags in COUNTER_PASSES.items()] + [
        "python3 bench.py --summarize-counters <manifest.json> " +
        " ".join(f"{t}=<dir_{t}>/run_results.db" for t in COUNTER_PASSES)]
    Path(out_path or COUNTERS_JSON).write_text(json.dumps(out, indent=1) + "\n")
    return out


def load_counters():
    """The headline figures of profiles/counters_hot_kernels.json for the bench line."""
    try:
        c = json.loads(COUNTERS_JSON.read_text())["phases"]
    except Exception:
        return None
    pick = {"encode_model_set": ("hbm_frac", "traffic_over_algorithmic", "VALUBusy", "valu_insts_per_512_elements"),
            "encode_14336x4096": ("hbm_frac", "traffic_over_algorithmic", "VALUBusy"),
            "gemv_m1_14336x4096": ("hbm_frac", "traffic_over_algorithmic", "VALUBusy"),
            "prefill_m2048_14336x4096": ("mfma_frac", "MfmaUtil", "LDSBankConflict", "lds_active_pct"),
            "prefill_m64_14336x4096": ("hbm_frac", "mfma_frac", "MfmaUtil", "LDSBankConflict", "lds_active_pct"),
            "int8_gemm_2048x8192x8192": ("mfma_frac", "MfmaUtil"),
            "int8_mma_gemm_abi_2048x8192x8192": ("mfma_frac", "MfmaUtil", "VALUBusy")}
    return {k: {f: round(c[k][f], 4) for f in fs if f in c[k]} for k, fs in pick.items() if k in c}


def load_traffic():
    p = TRAFFIC_JSON
    if p.is_file():
        try:
            return json.loads(p.read_text()).get("traffic_bytes")
        except Exception:
            return None
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--quick", action="store_true", help="headline GEMV only")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run 10 plain 256 MiB device copies (the reference kernel for scaling PMC byte counters)")
    ap.add_argument("--headline-only", action="store_true", help="only the bf16-out 14336x4096 GEMV loop")
    ap.add_argument("--parts", default="all",
                    help="comma list of extra measurements to run (copy,encode4096,model,prefill,int8,int8abi,w8a16,"
                         "kmajor,hostabi,pintools, and gemvpair, which 'all' leaves out) or 'all'")
    ap.add_argument("--summarize-traffic", nargs=2, metavar=("FETCH_DB", "WRITE_DB"),
                    help="write the traffic figures from two rocprofv3 --pmc databases (no GPU needed)")
    ap.add_argument("--counter-workload", metavar="MANIFEST",
                    help="run the fixed hot-kernel workload for the rocprofv3 counter passes, write its manifest")
    ap.add_argument("--summarize-counters", nargs="+", metavar="ARG",
                    help="MANIFEST tag=DB ... (tags fetch, write, util, inst, trace): write the counter summary")
    ap.add_argument("--timeline", metavar="OUT",
                    help="write the per-wave timeline summary of the decode GEMV (libglint_encode_tl.so) to OUT")
    ap.add_argument("--summarize-trace", nargs="+", metavar="DB",
                    help="print the per-kernel table of a rocprofv3 --kernel-trace database [and bench JSON]")
    args = ap.parse_args()
    if args.summarize_traffic:
        print(json.dumps(summarize_traffic(*args.summarize_traffic), indent=1))
        return 0
    if args.summarize_trace:
        print(summarize_trace(*args.summarize_trace[:2]))
        return 0
    if args.summarize_counters:
        dbs = dict(a.split("=", 1) for a in args.summarize_counters[1:])
        print(json.dumps(summarize_counters(args.summarize_counters[0], dbs), indent=1))
        return 0
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
    if args.counter_workload:
        counter_workload(torch, H, args.counter_workload)
        return 0
    if args.timeline:
        gemv_timeline(torch, H, args.timeline, args.steps)
        return 0
    if args.calibrate_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    gemv, pins, x = bench_gemv(torch, H, args.steps, args.warmup, args.headline_only)
    log(f"gemv {gemv['ms'] * 1e3:.2f} us {gemv['gbs']:.0f} GB/s")
    del pins
    torch.cuda.empty_cache()
    extra = {}
    parts = set(args.parts.split(",")) if args.parts != "all" else {
        "copy", "encode4096", "model", "prefill", "int8", "int8abi", "w8a16", "kmajor", "hostabi", "pintools"}
    if not args.quick:
        if "copy" in parts:
            extra["hbm_copy_1gib"] = bench_copy_ceiling(torch)
            log(f"device copy 1 GiB {extra['hbm_copy_1gib']['gbs']:.0f} GB/s (read + write)")
            extra["hbm_read"] = bench_read_ceiling(torch, H, args.steps)
            log(f"read ceiling: 1 GiB {extra['hbm_read']['stream_1gib']['gbs']:.0f} GB/s, GEMV-sized "
                f"{extra['hbm_read']['gemv_sized']['ms'] * 1e3:.2f} us ({extra['hbm_read']['gemv_sized']['frac']:.3f})")
        if "encode4096" in parts:
            extra["encode_4096x4096"] = bench_encode_4096(torch, H)
            log(f"encode 4096^2 {extra['encode_4096x4096']['encode_bf16_in_gbs']:.0f} GB/s bf16-in")
        if "model" in parts:
            extra["model_encode"] = bench_model_encode(torch, H, passes=3)
            log(f"model encode {extra['model_encode']['encode_bf16_in_gbs']:.0f} GB/s bf16-in")
        if "prefill" in parts:
            extra["prefill"] = bench_prefill(torch, H, steps=12)
            log("prefill " + ", ".join(f"{k} {v['ms'] * 1e3:.1f} us (f32 out {v['f32_out']['ms'] * 1e3:.1f})"
                                       for k, v in extra["prefill"].items() if k != "batched_decode"))
            log("batched decode " + ", ".join(f"{k} {v['ms'] * 1e3:.1f} us (f32 out {v['f32_out']['ms'] * 1e3:.1f})"
                                              for k, v in extra["prefill"]["batched_decode"].items()))
        if "int8" in parts:
            extra["int8_gemm"] = bench_int8(torch, H, steps=10)
            log(f"int8 {extra['int8_gemm']['tops']:.0f} TOPS")
        if "int8abi" in parts:
            extra["int8_mma_gemm_abi"] = bench_int8_abi(torch, H, steps=10)
            log("int8_mma_gemm abi " + ", ".join(f"{k} {v['ms'] * 1e3:.1f} us"
                                                 for k, v in extra["int8_mma_gemm_abi"].items()))
        if "w8a16" in parts:
            extra["w8a16"] = bench_w8a16(torch, H, steps=10)
            log("w8a16 done")
        if "gemvpair" in parts:
            extra["gemv_pair"] = bench_gemv_pair(torch, H, args.steps, args.warmup)
            gp = extra["gemv_pair"]
            log(f"gate/up pair on two streams {gp['two_streams']['ms_per_gemv'] * 1e3:.2f} us per GEMV "
                f"({gp['two_streams']['frac']:.3f}); stacked 28672x4096 {gp['stacked_28672x4096']['ms'] * 1e3:.2f} us "
                f"({gp['stacked_28672x4096']['frac']:.3f})")
        if "kmajor" in parts:
            extra["kmajor_decode"] = bench_kmajor(torch, H)
            log(f"k-major fold {extra['kmajor_decode']['fold_ms'] * 1e3:.1f} us")
        if "hostabi" in parts:
            extra["host_abi_pcie"] = bench_host_abi(H)
            log(f"host ABI encode {extra['host_abi_pcie']['encode_bf16_in_gbs']:.1f} GB/s bf16-in (PCIe inclusive)")
        if "pintools" in parts:
            extra["pin_tools"] = bench_pin_tools()
            log(f"pin tools convert {extra['pin_tools']['convert_bf16_in_gbs']:.2f} GB/s bf16-in "
                "(files and PCIe inclusive)")
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
        "counters": load_counters(),
        "gemv": gemv,
        **extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
