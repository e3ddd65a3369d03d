#!/usr/bin/env python3
"""Benchmark of the MXFP4 A4W4 GEMM on one MI355X.

    python bench.py [--gpus 1] [--steps 200] [--warmup 150]

Headline workload: C[8192,8192] bf16 =
dequant(A)·dequant(B)^T with M=N=K=8192, operands drawn by the seeded
generator (A ~ N(0,1) with 1% of K-channels x20, W ~ N(0,0.02)), quantized
to MXFP4 and preshuffled on the GPU by this package, resident in HBM before
timing.  A step is one call of the drop-in operator mbs_gemm_a4w4.gemm_a4w4.

Also reported (same JSON line): the decode shapes of configs[2]
(M in {1,4,16,32}, N=K=8192) measured cold -- ten rotating weight copies,
more than the 256 MB MALL -- replayed from a HIP graph; and the CPU baseline
(the oracle's restatement of the reference's run_torch on this host's cores,
on a bounded sample); the grouped (mixture-of-experts) GEMM on
configs[3]'s expert shapes, one launch against one dense launch per expert;
and the activation quantizer (bf16 -> MXFP4) against HBM bandwidth.

One GPU only: --gpus above 1 exits with an explanation.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MXFP4 GEMM TFLOPS & % FP4 MFMA peak (M=N=K=8192); decode HBM GB/s (M=1–16)"
PEAK_FP4_TFLOPS = 10100.0      # MI355X dense MXFP4 MFMA
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E


def algo_bytes(M, N, K):
    return M * K // 2 + N * K // 2 + (M + N) * K // 32 + 2 * M * N


def prepare(M, N, K, cfg, dev):
    """Seeded bf16 operands -> MXFP4 bytes on the GPU (product kernels)."""
    import mbs_amd
    from mbs_amd import synthetic

    x, w = synthetic.make_operands(cfg, M, N, K)
    xd, wd = x.to(dev), w.to(dev)
    A, As = mbs_amd.quantize_mxfp4(xd, shuffle=True)
    Wp, Bs = mbs_amd.quantize_mxfp4(wd, shuffle=True)
    B = mbs_amd.shuffle_weight(Wp)
    del xd, wd, Wp
    return (A, B, As, Bs), (x, w)


def time_steps(fn, steps, warmup):
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(s)
    for _ in range(steps):
        fn()
    e1.record(s)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return e0.elapsed_time(e1) / 1e3, wall   # seconds (events), seconds (host clock)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def graph_blocks(fn, launches=100, blocks=7):
    """The reference's timing method (asm_vs_wg_kernel.md:179-180): a HIP
    graph of `launches` back-to-back calls (L2 warm), replayed `blocks` times;
    returns the per-launch microseconds of every block."""
    import torch

    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(launches):
            fn()
    g.replay()
    torch.cuda.synchronize()
    out = []
    for _ in range(blocks):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        out.append(e0.elapsed_time(e1) * 1e3 / launches)
    del g
    return out


def phase_lib():
    """ctypes handle on the phase-timer build of the C library, or None."""
    import ctypes

    import mbs_amd

    path = os.path.join(mbs_amd.LIB_DIR, "libmbs_gemm_phase.so")
    if not os.path.exists(path):
        return None
    L = ctypes.CDLL(path)
    P, I, S = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    L.mbs_gemm_a4w4_launch.argtypes = [P, P, P, P, P, P, P, I, I, I, I, I, P, S, P]
    L.mbs_gemm_a4w4_launch.restype = I
    L.mbs_gemm_a4w4_launch_config.argtypes = [I, I, P, P, P, P, P, P, P, I, I, I, I, I, P, S, P]
    L.mbs_gemm_a4w4_launch_config.restype = I
    L.mbs_gemm_a4w4_workspace_bytes.argtypes = [I, I, I]
    L.mbs_gemm_a4w4_workspace_bytes.restype = S
    L.mbs_phase_timer_attach.argtypes = [P]
    L.mbs_phase_timer_slots.restype = I
    return L


PHASES = ("prologue", "stage_wait", "barrier", "stage_body", "epilogue", "next_unit")


def phase_split(ops, M, N, K, launches=20, config=None):
    """In-kernel cycle split of the persistent GEMM on operands `ops` (the
    phase-timer build: s_memtime per phase per wave), with the shader clock
    from s_memtime / s_memrealtime and the kernel time with and without the
    timer (HIP events, eager launches).  `config`: a persistent configuration
    name to force (one split) instead of the planner's plan."""
    import ctypes

    import torch

    import mbs_amd

    L = phase_lib()
    if L is None:
        return {"error": "libmbs_gemm_phase.so not built (python -m mbs_amd._build --phase-timer)"}
    A, B, As, Bs = ops
    dev = A.device
    Mpad, snp = mbs_amd.round_up(M, 32), mbs_amd.scale_pad(K)
    out = torch.empty(Mpad, N, dtype=torch.bfloat16, device=dev)
    wsb = L.mbs_gemm_a4w4_workspace_bytes(M, N, K)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    slots = L.mbs_phase_timer_slots()
    sums = torch.zeros(1024 * slots, dtype=torch.int64, device=dev)   # per workgroup
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    strm = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    cfg = -1
    if config:
        L.mbs_gemm_a4w4_config_name.restype = ctypes.c_char_p
        names = [L.mbs_gemm_a4w4_config_name(i).decode() for i in range(L.mbs_gemm_a4w4_num_configs())]
        cfg = names.index(config)

    def call():
        if cfg >= 0:
            st = L.mbs_gemm_a4w4_launch_config(cfg, 1, p(A), p(B), p(As), p(Bs), None, None, p(out), M, N, K,
                                               Mpad, snp, p(ws), wsb, strm())
        else:
            st = L.mbs_gemm_a4w4_launch(p(A), p(B), p(As), p(Bs), None, None, p(out), M, N, K, Mpad, snp,
                                        p(ws), wsb, strm())
        assert st == 0, st

    def timed(n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            call()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / n

    L.mbs_phase_timer_attach(None)
    for _ in range(5):
        call()
    torch.cuda.synchronize()
    us_plain = timed(launches)
    L.mbs_phase_timer_attach(p(sums))
    us_timed = timed(launches)
    L.mbs_phase_timer_attach(None)
    v = [int(x) for x in sums.view(1024, slots).sum(0).cpu().tolist()]
    cyc = dict(zip(PHASES, v[:len(PHASES)]))
    total = sum(cyc.values())
    stages, units, clk, rt = v[len(PHASES):len(PHASES) + 4]
    res = {
        "shape": [M, N, K], "plan": config or mbs_amd.ext().plan_name(M, N, K), "launches": launches,
        "kernel_us_plain": round(us_plain, 2), "kernel_us_timed": round(us_timed, 2),
        "sclk_mhz": round(clk / rt * 100.0, 1) if rt else None,
        "wave_cycles": total,
        "fraction": {k: round(c / total, 4) for k, c in cyc.items()} if total else None,
        "cycles_per_stage": {k: round(cyc[k] / stages, 1) for k in ("stage_wait", "barrier", "stage_body")}
        if stages else None,
        "epilogue_cycles_per_unit": round(cyc["epilogue"] / units, 1) if units else None,
        "next_unit_cycles_per_unit": round(cyc["next_unit"] / units, 1) if units else None,
        "stages": stages, "units": units,
    }
    return res


def stream_floor(dev, nbytes=None, copies=10, replays=20, grids=(256, 512, 1024, 2048)):
    """The streaming-read floor of the decode shapes: libmbs_probe.so reads
    `nbytes` (default: the bytes of a decode GEMM at N=K=8192, M=1) with
    16-byte non-temporal loads, cold over `copies` rotating buffers (more
    than the 256 MB MALL), graph-replayed; best grid of `grids`."""
    import ctypes

    import torch

    import mbs_amd

    path = os.path.join(mbs_amd.LIB_DIR, "libmbs_probe.so")
    if not os.path.exists(path):
        return {"error": "libmbs_probe.so not built"}
    L = ctypes.CDLL(path)
    L.mbs_probe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int,
                                        ctypes.c_void_p]
    if nbytes is None:
        nbytes = (algo_bytes(1, 8192, 8192) + 4095) // 4096 * 4096
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1) for _ in range(copies)]
    sink = torch.empty(max(grids) * 4, dtype=torch.int32, device=dev)
    res = {}
    for grid in grids:
        def run():
            st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for b in bufs:
                assert L.mbs_probe_stream_read(ctypes.c_void_p(b.data_ptr()), nbytes,
                                               ctypes.c_void_p(sink.data_ptr()), grid, st) == 0
        run()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            run()
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(replays):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        res[grid] = e0.elapsed_time(e1) * 1e3 / (replays * copies)
        del g
    best = min(res, key=res.get)
    us = res[best]
    return {"bytes": nbytes, "us": round(us, 3), "GBps": round(nbytes / us / 1e3, 1),
            "frac_hbm": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4), "grid": best,
            "us_by_grid": {str(k): round(v, 3) for k, v in res.items()},
            "method": f"cold, {copies} rotating buffers, graph of {copies} launches replayed {replays}x"}


def decode_bench(dev, Ms=(1, 4, 8, 16, 32), N=8192, K=8192, copies=10, replays=20):
    """Cold (rotating copies) and warm per-launch time of the decode shapes,
    from HIP-graph replay so host launch overhead is excluded.  Also, cold,
    the reference's decode flow from a bf16 activation: quantize_mxfp4, then
    gemm_a4w4 (two launches), and the same product in one launch
    (gemm_a4w4_from_bf16(one_launch=True): the decode kernel quantizes in
    registers); for M <= 8 also both with MBS activations (quantize_mxfp4_mbs
    and the factor GEMM, against the one-launch MBS form)."""
    import torch

    import mbs_amd

    def two_step(x, B, Bs):
        a, s = mbs_amd.quantize_mxfp4(x, shuffle=True)
        return mbs_amd.gemm_a4w4(a, B, s, Bs)

    def two_step_mbs(x, B, Bs, Bf):
        a, s, f = mbs_amd.quantize_mxfp4_mbs(x, shuffle=True)
        return mbs_amd.gemm_a4w4(a, B, s, Bs, f, Bf)

    (_, B, _, Bs), _ = prepare(32, N, K, 2, dev)
    Bc = [B.clone() for _ in range(copies)]
    Bsc = [Bs.clone() for _ in range(copies)]
    Bf = torch.randint(0, 256, (N,), dtype=torch.uint8, generator=torch.Generator().manual_seed(7)).to(dev)
    del B, Bs
    res = {}
    for M in Ms:
        (A, _, As, _), (xh, _) = prepare(M, 16, K, 2, dev)
        x = xh.to(dev)
        modes = ["cold", "warm", "quantize+gemm", "one_launch"]
        if M <= 8:   # MBS activations (the one-launch MBS form takes M <= 8)
            modes += ["quantize_mbs+gemm", "one_launch_mbs"]
        for mode in modes:
            idx = [0] * copies if mode == "warm" else list(range(copies))
            if mode == "quantize+gemm":
                run = lambda: [two_step(x, Bc[i], Bsc[i]) for i in idx]
            elif mode == "one_launch":
                run = lambda: [mbs_amd.gemm_a4w4_from_bf16(x, Bc[i], Bsc[i], one_launch=True)
                               for i in idx]
            elif mode == "quantize_mbs+gemm":
                run = lambda: [two_step_mbs(x, Bc[i], Bsc[i], Bf) for i in idx]
            elif mode == "one_launch_mbs":
                run = lambda: [mbs_amd.gemm_a4w4_from_bf16(x, Bc[i], Bsc[i], B_factor=Bf,
                                                           one_launch=True) for i in idx]
            else:
                run = lambda: [mbs_amd.gemm_a4w4(A, Bc[i], As, Bsc[i]) for i in idx]
            run()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                run()
            g.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(replays):
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (replays * copies)
            gbs = algo_bytes(M, N, K) / (us * 1e-6) / 1e9
            if mode not in ("cold", "warm"):
                res.setdefault(f"M={M}", {})[f"cold_{mode}_us"] = round(us, 3)
            else:
                res.setdefault(f"M={M}", {})[mode] = {
                    "us": round(us, 3), "GBps": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}
            del g
        res[f"M={M}"]["plan"] = mbs_amd.ext().plan_name(M, N, K)
    return res


def quantize_bench(dev, shapes=((8192, 8192), (2048, 7168), (32, 8192)), replays=5, reps=3):
    """The activation quantizer (bf16 -> packed e2m1 + shuffled E8M0, the
    reference's aiter per_1x32 step) on configs[1]'s A, configs[3]'s
    M=2048 x K=7168 A and a decode-sized A: HIP-graph replays of 10 calls,
    HBM bytes = 2*R*K read + R*K/2 + R*K/32 written, against 8 TB/s."""
    import torch

    import mbs_amd

    g = torch.Generator(device=dev)
    g.manual_seed(1005)
    res = {}
    for R, K in shapes:
        x = torch.randn(R, K, generator=g, device=dev).to(torch.bfloat16)
        call = lambda: mbs_amd.quantize_mxfp4(x, shuffle=True)
        call()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for _ in range(10):
                call()
        gr.replay()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(replays):
                gr.replay()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e3 / (replays * 10))
        us = statistics.median(ts)
        nbytes = 2 * R * K + R * K // 2 + R * K // 32
        gbs = nbytes / (us * 1e-6) / 1e9
        res[f"{R}x{K}"] = {"us": round(us, 2), "GBps": round(gbs, 1),
                           "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}
        del gr, x
    return res


def grouped_bench(dev, experts=8, rows=256, shapes=((7168, 2048), (4096, 7168), (2112, 7168)),
                  replays=10):
    """Grouped GEMM over `experts` experts of `rows` tokens each (configs[3]'s
    M=256 expert shapes, 8 experts = 2048 tokens): one grouped launch against
    one dense launch per expert, both replayed from HIP graphs."""
    import torch

    import mbs_amd

    g = torch.Generator(device=dev)
    g.manual_seed(1003)
    M = experts * rows
    offs = torch.arange(0, M + 1, rows, dtype=torch.int32, device=dev)
    res = {}
    for N, K in shapes:
        x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        w = (torch.randn(experts * N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        A, As = mbs_amd.quantize_mxfp4(x, shuffle=True)
        Bp, Bs_all = [], []
        for e in range(experts):
            wq, ws = mbs_amd.quantize_mxfp4(w[e * N:(e + 1) * N], shuffle=True)
            Bp.append(mbs_amd.shuffle_weight(wq))
            Bs_all.append(ws.reshape(-1))
        B, Bs = torch.stack(Bp), torch.stack(Bs_all)
        snp = ((K + 31) // 32 + 7) // 8 * 8
        grouped = lambda: mbs_amd.gemm_a4w4_grouped(A, B, As, Bs, offs)
        dense = lambda: [mbs_amd.gemm_a4w4(A[e * rows:(e + 1) * rows], B[e],
                                           As.reshape(-1)[e * rows * snp:(e + 1) * rows * snp], Bs[e])
                         for e in range(experts)]
        times = {}
        for name, fn in (("grouped", grouped), ("per_expert", dense)):
            fn()
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                fn()
            gr.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(replays):
                gr.replay()
            e1.record()
            torch.cuda.synchronize()
            times[name] = e0.elapsed_time(e1) * 1e3 / replays
            del gr
        flops = 2.0 * M * N * K
        res[f"{experts}x{rows}x{N}x{K}"] = {
            "grouped_us": round(times["grouped"], 2), "per_expert_us": round(times["per_expert"], 2),
            "grouped_TFLOPS": round(flops / times["grouped"] / 1e6, 1),
            "speedup_vs_per_expert": round(times["per_expert"] / times["grouped"], 3)}
        del A, As, B, Bs, Bp, Bs_all, x, w
    return res


def cpu_baseline(x, w, rows=8192, reps=3):
    """The oracle's run_torch restatement (dequant to fp32, torch.mm fp32,
    bf16) on this host: `rows` rows of the config-1 A against the full W.
    The three steps are timed separately (median of `reps` each) and the
    total is their sum: run_torch runs them one after the other."""
    import torch

    import oracle  # the CPU checker; timed here as the reported baseline

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    xp, xs = oracle.quantize_mxfp4(x[:rows].float().numpy())
    wp, ws = oracle.quantize_mxfp4(w.float().numpy())
    N, K = w.shape
    t_dq, t_mm, t_bf = [], [], []
    for _ in range(reps):
        t0 = time.perf_counter()
        xf = oracle.dequant_mxfp4(xp, xs)
        wf = oracle.dequant_mxfp4(wp, ws)
        t1 = time.perf_counter()
        c = torch.mm(torch.from_numpy(xf), torch.from_numpy(wf).T).numpy()
        t2 = time.perf_counter()
        oracle.epilogue_bf16(c)
        t3 = time.perf_counter()
        t_dq.append(t1 - t0)
        t_mm.append(t2 - t1)
        t_bf.append(t3 - t2)
        del xf, wf, c
    dq, mm, bf = (statistics.median(t) for t in (t_dq, t_mm, t_bf))
    t = dq + mm + bf
    flops = 2.0 * rows * N * K
    return {
        "value": round(flops / t / 1e12, 4), "unit": "TFLOPS", "cores": cores, "kind": "port",
        "cpu_model": cpu_model(),
        "dequant_s": round(dq, 3), "matmul_s": round(mm, 3), "bf16_s": round(bf, 3),
        "total_s": round(t, 3), "matmul_TFLOPS": round(flops / mm / 1e12, 4),
        "sample": f"config-1 rows 0..{rows - 1} of A x full W ({rows}x{N}x{K}): oracle dequant (C) "
                  f"+ fp32 torch.mm + bf16, each step median of {reps}",
    }


def shape_bench(M, N, K, iters):
    """One shape, as the reference's bench_one.py drives it (bench_one.py:1-48):
    bf16 x, w ~ N(0,1) quantized to MXFP4, 10 warmup calls, then `iters`
    timed calls of gemm_a4w4 between two events on the current stream."""
    import torch

    import mbs_amd

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    w = torch.randn(N, K, generator=g, device=dev).to(torch.bfloat16)
    A, As = mbs_amd.quantize_mxfp4(x, shuffle=True)
    Wp, Bs = mbs_amd.quantize_mxfp4(w, shuffle=True)
    B = mbs_amd.shuffle_weight(Wp)
    call = lambda: mbs_amd.gemm_a4w4(A, B, As, Bs)
    for _ in range(10):
        call()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        call()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / iters
    tflops = M * N * K * 2 / us / 1e6
    print(f"mbs  M={M} N={N} K={K}  {us:8.2f} us  {tflops:8.1f} TFLOPS", flush=True)
    print(json.dumps({"shape": [M, N, K], "us": round(us, 3), "TFLOPS": round(tflops, 1),
                      "TB/s_ref": round((A.numel() + B.numel()) / us / 1e6, 4),
                      "plan": mbs_amd.ext().plan_name(M, N, K), "iters": iters}), flush=True)


def operand_data(dev, launches=100, rounds=2):
    """configs[1]'s kernel (same plan, same instruction stream) on its own
    operands and on operands with less bit activity: A or B or both all-zero
    codes, and A all 1.0 codes.  Per case the phase-timer build's kernel time
    (HIP events, eager launches) and in-kernel shader clock; the cases are
    interleaved (order reversed in the second round), so the power
    management's state is shared between them."""
    import torch

    M = N = K = 8192
    (A, B, As, Bs), _ = prepare(M, N, K, 1, dev)
    cases = [("cfg1", (A, B, As, Bs)),
             ("A=0", (torch.zeros_like(A), B, As, Bs)),
             ("B=0", (A, torch.zeros_like(B), As, Bs)),
             ("A=B=0", (torch.zeros_like(A), torch.zeros_like(B), As, Bs)),
             ("A=1.0", (torch.full_like(A, 0x22), B, As, Bs))]   # e2m1 code 2 = 1.0 in both nibbles
    res = {}
    for r in range(rounds):
        for name, ops in (cases if r % 2 == 0 else cases[::-1]):
            ph = phase_split(ops, M, N, K, launches=launches)
            if "error" in ph:
                return ph
            res.setdefault(name, []).append({"kernel_us": ph["kernel_us_plain"], "sclk_mhz": ph["sclk_mhz"]})
    flop = 2.0 * M * N * K
    return {name: {"kernel_us": [v["kernel_us"] for v in vs], "sclk_mhz": [v["sclk_mhz"] for v in vs],
                   "TFLOPS_best": round(flop / min(v["kernel_us"] for v in vs) / 1e6, 1)}
            for name, vs in res.items()}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    # Defaults: under sustained fp4 MFMA load the GPU's power management
    # first lowers the clock (launches ~10-25 after idle run up to 35% slower)
    # and settles after ~100 launches (profiles/gemm_cfg1_power_ramp.txt); 150
    # warmup launches put the 200 timed ones in the settled state (~80 ms).
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=150)
    ap.add_argument("--no-decode", action="store_true", help="skip the decode shapes")
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-grouped", action="store_true", help="skip the grouped (MoE) shapes")
    ap.add_argument("--no-quantize", action="store_true", help="skip the activation quantizer")
    ap.add_argument("--decode-only", action="store_true",
                    help="only run the decode shapes (cold and warm graph replays) and print "
                         "their block; for counter runs of the decode kernel")
    ap.add_argument("--shape", type=str, default=None, metavar="M,N,K",
                    help="only time one shape the way the reference's bench_one.py does "
                         "(10 warmup + --iters timed calls) and print it")
    ap.add_argument("--iters", type=int, default=50, help="timed calls of --shape")
    ap.add_argument("--phase-split", action="store_true",
                    help="only print the in-kernel phase split of configs[1] (or --shape) from "
                         "the phase-timer build")
    ap.add_argument("--config", type=str, default="",
                    help="with --phase-split: force this persistent configuration (by name, one split)")
    ap.add_argument("--sustain", type=int, default=0, metavar="N",
                    help="only run N back-to-back eager launches of configs[1] after 1 s idle and "
                         "print their event times (for a kernel trace of the clock's response)")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the graph-replayed blocks and the in-kernel clock measurement "
                         "(hardware-counter runs see only the timed launches)")
    ap.add_argument("--operand-data", action="store_true",
                    help="only time configs[1]'s kernel on its operands and on all-zero / "
                         "constant operands (phase-timer build: kernel time and shader clock)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run 20 device-to-device copies of MIB MiB (scales the HBM "
                         "FETCH_SIZE/WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.calibrate_copy:
        import torch

        a = torch.ones(args.calibrate_copy << 20, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(20):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": a.numel(), "copies": 20}))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures a single MI355X; the MXFP4 GEMM is a one-GPU "
              "kernel here (a shard across GPUs is an ordinary (M, N/g, K) problem; no "
              "multi-GPU run is part of it). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    import mbs_amd

    dev = torch.device("cuda:0")
    if args.decode_only:
        print(json.dumps({"decode": decode_bench(dev), "stream_floor": stream_floor(dev)}), flush=True)
        return
    if args.sustain:
        ops, _ = prepare(8192, 8192, 8192, 1, dev)
        step = lambda: mbs_amd.gemm_a4w4(*ops)
        step()
        torch.cuda.synchronize()
        time.sleep(1.0)
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.sustain)]
        for e0, e1 in ev:
            e0.record()
            step()
            e1.record()
        torch.cuda.synchronize()
        us = [round(e0.elapsed_time(e1) * 1e3, 1) for e0, e1 in ev]
        print(json.dumps({"sustain_us": us, "first8_mean": round(statistics.mean(us[:8]), 1),
                          "last50_mean": round(statistics.mean(us[-50:]), 1)}), flush=True)
        return
    if args.shape and not args.phase_split:
        M, N, K = (int(v) for v in args.shape.split(","))
        shape_bench(M, N, K, args.iters)
        return
    if args.operand_data:
        print(json.dumps({"operand_data": operand_data(dev)}), flush=True)
        return
    if args.phase_split:
        M, N, K = (int(v) for v in args.shape.split(",")) if args.shape else (8192, 8192, 8192)
        ops, _ = prepare(M, N, K, 1, dev)
        print(json.dumps({"phase_split": phase_split(ops, M, N, K, config=args.config or None)}), flush=True)
        return
    M = N = K = 8192
    (A, B, As, Bs), (x, w) = prepare(M, N, K, 1, dev)
    step = lambda: mbs_amd.gemm_a4w4(A, B, As, Bs)
    t_ev, t_wall = time_steps(step, args.steps, args.warmup)
    t_step = max(t_ev, t_wall)
    flops = 2.0 * M * N * K
    tflops = flops * args.steps / t_step / 1e12
    kern_us = t_ev / args.steps * 1e6
    achieved = flops / (kern_us * 1e-6) / 1e12
    # the reference's method: median of 7 graph-replayed blocks of 100 launches
    blocks = [0.0] if args.no_extras else graph_blocks(step)
    med = statistics.median(blocks)
    # the shader clock the kernel runs at, from the phase-timer build
    # (s_memtime / s_memrealtime inside the same kernel on the same operands)
    ph = {} if args.no_extras else phase_split((A, B, As, Bs), M, N, K, launches=10)

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_cfg1.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    line = {
        "metric": METRIC, "value": round(tflops, 2), "unit": "TFLOPS", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(t_step / args.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "mxfp4",
        "data": "synthetic (seeded; BASELINE configs[1] distributions, quantized on-GPU)",
        "config": {"workload": "configs[1]: MXFP4 A4W4 GEMM M=N=K=8192, bf16 out",
                   "M": M, "N": N, "K": K, "plan": mbs_amd.ext().plan_name(M, N, K)},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP4_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP4_TFLOPS, 4),
                     "traffic": traffic, "kernel_us": round(kern_us, 2),
                     "algorithmic_bytes": algo_bytes(M, N, K)},
        "graph_replay": {"method": "7 blocks x 100 launches, HIP graph, L2 warm (the reference's)",
                         "us_median": round(med, 2), "us_blocks": [round(b, 2) for b in blocks],
                         "TFLOPS_median": round(flops / med / 1e6, 1) if med else None,
                         "frac_median": round(flops / med / 1e6 / PEAK_FP4_TFLOPS, 4) if med else None},
        # the reference's narrow "TB/s" column: packed A and B only
        # (test_gemm_a4w4.py:168-170)
        "TBps_ref": round((A.numel() + B.numel()) / kern_us / 1e6, 4),
        "sclk_mhz": ph.get("sclk_mhz"),
        "sclk_source": "s_memtime / s_memrealtime inside the GEMM kernel (phase-timer build, "
                       "same operands, 10 launches after the timed block)",
        "peak_at_sclk": round(PEAK_FP4_TFLOPS * ph["sclk_mhz"] / 2400.0, 1) if ph.get("sclk_mhz") else None,
    }
    if not args.no_decode:
        line["decode"] = decode_bench(dev)
        line["decode"]["stream_floor"] = stream_floor(dev)
    del A, B, As, Bs
    if not args.no_grouped:
        line["grouped"] = grouped_bench(dev)
    if not args.no_quantize:
        line["quantize"] = quantize_bench(dev)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(x, w)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
