#!/usr/bin/env python3
"""Side-by-side GPU timing of this library's GEMM and the reference's own
kernel (built from its sources into oracle/_ref/libref_gemm.so by
oracle/Makefile), on identical operand bytes.  Test infrastructure: run by
hand on a GPU box, not collected by pytest.

    python tests/compare_ref_kernel.py [--replays 10] [--rounds 7]

For every shape both launchers get the same A, B, scales (and factors where
the reference's workgroup path needs them: kernel/gemm_a4w4.hip:1044-1146
takes its factor pointers unconditionally there), the outputs are compared
against each other with the north-star tolerance, and each launcher is timed
by HIP-graph replay (one graph of `copies` launches; a timed block replays it
`replays` times; `rounds` interleaved rounds of one block per launcher, the
order alternating; medians).  Decode shapes rotate ten weight copies (cold: more bytes than the
MALL); large shapes reuse one copy, as the reference's own measurement does
(asm_vs_wg_kernel.md:179-180).  Prints one JSON object per shape.

    python tests/compare_ref_kernel.py --only MxNxK --eager 4 [--own-configs a,b]

launches each kernel 4 times eagerly (synchronised, untimed) instead: the
form for hardware-counter runs (rocprofv3 --pmc ... -- python3 ...), which
then see the reference's kernel, this library's plan and any named
configurations on the same bytes.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

REF = os.path.join(ROOT, "oracle", "_ref", "libref_gemm.so")
SYM = "_Z22gemm_a4w4_mxfp4_launchPKhS0_S0_S0_S0_S0_PviiiiiS1_"

# (M, N, K, factors): the reference's published shapes (asm_vs_wg_kernel.md:191-196),
# the headline 8192^3, and the decode slice (single-wave path: no factors).
SHAPES = [
    (8192, 8192, 8192, True),
    (8192, 17408, 5120, True),
    (8192, 5120, 17408, True),
    (8192, 10240, 5120, True),
    (8192, 12288, 5120, True),
    (1024, 17408, 5120, True),
    (1024, 1024, 5120, True),
    # BASELINE configs 3 and 4 (reference: workgroup path, which needs the
    # factors, when K % 1024 == 0; otherwise its single-wave path, without)
    (256, 7168, 2048, True), (2048, 7168, 2048, True),
    (256, 4096, 7168, True), (2048, 4096, 7168, True),
    (256, 2112, 7168, True), (2048, 2112, 7168, True),
    (1000, 1280, 512, False), (3333, 5120, 512, False),
    (1000, 5120, 12288, True), (3333, 1280, 12288, True),
    (1, 8192, 8192, False),
    (4, 8192, 8192, False),
    (16, 8192, 8192, False),
    (32, 8192, 8192, False),
]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--replays", type=int, default=10, help="graph replays per timed block")
    ap.add_argument("--rounds", type=int, default=7, help="interleaved rounds (median)")
    ap.add_argument("--only", type=str, default="", help="comma list of MxNxK to run")
    ap.add_argument("--eager", type=int, default=0, metavar="N",
                    help="N synchronised eager launches of each kernel, no timing (counter runs)")
    ap.add_argument("--own-configs", type=str, default="",
                    help="with --eager: also launch these named configurations")
    args = ap.parse_args()

    import torch

    import mbs_amd
    from gpu_util import assert_close, bf16_to_f32, clib

    if not os.path.exists(REF):
        sys.exit("reference kernel library not built: " + REF)
    P, I = ctypes.c_void_p, ctypes.c_int
    ref = getattr(ctypes.CDLL(REF), SYM)
    ref.argtypes = [P, P, P, P, P, P, P, I, I, I, I, I, P]
    ref.restype = ctypes.c_bool
    L = clib()
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    only = {s for s in args.only.split(",") if s}

    for M, N, K, factors in SHAPES:
        if only and f"{M}x{N}x{K}" not in only:
            continue
        print(f"[case] {M}x{N}x{K} factors={factors}", file=sys.stderr, flush=True)
        x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        w = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        A, As = mbs_amd.quantize_mxfp4(x, shuffle=True)
        Wq, Bs = mbs_amd.quantize_mxfp4(w, shuffle=True)
        B = mbs_amd.shuffle_weight(Wq)
        del x, w, Wq
        Mpad = (M + 31) // 32 * 32
        snp = ((K + 31) // 32 + 7) // 8 * 8
        cold = M <= 32
        copies = 10 if cold else 4
        Bc = [B] + [B.clone() for _ in range(copies - 1)] if cold else [B] * copies
        Bsc = [Bs] + [Bs.clone() for _ in range(copies - 1)] if cold else [Bs] * copies
        Af = torch.randint(0, 256, (M,), dtype=torch.uint8, device=dev, generator=g) if factors else None
        Bf = torch.randint(0, 256, (N,), dtype=torch.uint8, device=dev, generator=g) if factors else None
        pf = lambda t: None if t is None else P(t.data_ptr())
        out_ref = torch.zeros(Mpad, N, dtype=torch.bfloat16, device=dev)
        out_own = torch.zeros(Mpad, N, dtype=torch.bfloat16, device=dev)
        ws_bytes = L.mbs_gemm_a4w4_workspace_bytes(M, N, K)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)

        def launch_ref(i):
            s = P(torch.cuda.current_stream().cuda_stream)
            return ref(P(A.data_ptr()), P(Bc[i].data_ptr()), P(As.data_ptr()), P(Bsc[i].data_ptr()),
                       pf(Af), pf(Bf), P(out_ref.data_ptr()), M, N, K, Mpad, snp, s)

        def launch_own(i):
            s = P(torch.cuda.current_stream().cuda_stream)
            st = L.mbs_gemm_a4w4_launch(P(A.data_ptr()), P(Bc[i].data_ptr()), P(As.data_ptr()),
                                        P(Bsc[i].data_ptr()), pf(Af), pf(Bf), P(out_own.data_ptr()),
                                        M, N, K, Mpad, snp, P(ws.data_ptr()), ws_bytes, s)
            assert st == 0, L.mbs_last_error()
            return True

        if not launch_ref(0) and factors:
            # the reference took its single-wave path, which refuses factors:
            # compare both without them
            factors = False
            Af = Bf = None
            if not launch_ref(0):
                print(json.dumps({"shape": [M, N, K], "reference": "refused"}), flush=True)
                continue
        launch_own(0)
        torch.cuda.synchronize()
        got, want = bf16_to_f32(out_own[:M]), bf16_to_f32(out_ref[:M])
        ratio = assert_close(got, want, "ours vs reference kernel")
        if args.eager:
            L.mbs_gemm_a4w4_config_name.restype = ctypes.c_char_p
            names = [L.mbs_gemm_a4w4_config_name(i).decode() for i in range(L.mbs_gemm_a4w4_num_configs())]
            for _ in range(args.eager):
                launch_ref(0)
                torch.cuda.synchronize()
            for _ in range(args.eager):
                launch_own(0)
                torch.cuda.synchronize()
            for nm in [c for c in args.own_configs.split(",") if c]:
                c = names.index(nm)
                wsc = L.mbs_gemm_a4w4_config_workspace_bytes(c, 1, M, N, K)
                wst = torch.empty(max(wsc, 1), dtype=torch.uint8, device=dev)
                for _ in range(args.eager):
                    st = L.mbs_gemm_a4w4_launch_config(
                        c, 1, P(A.data_ptr()), P(B.data_ptr()), P(As.data_ptr()), P(Bs.data_ptr()),
                        pf(Af), pf(Bf), P(out_own.data_ptr()), M, N, K, Mpad, snp, P(wst.data_ptr()),
                        wsc, P(torch.cuda.current_stream().cuda_stream))
                    assert st == 0, L.mbs_last_error()
                    torch.cuda.synchronize()
            print(json.dumps({"shape": [M, N, K], "eager": args.eager, "factors": factors,
                              "max_err_over_bound": round(ratio, 4)}), flush=True)
            del A, B, As, Bs, Bc, Bsc, out_ref, out_own, ws
            torch.cuda.empty_cache()
            continue

        def make_graph(launch):
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                for i in range(copies):
                    launch(i)
            gr.replay()
            torch.cuda.synchronize()
            return gr

        def block_time(gr):
            gr.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(args.replays):
                gr.replay()
            e1.record()
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) * 1e3 / (args.replays * copies)

        # Interleaved rounds, the order alternating, medians: the shader clock
        # follows the load (power management), so blocks timed back to back
        # in a fixed order would favour whichever kernel runs first.
        g_ref, g_own = make_graph(launch_ref), make_graph(launch_own)
        ts = {"ref": [], "own": []}
        for r in range(args.rounds):
            for k in (("ref", "own") if r % 2 == 0 else ("own", "ref")):
                ts[k].append(block_time(g_ref if k == "ref" else g_own))
        t_ref, t_own = statistics.median(ts["ref"]), statistics.median(ts["own"])
        del g_ref, g_own
        flops = 2.0 * M * N * K
        byts = M * K // 2 + N * K // 2 + (M + N) * K // 32 + 2 * M * N
        buf = ctypes.create_string_buffer(128)
        mbs_amd.clib().mbs_gemm_a4w4_plan_name(M, N, K, buf, 128)
        print(json.dumps({
            "shape": [M, N, K], "factors": factors, "cold": cold,
            "ref_us": round(t_ref, 2), "own_us": round(t_own, 2),
            "speedup": round(t_ref / t_own, 3),
            "ref_TFLOPS": round(flops / t_ref / 1e6, 1), "own_TFLOPS": round(flops / t_own / 1e6, 1),
            "ref_GBps": round(byts / t_ref / 1e3, 1), "own_GBps": round(byts / t_own / 1e3, 1),
            "max_err_over_bound": round(ratio, 4), "own_plan": buf.value.decode(),
        }), flush=True)
        del A, B, As, Bs, Bc, Bsc, out_ref, out_own, ws
        torch.cuda.empty_cache()


if __name__ == "__main__":
    main()
