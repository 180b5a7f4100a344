#!/usr/bin/env python3
"""Bench driver for the MI355X Q4_K linear path (one GPU).

Headline (the metric BASELINE.json quotes, config 2 at M=1): the whole
q3_cuda_q4k_linear call (Q8_1 quantize + MMVQ) on the Qwen3-32B gate/up
projection, 5120 -> 25600, M=1, as algorithmic HBM GB/s:
    bytes/step = N*K*144/256 (Q4_K weights) + M*K*36/32 (Q8_1 read) + M*N*4 (Y write)
Weights are seeded N(0,0.02) fp32 quantized to Q4_K on the device; eight
copies (590 MB) are used round robin so that every step reads HBM, not the
256 MB last-level cache. Activations are N(0,1) with 1% of channels x20.

Also printed in the same JSON line:
  roofline      the MMVQ kernel alone: algorithmic bytes per launch over its
                average launch duration (back-to-back launches between one HIP
                event pair on the launch stream), against 8 TB/s; `traffic` is
                the HBM bytes per launch from the FETCH_SIZE / WRITE_SIZE
                counter summary in profiles/ when one is present for the same
                kernel, scaled by the copy-kernel calibration it records
  cpu_baseline  the reference's CPU path on this host: Q4_K dequant with the
                reference's q3_quant.c (oracle/_ref, single thread) plus
                numpy fp32 matmul, on the full gate/up matrix at M=1
  results       every BASELINE configuration, each with its kernel's fraction
                of the bound that limits it (HBM 8 TB/s or int8 MFMA 5.0 POPS):
                config 1 (q_proj 8192x5120, M=1), config 2 (MMVQ sweep M in
                {1,2,4,8} x {gate/up, down}), config 3 (all seven projections
                at M=512), config 4 (gate/up and down at M=2048, the LM head
                151936x5120 at M=16), config 5 (the 64-layer decode stream,
                449 calls per token, plain, graph-replayed and fused); plus
                9-16 token MMQ-path cases, the selected-row LM head and Q6_K
                (GGUF type 14) through the same ABI on the 25600 -> 5120 down
                shape and the LM head
Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "sera.c_amd"))

HBM_PEAK_GBS = 8000.0
WARM_MS = 40.0   # GPU time of the timed launch repeated before each measurement
INT8_PEAK_TOPS = 5000.0


def mmvq_waves(M, K):
    """Waves per workgroup of the dot4 MMVQ kernel (dispatch_nw in q4k_mmvq.hip)."""
    groups = (K // 256 + 7) // 8
    if M == 1 and groups >= 8:
        return 8
    return 4 if groups >= 4 or (M == 1 and groups == 3) else groups
METRIC = "MMVQ HBM GB/s @M=1; MMQ int8 TOPS @M=512; % of MI355X roofline"
SHAPES = {  # name: (N, K) as (output features, input features)
    "q": (8192, 5120), "k": (1024, 5120), "v": (1024, 5120), "o": (5120, 8192),
    "gate": (25600, 5120), "up": (25600, 5120), "down": (5120, 25600),
    "lm_head": (151936, 5120),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def alg_bytes(M, N, K, block_bytes=144):
    return N * K * block_bytes // 256 + M * K * 36 // 32 + M * N * 4


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--copies", type=int, default=8)
    ap.add_argument("--full", action="store_true", help="accepted for compatibility: every config runs by default")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true",
                    help="headline only (gate/up M=1): for counter-collection runs")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MB",
                    help="only run a plain device copy of MB megabytes 20 times (counter scale)")
    ap.add_argument("--linear-case", default="", metavar="M,N,K",
                    help="only time q3_cuda_q4k_linear on one Q4_K shape over --copies weight copies, "
                         "--steps calls (for counter-collection runs and batch sweeps)")
    ap.add_argument("--no-tiled", action="store_true",
                    help="skip the tiled-layout A/B cases (kernel traces that group launches by kernel name)")
    ap.add_argument("--tiled", action="store_true",
                    help="with --linear-case: the weights in the tiled Q4_K layout (qtype 268)")
    ap.add_argument("--q6k", action="store_true",
                    help="with --linear-case: Q6_K weights (GGUF bytes, or with --split the split layout)")
    ap.add_argument("--split", action="store_true", help="with --q6k: the split Q6_K layout (qtype 270)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(the Q4_K linear path has no multi-GPU split here)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import q3q4

    if args.copy_calibration:
        n = args.copy_calibration * 1000 * 1000 // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copy calibration: 20 copies of {n * 4} bytes")
        return

    L = q3q4.load()
    dev = torch.device("cuda:0")
    lin = q3q4.Linear(device=0, max_tokens=2048, max_features=151936, max_k=25600)
    stream = torch.cuda.current_stream()
    sptr = ctypes.c_void_p(stream.cuda_stream)

    def quantized(N, K, seed):
        gen = torch.Generator(device=dev).manual_seed(seed)
        w = torch.randn((N, K), generator=gen, device=dev, dtype=torch.float32) * 0.02
        out = torch.empty((N, K // 256 * 144), dtype=torch.uint8, device=dev)
        q3q4.quantize_weights(w, out)
        del w
        return out

    def weight_set(N, K, seed, copies):
        ws = [quantized(N, K, seed + i) for i in range(copies)]
        arr = (ctypes.c_void_p * copies)(*[w.data_ptr() for w in ws])
        return ws, arr

    def activations(M, K, seed):
        rng = np.random.default_rng(seed)
        x = rng.standard_normal((M, K)).astype(np.float32)
        ch = np.random.default_rng(K).choice(K, int(np.ceil(0.01 * K)), replace=False)
        x[:, ch] *= 20.0
        return torch.from_numpy(x).to(dev)

    def warm_clocks(run):
        """run(iters) -> ms of `iters` back-to-back launches. Repeats the timed
        launch for WARM_MS of GPU time first: from idle the clocks take
        10-20 ms of load to rise (the Q6_K tile kernel at 512 tokens ran 380
        us in its first launches, 310 us after a second of load)."""
        spent, n = 0.0, 2
        while spent < WARM_MS:
            spent += run(n)
            n = min(2 * n, 1024)

    def bench_linear(geo, arr, n, x, y, warmup, iters, warm=True):
        ms = ctypes.c_double()

        def run(k, w=0):
            rc = L.sera_q4k_bench_linear(ctypes.byref(geo), arr, n, ctypes.c_void_p(x.data_ptr()),
                                         x.shape[0], ctypes.c_void_p(y.data_ptr()), sptr, w, k, ctypes.byref(ms))
            if rc != 0:
                raise RuntimeError(f"bench_linear rc={rc}")
            return ms.value
        if warm:
            warm_clocks(run)
        return run(iters, warmup) / iters

    def bench_kernel(path, arr, n, stage, y, partial, M, N, K, param, warmup, iters):
        avg, tot = ctypes.c_double(), ctypes.c_double()

        def run(k, w=0):
            rc = L.sera_q4k_bench_kernel(path, arr, n, ctypes.c_void_p(stage.data_ptr()),
                                         ctypes.c_void_p(y.data_ptr()),
                                         ctypes.c_void_p(partial.data_ptr() if partial is not None else 0),
                                         partial.numel() * partial.element_size() // 4 if partial is not None else 0,
                                         M, N, K, param, sptr, w, k, ctypes.byref(avg), ctypes.byref(tot))
            if rc != 0:
                raise RuntimeError(f"bench_kernel rc={rc}: {L.sera_q4k_last_error().decode()}")
            return tot.value
        warm_clocks(run)
        run(iters, warmup)
        return avg.value, tot.value / iters

    if args.linear_case:
        M, N, K = (int(v) for v in args.linear_case.split(","))
        if args.q6k:
            qt = q3q4.QTYPE_Q6K_SPLIT if args.split else q3q4.QTYPE_Q6_K
            ws = []
            for i in range(args.copies):
                gen = torch.Generator(device=dev).manual_seed(7 + i)
                w = torch.randint(0, 256, (N, K // 256, 210), generator=gen, device=dev, dtype=torch.uint8)
                d = (torch.rand((N, K // 256), generator=gen, device=dev) + 0.5) * 2e-5
                w[:, :, 208:210] = d.to(torch.float16).view(torch.uint8).view(N, K // 256, 2)
                if args.split:
                    sp = torch.empty(w.numel(), dtype=torch.uint8, device=dev)
                    q3q4.weight_to_device_layout(qt, N, K, w, sp)
                    w = sp
                ws.append(w.view(-1))
            arr = (ctypes.c_void_p * len(ws))(*[w.data_ptr() for w in ws])
            launches = L.sera_q6k_kernel_launches_qt(qt, M, N, K)
        else:
            ws, arr = weight_set(N, K, 7, args.copies)
            qt = q3q4.QTYPE_Q4K_TILED if args.tiled else q3q4.QTYPE_Q4_K
            launches = L.sera_q4k_kernel_launches(M, N, K)
        if args.tiled and not args.q6k:
            tw = []
            for w in ws:
                t = torch.empty(w.numel(), dtype=torch.uint8, device=dev)
                q3q4.weight_to_device_layout(qt, N, K, w, t)
                tw.append(t)
            ws = tw
            arr = (ctypes.c_void_p * len(ws))(*[w.data_ptr() for w in ws])
        geo = q3q4.bind_geometry(qt, K, N)
        x = activations(M, K, 3)
        y = torch.empty((M, N), dtype=torch.float32, device=dev)
        # no clock warm-up: counter runs record every dispatch
        ms = bench_linear(geo, arr, args.copies, x, y, 2, args.steps, warm=False)
        log(f"[bench] linear case M={M} N={N} K={K} qtype {qt} "
            f"({L.q3_cuda_q4k_linear_path_for_batch(M).decode()}, "
            f"{launches} launches, {args.copies} weight copies): "
            f"{ms * 1e3:.2f} us per call over {args.steps} calls")
        return

    results = {}

    # ---------------- config 2: MMVQ decode sweep --------------------------
    log("[bench] building weights: gate/up and down, "
        f"{args.copies} copies each ({args.copies * 73.7 * 2:.0f} MB)")
    t0 = time.time()
    sets = {"gate_up": (25600, 5120, weight_set(25600, 5120, 0, args.copies)),
            "down": (5120, 25600, weight_set(5120, 25600, 100, args.copies))}
    torch.cuda.synchronize()
    log(f"[bench] weights ready in {time.time() - t0:.1f}s")

    sweep = []
    headline = None
    for name, (N, K, (ws, arr)) in sets.items():
        geo = q3q4.bind_geometry(q3q4.QTYPE_Q4_K, K, N)
        for M in ((1,) if args.quick else (1, 2, 4, 8)):
            if args.quick and name != "gate_up":
                break
            x = activations(M, K, 1 + M)
            y = torch.empty((M, N), dtype=torch.float32, device=dev)
            step_ms = bench_linear(geo, arr, args.copies, x, y, args.warmup, args.steps)
            stage = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device=dev)
            q3q4.quantize_row(x, stage)
            rpw = L.sera_q4k_mmvq_rows_per_tile(M, N, K)
            if L.sera_q4k_vec_uses_fewtok(M, N, K):
                # the MMVQ path's few-token MFMA kernel (MMVQ arithmetic): split
                # slots, then the zeroed row-group counters
                sp = q3q4.fewtok_splits(M, N, K)
                part = torch.zeros(sp * M * N + q3q4.fewtok_groups(M, N, K), dtype=torch.float32,
                                   device=dev)
                kavg, _ = bench_kernel(12, arr, args.copies, stage, y, part, M, N, K, 0,
                                       args.warmup, args.steps)
                rpw = None
            else:
                kavg, _ = bench_kernel(0, arr, args.copies, stage, y, None, M, N, K, 0,
                                       args.warmup, args.steps)
            b = alg_bytes(M, N, K)
            row = {"proj": name, "M": M, "N": N, "K": K,
                   "kernel": (f"sera_q4k_fewtok_kernel<{8 if N >= 16384 or K >= 16384 else 4}> "
                              f"(splits {q3q4.fewtok_splits(M, N, K)})") if rpw is None else
                             f"sera_q4k_mmvq_kernel<{M}, {rpw}, {mmvq_waves(M, K)}, false, false>",
                   "step_us": round(step_ms * 1e3, 3),
                   "step_GBps": round(b / (step_ms * 1e-3) / 1e9, 1),
                   "kernel_us": round(kavg * 1e3, 3),
                   "kernel_GBps": round(b / (kavg * 1e-3) / 1e9, 1),
                   "kernel_frac_hbm": round(b / (kavg * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
            log(f"[bench] mmvq {name} M={M}: step {row['step_us']} us ({row['step_GBps']} GB/s), "
                f"kernel {row['kernel_us']} us ({row['kernel_GBps']} GB/s, "
                f"{100 * row['kernel_frac_hbm']:.1f}% of HBM)")
            sweep.append(row)
            if name == "gate_up" and M == 1:
                headline = (row, step_ms, b)
    results["mmvq_sweep"] = sweep

    # ---------------- the achievable read rate: a plain streaming read ------
    # of the same weight copies (73,728,000 B each, walked round robin, no
    # compute, no output), the ceiling the MMVQ kernel is judged against
    ceiling = []
    sink = torch.zeros(256, dtype=torch.int32, device=dev)
    dummy = torch.zeros(16, dtype=torch.uint8, device=dev)
    for name, (N, K, (ws, arr)) in sets.items():
        wbytes = N * (K // 256) * 144
        for lpt in (1, 2, 4, 8, 16):
            kavg, _ = bench_kernel(14, arr, args.copies, dummy, sink, None, 1, N, K, lpt, args.warmup, args.steps)
            ceiling.append({"proj": name, "bytes": wbytes, "loads_per_thread": lpt,
                            "kernel": f"sera_stream_read_kernel<{lpt}>",
                            "workgroups": -(-wbytes // (16 * 256 * lpt)),
                            "us": round(kavg * 1e3, 3),
                            "GBps": round(wbytes / (kavg * 1e-3) / 1e9, 1)})
            log(f"[bench] plain read of {name} ({wbytes} B, {lpt} loads per thread): "
                f"{ceiling[-1]['us']} us, {ceiling[-1]['GBps']} GB/s")
    results["hbm_read_ceiling"] = ceiling
    read_best = {name: max((c for c in ceiling if c["proj"] == name), key=lambda c: c["GBps"])
                 for name in sets}
    for row in sweep:
        best = read_best[row["proj"]]
        row["frac_of_read_ceiling"] = round(row["kernel_GBps"] / best["GBps"], 4)

    # ---------------- config 1: q_proj 8192 x 5120 at M=1 ------------------
    if not args.quick:
        N, K = SHAPES["q"]
        ncopy = 16   # 377 MB, more than the 256 MB last-level cache
        qws, qarr = weight_set(N, K, 200, ncopy)
        geo = q3q4.bind_geometry(q3q4.QTYPE_Q4_K, K, N)
        x = activations(1, K, 11)
        y = torch.empty((1, N), dtype=torch.float32, device=dev)
        step_ms = bench_linear(geo, qarr, ncopy, x, y, args.warmup, args.steps)
        stage = torch.empty(q3q4.row_stage_layout(1, K)["total"], dtype=torch.uint8, device=dev)
        q3q4.quantize_row(x, stage)
        kavg, _ = bench_kernel(0, qarr, ncopy, stage, y, None, 1, N, K, 0, args.warmup, args.steps)
        b = alg_bytes(1, N, K)
        row = {"proj": "q", "M": 1, "N": N, "K": K,
               "kernel": (f"sera_q4k_mmvq_kernel<1, {L.sera_q4k_mmvq_rows_per_tile(1, N, K)}, "
                          f"{mmvq_waves(1, K)}, false, false>"),
               "step_us": round(step_ms * 1e3, 3), "step_GBps": round(b / (step_ms * 1e-3) / 1e9, 1),
               "kernel_us": round(kavg * 1e3, 3), "kernel_GBps": round(b / (kavg * 1e-3) / 1e9, 1),
               "kernel_frac_hbm": round(b / (kavg * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
               "weight_copies": ncopy}
        log(f"[bench] config 1 q_proj M=1: step {row['step_us']} us, kernel {row['kernel_us']} us "
            f"({100 * row['kernel_frac_hbm']:.1f}% of HBM)")
        results["config1_q_proj_m1"] = row
        del qws, qarr
        torch.cuda.empty_cache()

    # ---------------- config 3: MMQ M=512 (gate first, then the seven projections) -----
    def mmq_case(label, N, K, M, arr, ncopies, iters):
        x = activations(M, K, 7)
        y = torch.empty((M, N), dtype=torch.float32, device=dev)
        geo = q3q4.bind_geometry(q3q4.QTYPE_Q4_K, K, N)
        step_ms = bench_linear(geo, arr, ncopies, x, y, 3, iters)
        stage = torch.empty(q3q4.mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device=dev)
        q3q4.quantize_mmq(x, stage)
        wgs = L.sera_q4k_mmq_streamk_wgs(M)
        tiles = L.sera_q4k_mmq_tiles(M, N)
        if L.sera_q4k_mmq_uses_fewtok(M, N, K):
            # few-token kernel, MMQ formula: split slots, then the zeroed counters
            splits = -q3q4.fewtok_splits(M, N, K)
            partial = torch.zeros(-splits * M * N + q3q4.fewtok_groups(M, N, K), dtype=torch.float32,
                                  device=dev)
            kavg, _ = bench_kernel(13, arr, ncopies, stage, y, partial, M, N, K, 0, 3, iters)
        elif L.sera_q4k_mmq_schedule(M, N, K) == 2:
            # whole tiles + split tail: slots, then the zeroed tile counters
            dp, pieces = q3q4.mmq_tail_plan(M, N, K)
            splits = None
            nslot = q3q4.mmq_tail_slot_floats(M, N, dp, pieces)
            partial = torch.zeros(nslot + tiles, dtype=torch.float32, device=dev)
            kavg, _ = bench_kernel(15, arr, ncopies, stage, y, partial, M, N, K, dp * 64 + pieces, 3, iters)
        elif L.sera_q4k_mmq_schedule(M, N, K) == 1:
            # stream-K schedule: slots, then the zeroed tile counters
            splits = 0
            nslot = 2 * wgs * L.sera_q4k_mmq_slot_floats(M)
            partial = torch.zeros(nslot + tiles, dtype=torch.float32, device=dev)
            kavg, _ = bench_kernel(4, arr, ncopies, stage, y, partial, M, N, K, wgs, 3, iters)
        else:
            splits = q3q4.mmq_splits(M, N, K)
            partial = (torch.empty(splits * M * N, dtype=torch.float32, device=dev)
                       if splits > 1 else None)
            kavg, _ = bench_kernel(1, arr, ncopies, stage, y, partial, M, N, K, splits, 3, iters)
        ops = 2.0 * M * N * K
        row = {"case": label, "M": M, "N": N, "K": K,
               "schedule": (f"{dp} whole tiles of {tiles}, the rest in {pieces} K pieces" if splits is None
                            else "stream-K" if splits == 0 else f"split-K x{splits}" if splits > 0
                            else f"few-token kernel, {-splits} K split(s) summed in-kernel"),
               "step_us": round(step_ms * 1e3, 2), "kernel_us": round(kavg * 1e3, 2),
               "kernel_TOPS": round(ops / (kavg * 1e-3) / 1e12, 1),
               "step_TOPS": round(ops / (step_ms * 1e-3) / 1e12, 1),
               "kernel_frac_int8": round(ops / (kavg * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
               "kernel_GBps": round(alg_bytes(M, N, K) / (kavg * 1e-3) / 1e9, 1)}
        log(f"[bench] mmq {label} M={M} N={N} K={K}: kernel {row['kernel_us']} us, "
            f"{row['kernel_TOPS']} TOPS ({100 * row['kernel_frac_int8']:.1f}% of int8 peak)")
        return row

    gN, gK, (gws, garr) = sets["gate_up"]
    if not args.quick:
        results["mmq_m512_gate"] = mmq_case("gate", gN, gK, 512, garr, args.copies, 20)

    if not args.quick:
        results["selected_row_lm_head"] = lm_head_rows(torch, dev, bench_kernel)
        results["q6k"] = q6k_cases(torch, q3q4, L, dev, sptr, activations, bench_linear, bench_kernel,
                                        args)

    if not args.quick:
        full = []
        for name in ("q", "k", "v", "o", "gate", "up", "down"):
            N, K = SHAPES[name]
            if name == "gate":
                full.append(results["mmq_m512_gate"])
                continue
            ws, arr = (sets["down"][2] if name == "down" else weight_set(N, K, 300 + len(full), 2))
            full.append(mmq_case(name, N, K, 512, arr, len(ws), 20))
        results["config3_m512"] = full
        results["config4_m2048"] = [mmq_case("gate_up", gN, gK, 2048, garr, args.copies, 5),
                                    mmq_case("down", 5120, 25600, 2048, sets["down"][2][1],
                                             args.copies, 5)]
        # 9-16 tokens (a few speculative branches): the few-token kernel (MMQ
        # formula) at 9, the paired 16-token MMQ tile above
        results["mmq_few_tokens"] = [mmq_case("gate_up", gN, gK, 9, garr, args.copies, 20),
                                     mmq_case("gate_up", gN, gK, 12, garr, args.copies, 20),
                                     mmq_case("gate_up", gN, gK, 16, garr, args.copies, 20),
                                     mmq_case("down", 5120, 25600, 12, sets["down"][2][1], args.copies, 20),
                                     mmq_case("down", 5120, 25600, 16, sets["down"][2][1], args.copies, 20)]
        lmw, lmarr = weight_set(151936, 5120, 500, 1)
        lm = mmq_case("lm_head", 151936, 5120, 16, lmarr, 1, 20)
        # at 16 tokens the LM head is bound by its 437 MB of weights
        lm["kernel_frac_hbm"] = round(lm["kernel_GBps"] / HBM_PEAK_GBS, 4)
        results["config4_lm_head_m16"] = lm
        if not args.no_tiled:
            results["q4k_tiled_layout"] = tiled_cases(
                torch, q3q4, L, dev, activations, bench_linear, bench_kernel,
                {"gate_up": (gN, gK, gws), "down": (5120, 25600, sets["down"][2][0]), "lm_head": (151936, 5120, lmw)},
                args)
        del lmw
        results["config5_decode_stream"] = decode_stream(torch, q3q4, L, lin, quantized, activations, dev, sptr,
                                                            bench_kernel)

    # ---------------- roofline of the dominant kernel (MMVQ, M=1 gate/up) ---
    row, step_ms, b = headline
    kernel_ms = row["kernel_us"] * 1e-3
    achieved = b / (kernel_ms * 1e-3) / 1e9
    kname = row["kernel"]
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": hbm_traffic(kname),
                "kernel": kname,
                "avg_launch_us": row["kernel_us"], "algorithmic_bytes_per_launch": b,
                # the same kernel against the device's measured plain-read rate
                # of the same weight copies (results.hbm_read_ceiling)
                "read_ceiling_GBps": read_best["gate_up"]["GBps"],
                "frac_of_read_ceiling": row["frac_of_read_ceiling"]}

    # ---------------- CPU baseline ------------------------------------------
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(np, torch, gws[0], gN, gK, activations(1, gK, 2).cpu().numpy())

    value = b / (step_ms * 1e-3) / 1e9
    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(step_ms, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": (f"synthetic: seeded N(0,0.02) fp32 weights quantized to Q4_K on the GPU "
                 f"({args.copies} copies round robin, {args.copies * 73.728:.0f} MB > 256 MB MALL); "
                 "N(0,1) activations with 1% of channels x20"),
        "config": {"workload": "config 2 headline: q3_cuda_q4k_linear (Q8_1 quantize + MMVQ), "
                               "Qwen3-32B gate/up 5120->25600, M=1",
                   "N": gN, "K": gK, "M": 1, "bytes_per_step": b},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "results": results,
    }
    print(json.dumps(out), flush=True)


def tiled_cases(torch, q3q4, L, dev, activations, bench_linear, bench_kernel, mats, args):
    """The same Q4_K matrices in the 16-row tiled layout (qtype 268, made
    on the device from the GGUF copies): the whole q3_cuda_q4k_linear call
    and the kernel alone on the tiled copies, and the kernel alone on the
    GGUF copies measured right after for an A/B on the same box (the GGUF
    rule's own kernel choice is in mmvq_sweep and mmq_few_tokens). Decode
    batch sizes where the few-token kernel runs (2-16 tokens), M=1 (dot4
    MMVQ), the LM head at 4-16 tokens, and the whole call at 512 tokens
    (MMQ path) on both layouts."""
    T = q3q4.QTYPE_Q4K_TILED
    rows = []
    plan = {"gate_up": (1, 2, 4, 8, 16, 512), "down": (1, 4, 8, 16, 512), "lm_head": (4, 8, 16)}
    for name, (N, K, gbufs) in mats.items():
        tbufs = []
        for w in gbufs:
            t = torch.empty(w.numel(), dtype=torch.uint8, device=dev)
            q3q4.weight_to_device_layout(T, N, K, w, t)
            tbufs.append(t)
        torch.cuda.synchronize()
        n = len(gbufs)
        garr = (ctypes.c_void_p * n)(*[w.data_ptr() for w in gbufs])
        tarr = (ctypes.c_void_p * n)(*[w.data_ptr() for w in tbufs])
        geo = q3q4.bind_geometry(T, K, N)
        iters = 20 if name == "lm_head" else max(50, args.steps // 2)
        for M in plan[name]:
            x = activations(M, K, 60 + M)
            y = torch.empty((M, N), dtype=torch.float32, device=dev)
            if M > 16:
                # prefill: the whole call (quantize + MMQ schedule) on either layout
                gg = q3q4.bind_geometry(q3q4.QTYPE_Q4_K, K, N)
                ts, gs = [], []
                for _ in range(3):   # interleaved, median of three
                    ts.append(bench_linear(geo, tarr, n, x, y, 2, 10))
                    gs.append(bench_linear(gg, garr, n, x, y, 2, 10))
                st, sg = sorted(ts)[1], sorted(gs)[1]
                ops = 2.0 * M * N * K
                row = {"proj": name, "M": M, "N": N, "K": K, "kernel": "MMQ path (whole call)",
                       "step_us": round(st * 1e3, 2), "step_TOPS": round(ops / (st * 1e-3) / 1e12, 1),
                       "gguf_step_us": round(sg * 1e3, 2), "gguf_step_TOPS": round(ops / (sg * 1e-3) / 1e12, 1)}
                log(f"[bench] tiled {name} M={M}: step {row['step_us']} us ({row['step_TOPS']} TOPS); "
                    f"GGUF bytes {row['gguf_step_us']} us ({row['gguf_step_TOPS']} TOPS)")
                rows.append(row)
                continue
            step_ms = bench_linear(geo, tarr, n, x, y, 5, iters)
            if M <= 8:
                stage = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device=dev)
                q3q4.quantize_row(x, stage)
                path = 12 if L.sera_q4k_vec_uses_fewtok_qt(T, M, N, K) else 0
            else:
                stage = torch.empty(q3q4.mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device=dev)
                q3q4.quantize_mmq(x, stage)
                path = 13
                assert L.sera_q4k_mmq_uses_fewtok(M, N, K)
            part = None
            if path != 0:
                part = torch.zeros(q3q4.fewtok_splits(M, N, K) * M * N + q3q4.fewtok_groups(M, N, K),
                                   dtype=torch.float32, device=dev)
            kt, _ = bench_kernel(256 + path, tarr, n, stage, y, part, M, N, K, 0, 5, iters)
            kg, _ = bench_kernel(path, garr, n, stage, y, part, M, N, K, 0, 5, iters)
            b = alg_bytes(M, N, K)
            row = {"proj": name, "M": M, "N": N, "K": K,
                   "kernel": "dot4 MMVQ" if path == 0 else f"few-token (form {path - 12})",
                   "step_us": round(step_ms * 1e3, 2), "kernel_us": round(kt * 1e3, 2),
                   "kernel_frac_hbm": round(b / (kt * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                   "same_kernel_on_gguf_us": round(kg * 1e3, 2),
                   "same_kernel_on_gguf_frac_hbm": round(b / (kg * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
            log(f"[bench] tiled {name} M={M}: step {row['step_us']} us, {row['kernel']} {row['kernel_us']} us "
                f"({100 * row['kernel_frac_hbm']:.1f}% of HBM); the same kernel on GGUF bytes "
                f"{row['same_kernel_on_gguf_us']} us ({100 * row['same_kernel_on_gguf_frac_hbm']:.1f}%)")
            rows.append(row)
        del tbufs
        torch.cuda.empty_cache()
    return rows


def lm_head_rows(torch, dev, bench_kernel):
    """Selected-row LM head (sera_candidate_logits) on a Q6_K 151936 x 5120
    output.weight (random Q6_K bytes, fp16 d ~2e-5): 16 branches x 128
    candidates per call, fp32 hidden; bytes = candidate rows read."""
    N, K, branches, per = 151936, 5120, 16, 128
    gen = torch.Generator(device=dev).manual_seed(900)
    w = torch.randint(0, 256, (N, K // 256, 210), generator=gen, device=dev, dtype=torch.uint8)
    d = (torch.rand((N, K // 256), generator=gen, device=dev) + 0.5) * 2e-5
    w[:, :, 208:210] = d.to(torch.float16).view(torch.uint8).view(N, K // 256, 2)
    arr = (ctypes.c_void_p * 1)(w.data_ptr())
    hidden = torch.randn((branches, K), generator=gen, device=dev)
    ids = torch.randint(0, N, (branches * per,), generator=gen, device=dev, dtype=torch.int32)
    logits = torch.empty(branches * per, dtype=torch.float32, device=dev)
    kavg, _ = bench_kernel(7, arr, 1, hidden, logits, ids, branches, N, K, per, 10, 200)
    b = branches * per * (K // 256 * 210) + branches * K * 4 + branches * per * 4
    row = {"qtype": "Q6_K", "N": N, "K": K, "branches": branches, "candidates_per_branch": per,
           "kernel": "sera_candidate_logits_kernel<14>", "kernel_us": round(kavg * 1e3, 2),
           "rows_GBps": round(b / (kavg * 1e-3) / 1e9, 1)}
    log(f"[bench] selected-row LM head {branches}x{per} Q6_K rows: {row['kernel_us']} us "
        f"({row['rows_GBps']} GB/s of candidate rows)")
    del w
    return row


def q6k_cases(torch, q3q4, L, dev, sptr, activations, bench_linear, bench_kernel, args):
    """Q6_K weights (random ql/qh/scale bytes, fp16 d ~2e-5: the reference
    repo has no Q6_K quantizer) on the down shape 25600 -> 5120, 4 copies
    (430 MB) round robin, in both device layouts (GGUF bytes, qtype 14, and
    the split layout, qtype 270): the whole q3_cuda_q4k_linear call and the
    kernel alone (MMVQ kernel up to 4 tokens, the fp16-MFMA tile kernel from
    5). Then the full-vocabulary LM head (151936 x 5120) at one token on
    both layouts, 2 copies (1.28 GB)."""
    def q6k_copies(N, K, copies, seed):
        ws, ss = [], []
        for i in range(copies):
            gen = torch.Generator(device=dev).manual_seed(seed + i)
            w = torch.randint(0, 256, (N, K // 256, 210), generator=gen, device=dev, dtype=torch.uint8)
            d = (torch.rand((N, K // 256), generator=gen, device=dev) + 0.5) * 2e-5
            w[:, :, 208:210] = d.to(torch.float16).view(torch.uint8).view(N, K // 256, 2)
            sp = torch.empty(w.numel(), dtype=torch.uint8, device=dev)
            q3q4.weight_to_device_layout(q3q4.QTYPE_Q6K_SPLIT, N, K, w, sp)
            ws.append(w.view(N, -1))
            ss.append(sp)
        torch.cuda.synchronize()
        return ws, ss

    def row_of(layout, M, N, K, kname, step_ms, kavg):
        b = alg_bytes(M, N, K, 210)
        ops = 2.0 * M * N * K
        row = {"layout": layout, "M": M, "N": N, "K": K, "kernel": kname,
               "step_us": round(step_ms * 1e3, 2) if step_ms is not None else None,
               "kernel_us": round(kavg * 1e3, 2),
               "kernel_GBps": round(b / (kavg * 1e-3) / 1e9, 1),
               "kernel_frac_hbm": round(b / (kavg * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
               "kernel_TOPS": round(ops / (kavg * 1e-3) / 1e12, 1),
               "kernel_frac_int8": round(ops / (kavg * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4)}
        log(f"[bench] q6k {layout} N={N} K={K} M={M}: step {row['step_us']} us, kernel {row['kernel_us']} us "
            f"({row['kernel_GBps']} GB/s, {row['kernel_TOPS']} TOPS)")
        return row

    N, K, copies = 5120, 25600, 4
    ws, ss = q6k_copies(N, K, copies, 700)
    rows = []
    iters = max(20, args.steps // 5)
    for layout, qt, bufs in (("gguf", q3q4.QTYPE_Q6_K, ws), ("split", q3q4.QTYPE_Q6K_SPLIT, ss)):
        arr = (ctypes.c_void_p * copies)(*[w.data_ptr() for w in bufs])
        geo = q3q4.bind_geometry(qt, K, N)
        split = qt == q3q4.QTYPE_Q6K_SPLIT
        for M in (1, 2, 4, 8, 512):
            x = activations(M, K, 40 + M)
            y = torch.empty((M, N), dtype=torch.float32, device=dev)
            step_ms = bench_linear(geo, arr, copies, x, y, 5, iters if M < 512 else 10)
            if M >= 5:
                stage = torch.empty(q3q4.q6k_mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device=dev)
                (q3q4.quantize_row_q6k if M <= 8 else q3q4.quantize_mmq_d4)(x, stage)
                tt = L.sera_q6k_mmq_tile_tokens(M, N, K) // 32
                plan = q3q4.q6k_mmq_tail_plan(M, N, K)
                if plan:
                    # the tail schedule the dense paths run: slots, then the zeroed counters
                    dp, pc = plan
                    nslot = q3q4.q6k_mmq_tail_slot_floats(M, N, K, dp, pc)
                    part = torch.zeros(nslot + L.sera_q6k_mmq_tiles(M, N, K), dtype=torch.float32, device=dev)
                    kavg, _ = bench_kernel(17 if split else 16, arr, copies, stage, y, part, M, N, K, dp * 64 + pc,
                                           5, iters if M < 512 else 10)
                    sched = f"tail: {dp} whole tiles, the rest in {pc} K pieces"
                else:
                    sp = q3q4.q6k_mmq_splits(M, N, K)
                    part = torch.empty(sp * M * N, dtype=torch.float32, device=dev) if sp > 1 else None
                    kavg, _ = bench_kernel(10 if split else 6, arr, copies, stage, y, part, M, N, K, sp, 5,
                                           iters if M < 512 else 10)
                    sched = f"split-K x{sp}"
                row = row_of(layout, M, N, K, f"sera_q6k_mmq_kernel<{tt}, 2, {str(split).lower()}>", step_ms, kavg)
                row["schedule"] = sched
                rows.append(row)
                continue
            stage = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device=dev)
            q3q4.quantize_row(x, stage)
            if split:
                # the built-in 4 rows per workgroup (the step above), then 2 for comparison
                for r in (4, 2):
                    kavg, _ = bench_kernel(9, arr, copies, stage, y, None, M, N, K, r, 5, iters)
                    rows.append(row_of(layout, M, N, K, f"sera_q6s_mmvq_kernel<{M}, {r}, 4>",
                                       step_ms if r == 4 else None, kavg))
            else:
                rpw = L.sera_q6k_mmvq_rows_per_wave(M, N)
                kavg, _ = bench_kernel(5, arr, copies, stage, y, None, M, N, K, rpw, 5, iters)
                rows.append(row_of(layout, M, N, K, f"sera_q6k_mmvq_kernel<{M}, {rpw}>", step_ms, kavg))
    del ws, ss
    torch.cuda.empty_cache()

    N, K, copies = 151936, 5120, 2
    ws, ss = q6k_copies(N, K, copies, 800)
    x = activations(1, K, 41)
    y = torch.empty((1, N), dtype=torch.float32, device=dev)
    stage = torch.empty(q3q4.row_stage_layout(1, K)["total"], dtype=torch.uint8, device=dev)
    q3q4.quantize_row(x, stage)
    for layout, path, bufs, kname in (("gguf", 5, ws, "sera_q6k_mmvq_kernel<1, 4>"),
                                      ("split", 9, ss, "sera_q6s_mmvq_kernel<1, 4, 3>")):
        arr = (ctypes.c_void_p * copies)(*[w.data_ptr() for w in bufs])
        geo = q3q4.bind_geometry(q3q4.QTYPE_Q6_K if path == 5 else q3q4.QTYPE_Q6K_SPLIT, K, N)
        step_ms = bench_linear(geo, arr, copies, x, y, 3, 20)
        kavg, _ = bench_kernel(path, arr, copies, stage, y, None, 1, N, K, 0, 3, 20)
        rows.append(row_of(layout, 1, N, K, kname, step_ms, kavg))
    del ws, ss
    torch.cuda.empty_cache()
    return rows


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "mmvq_gate_up_m1_hbm_traffic.json")


def hbm_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed counter summary:
    FETCH_SIZE and WRITE_SIZE (KiB per dispatch) times the factors that make
    the same counters read a plain copy of known size correctly. None when
    the summary is absent or was taken on another kernel."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("kernel") != kernel:
        return None
    return int(round(1024 * (t["fetch_kib"] * t["fetch_factor"] + t["write_kib"] * t["write_factor"])))


def cpu_baseline(np, torch, w_dev, N, K, x):
    """Stage A: Q4_K dequant of the whole matrix (reference q3_quant.c when
    built into oracle/_ref, else this repo's C restatement), one thread.
    Stage B: numpy fp32 X @ W_deq^T on the BLAS threads. Repeated until
    ~10 s of CPU work."""
    from oracle import oracle
    W = w_dev.cpu().numpy()
    kind = "reference" if oracle.ref_lib() is not None else "port"
    deq = oracle.ref_dequant if kind == "reference" else oracle.dequant
    try:
        import threadpoolctl
        blas = max([i.get("num_threads", 1) for i in threadpoolctl.threadpool_info()] or [1])
    except Exception:  # noqa: BLE001
        blas = os.cpu_count() or 1
    ta = tb = 0.0
    reps = 0
    t_start = time.time()
    while reps < 20 and (reps < 2 or time.time() - t_start < 10.0):
        t0 = time.perf_counter()
        Wd = deq(W, N, K)
        t1 = time.perf_counter()
        y = x @ Wd.T
        t2 = time.perf_counter()
        ta += t1 - t0
        tb += t2 - t1
        reps += 1
        del Wd, y
    ta /= reps
    tb /= reps
    # The reference test's own CPU oracle (tests/test_q3_q4_linear.cu:236-277):
    # dequantize, then a double-accumulated dot per output, one thread.
    tl = []
    for _ in range(2):
        t0 = time.perf_counter()
        oracle.gemm_dequant(W, x, N, K)
        tl.append(time.perf_counter() - t0)
    tloop = min(tl)
    wbytes = N * K // 256 * 144
    # The other configurations the baseline plan names, on rows of the same
    # matrix (Q4_K rows are independent): config 1 (q_proj 8192 x K, M=1,
    # with the test loop) and config 3 (the gate projection at M=512; its
    # double loop would take minutes and is left out).
    configs = []
    rng = np.random.default_rng(3)
    for label, rows, M, loop in (("1: q_proj 8192x5120 M=1", 8192, 1, True),
                                 ("3: gate 25600x5120 M=512", N, 512, False)):
        Wc = np.ascontiguousarray(W.reshape(N, -1)[:rows])
        xc = x[:1] if M == 1 else rng.standard_normal((M, K)).astype(np.float32)
        da = db = float("inf")
        for _ in range(2):   # best of 2: the first pass also pays the page faults of a fresh array
            t0 = time.perf_counter()
            Wd = deq(Wc, rows, K)
            t1 = time.perf_counter()
            y = xc @ Wd.T
            t2 = time.perf_counter()
            del Wd, y
            da, db = min(da, t1 - t0), min(db, t2 - t1)
        wb = rows * K // 256 * 144
        row = {"config": label, "dequant_ms": round(da * 1e3, 2), "matmul_ms": round(db * 1e3, 2),
               "total_ms": round((da + db) * 1e3, 2), "GB/s": round(wb / (da + db) / 1e9, 3),
               "GOPS": round(2.0 * M * rows * K / (da + db) / 1e9, 2)}
        if loop:
            t0 = time.perf_counter()
            oracle.gemm_dequant(Wc, xc, rows, K)
            row["test_loop_ms"] = round((time.perf_counter() - t0) * 1e3, 2)
        configs.append(row)
    return {"value": round(wbytes / (ta + tb) / 1e9, 3), "unit": "GB/s", "cores": int(blas),
            "kind": kind,
            "sample": (f"full gate/up matrix {N}x{K} Q4_K ({wbytes} B) at M=1, {reps} reps: "
                       f"dequant {ta * 1e3:.1f} ms on 1 thread + numpy matmul {tb * 1e3:.1f} ms "
                       f"on {blas} BLAS threads; nproc={os.cpu_count()}"),
            "dequant_ms": round(ta * 1e3, 2), "matmul_ms": round(tb * 1e3, 2),
            "test_loop": {"ms": round(tloop * 1e3, 2), "GB/s": round(wbytes / tloop / 1e9, 3), "cores": 1,
                          "what": "the reference test's cpu_reference restated (row dequant + "
                                  "double-accumulated dot, 1 thread), best of 2"},
            "configs": configs}


def decode_stream(torch, q3q4, L, lin, quantized, activations, dev, sptr, bench_kernel):
    """Config 5: 64 layers x 7 projections at M=1 plus the LM head, all
    resident (~18 GB); one token = 449 q3_cuda_q4k_linear calls, issued from
    C (sera_q4k_bench_stream) so no host language sits in the loop."""
    order = ["q", "k", "v", "o", "gate", "up", "down"]
    keep = []
    geos = {n: q3q4.bind_geometry(q3q4.QTYPE_Q4_K, SHAPES[n][1], SHAPES[n][0]) for n in SHAPES}
    xs = {K: activations(1, K, K) for K in (5120, 8192, 25600)}
    ys = {n: torch.empty((1, SHAPES[n][0]), dtype=torch.float32, device=dev) for n in SHAPES}
    calls = []
    total_w = 0
    for layer in range(64):
        for name in order:
            N, K = SHAPES[name]
            w = quantized(N, K, 10_000 + layer * 7 + order.index(name))
            keep.append(w)
            calls.append((name, w))
            total_w += N * K // 256 * 144
    lm = quantized(151936, 5120, 99_999)
    keep.append(lm)
    calls.append(("lm_head", lm))
    total_w += 151936 * 5120 // 256 * 144
    n = len(calls)
    g_arr = (ctypes.c_void_p * n)(*[ctypes.addressof(geos[c[0]]) for c in calls])
    w_arr = (ctypes.c_void_p * n)(*[c[1].data_ptr() for c in calls])
    x_arr = (ctypes.c_void_p * n)(*[xs[SHAPES[c[0]][1]].data_ptr() for c in calls])
    m_arr = (ctypes.c_size_t * n)(*([1] * n))
    y_arr = (ctypes.c_void_p * n)(*[ys[c[0]].data_ptr() for c in calls])
    torch.cuda.synchronize()
    out = {"calls_per_token": n, "weight_bytes": total_w}
    side = torch.cuda.Stream()   # graph capture needs a stream other than the null stream
    for label, use_graph, strm in (("", 0, sptr), ("graph_", 1, ctypes.c_void_p(side.cuda_stream))):
        ms = ctypes.c_double()
        rc = L.sera_q4k_bench_stream(g_arr, w_arr, x_arr, m_arr, y_arr, n, strm, 10, 10, use_graph,
                                     ctypes.byref(ms))
        if rc != 0:
            raise RuntimeError(f"bench_stream rc={rc}: {L.sera_q4k_last_error().decode()}")
        torch.cuda.synchronize()
        t = ms.value
        out.update({f"{label}ms_per_token": round(t, 3),
                    f"{label}sustained_GBps": round(total_w / (t * 1e-3) / 1e9, 1),
                    f"{label}frac_hbm": round(total_w / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
    # the same weights through the fused linear group: per layer q/k/v with the
    # input RMSNorm in one quantize + one grouped MMVQ, o with the residual add
    # in its store, gate/up with the MLP RMSNorm likewise grouped, down with
    # SiLU*up in its quantize and the residual add in its store; then the
    # final-norm LM head: 8 launches per layer instead of 14 plus 3 elementwise
    hid = torch.randn((1, 5120), device=dev)
    attn = torch.randn((1, 8192), device=dev)
    gam = [torch.rand(5120, device=dev) + 0.5 for _ in range(3)]
    bufs = {n: torch.empty((1, SHAPES[n][0]), dtype=torch.float32, device=dev)
            for n in ("q", "k", "v", "gate", "up", "lm_head")}
    G = q3q4
    fcalls = []
    for layer in range(64):
        w = {name: keep[layer * 7 + order.index(name)] for name in order}
        fcalls.append(G.group_call([geos["q"], geos["k"], geos["v"]], [w["q"], w["k"], w["v"]],
                                   [bufs["q"], bufs["k"], bufs["v"]], hid, gamma=gam[0], eps=1e-6,
                                   flags=G.LIN_RMSNORM))
        fcalls.append(G.group_call([geos["o"]], [w["o"]], [hid], attn, flags=G.LIN_ACCUMULATE))
        fcalls.append(G.group_call([geos["gate"], geos["up"]], [w["gate"], w["up"]], [bufs["gate"], bufs["up"]],
                                   hid, gamma=gam[1], eps=1e-6, flags=G.LIN_RMSNORM))
        fcalls.append(G.group_call([geos["down"]], [w["down"]], [hid], bufs["gate"], x2=bufs["up"],
                                   flags=G.LIN_SILU_MUL | G.LIN_ACCUMULATE))
    fcalls.append(G.group_call([geos["lm_head"]], [lm], [bufs["lm_head"]], hid, gamma=gam[2], eps=1e-6,
                               flags=G.LIN_RMSNORM))
    carr = (G.GroupCall * len(fcalls))(*fcalls)
    for label, use_graph, strm in (("fused_", 0, sptr), ("fused_graph_", 1, ctypes.c_void_p(side.cuda_stream))):
        ms = ctypes.c_double()
        rc = L.sera_q4k_bench_group_stream(carr, len(fcalls), strm, 10, 10, use_graph, ctypes.byref(ms))
        if rc != 0:
            raise RuntimeError(f"bench_group_stream rc={rc}: {L.sera_q4k_last_error().decode()}")
        torch.cuda.synchronize()
        t = ms.value
        out.update({f"{label}ms_per_token": round(t, 3),
                    f"{label}sustained_GBps": round(total_w / (t * 1e-3) / 1e9, 1),
                    f"{label}frac_hbm": round(total_w / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
    # each projection's one-token MMVQ kernel over its 64 layer copies (streamed
    # from HBM, round robin), timed alone: where the layer's time goes
    per = {}
    for name in order:
        N, K = SHAPES[name]
        arr = (ctypes.c_void_p * 64)(*[keep[layer * 7 + order.index(name)].data_ptr() for layer in range(64)])
        stage = torch.empty(q3q4.row_stage_layout(1, K)["total"], dtype=torch.uint8, device=dev)
        q3q4.quantize_row(xs[K], stage)
        # best of three: k/v last 2.7 us, near the host's launch rate, and a
        # run now and then includes a submission gap
        kavg = min(bench_kernel(0, arr, 64, stage, ys[name], None, 1, N, K, 0, 10, 128)[0] for _ in range(3))
        wb = N * K // 256 * 144
        per[name] = {"kernel_us": round(kavg * 1e3, 2), "GBps": round(wb / (kavg * 1e-3) / 1e9, 1),
                     "frac_hbm": round(wb / (kavg * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    out["projection_kernels_m1"] = per
    log("[bench] config 5 one-token kernels: " +
        ", ".join(f"{n} {v['kernel_us']} us ({100 * v['frac_hbm']:.1f}%)" for n, v in per.items()))
    del keep, lm
    out["note"] = ("449 q3_cuda_q4k_linear calls (Q8_1 quantize + MMVQ each) per token, issued from C; "
                   "graph_*: the same pass captured once into a HIP graph and replayed; fused_*: the layer as "
                   "4 sera_linear_group calls (input/MLP RMSNorm, SiLU*up and both residual adds fused; q/k/v "
                   "and gate/up grouped) plus the final-norm LM head, 514 launches per token; 10 timed tokens "
                   "after 10 untimed")
    return out


if __name__ == "__main__":
    main()
