"""bench.py -- MI355X throughput of r4dx's quantized-weight matrix-product path (BASELINE.json metric:
trellis GEMV effective HBM GB/s at M = 1 over one 27B-class layer's projections).

A step is one decode-time pass over config 1's ten projections at M = 1, KB = 4: for each, the input
transform (f16 x -> f16 A) and the trellis GEMV with its FWHT/svh epilogue (bf16 out). The weights
rotate over enough copies (> 1 GiB) that the 256 MB MALL cannot serve them, so every step reads its
compressed weights from HBM. Inputs are resident in HBM before the timed region.

value = compressed-weight bytes per step / step time. `roofline` is the GEMV kernel alone: its
algorithmic bytes (weights + A + svh + C) over its average launch duration, timed with HIP events on
the stream the kernel runs on. `cpu_baseline` is the CPU oracle (decode + fp64 linear) on a bounded
sample, timed on this host. Prints one JSON line.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
# Warm-up replays of every timed graph, right before its timed replay: a graph that starts after an idle gap (a capture,
# a pause between legs) runs its first replays below the steady clock (the M = 256 layer measured 577-580 TFLOP/s
# after one warm-up replay, 625 after 4 and 633 after 8 or 16, same box).
WARM_REPLAYS = 8


def _warm(g):
    for _ in range(WARM_REPLAYS):
        g.replay()


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=240)
    ap.add_argument("--kb", type=int, default=4)
    ap.add_argument("--m", type=int, default=1)
    ap.add_argument("--copies", type=int, default=0, help="weight copies (0: enough for > 1 GiB)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--kernel-only", action="store_true", help="only the GEMV launches (for rocprof)")
    ap.add_argument("--no-m256", action="store_true", help="skip the M = 256 prefill GEMM leg")
    ap.add_argument("--no-rows", action="store_true", help="skip the config-1 rows at M 2/4/8, KB 5 and the mix")
    ap.add_argument("--no-w4", action="store_true", help="skip the w4a16 LM-head leg")
    ap.add_argument("--no-i8", action="store_true", help="skip the int8 prefill GEMM legs")
    ap.add_argument("--no-vendor", action="store_true", help="skip the vendor-library GEMMs timed for context")
    ap.add_argument("--pmc-prefill", action="store_true",
                    help="counter pass for the prefill kernels: each config-2 M = 256 shape, then the config-4 "
                         "dense and trellis int8 GEMMs, launched twice each; prints the launch order, no JSON line")
    ap.add_argument("--pmc-dense-forms", action="store_true",
                    help="counter pass for the dense int8 launch forms: 5120 x 17408 row scales, three eager launches "
                         "at SKG 1, then three in stream-K; prints no JSON line")
    ap.add_argument("--pmc-w4", action="store_true",
                    help="counter pass for the w4a16 LM head: a 512 MiB copy (calibration), then per group (32, 64) "
                         "and M (1, 8) the GEMM and the fused argmax entry on two weight copies; prints the launch "
                         "order, no JSON line")
    ap.add_argument("--pmc", action="store_true",
                    help="counter pass for rocprofv3 --pmc: a 512 MiB copy (calibration) and two eager "
                         "passes of the GEMV launches; prints no JSON line")
    return ap.parse_args()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the "
              "multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    from r4dx_amd import api, workloads as WL

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.pmc_prefill:
        pmc_prefill(api, WL, args.kb)
        return
    if args.pmc_dense_forms:
        pmc_dense_forms(api, WL)
        return
    if args.pmc_w4:
        pmc_w4(api, WL)
        return
    KB, M = args.kb, args.m
    shapes = WL.LAYER_SHAPES
    layer_wbytes = sum(K * N * KB // 8 for _, K, N in shapes)
    copies = args.copies or max(2, int(np.ceil((1 << 30) / layer_wbytes)) + 1)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    # The engine's launches for one layer (src/model/linear.cpp ApplyLinear / SharedTrellisInput): the
    # projections that read the same activations share one input-transform launch (nout = 2 or 3 outputs,
    # kernels.h:110-128), and mlp.gate / mlp.up are the fused two-part linear mlp.gate_up
    # (src/model/container.cpp:312; part 1 = up, from n_split = 17408, reads its own transform).
    shape = {name: (K, N) for name, K, N in shapes}
    lin, groups = [], []
    for gi, (gname, members) in enumerate(WL.LAYER_GROUPS):
        K = shape[members[0][0]][0]
        x = torch.from_numpy(WL.activations_f16(M, K, 30 + gi, bf16_exact=True)).to(dev)
        g = dict(name=gname, x=x, suh=[], outs=[])
        for li, parts in enumerate(members):
            N = sum(shape[p][1] for p in parts)
            nw = K * N * KB // 32
            words = [torch.randint(-2**31, 2**31 - 1, (nw,), dtype=torch.int32, device=dev, generator=gen)
                     for _ in range(copies)]
            suh = [torch.from_numpy(WL.signs(K, 10 + 3 * gi + li + 7 * j)).to(dev) for j in range(len(parts))]
            a = [torch.empty((M, K), dtype=torch.float16, device=dev) for _ in parts]
            g["suh"] += suh
            g["outs"] += a
            svh = torch.from_numpy(WL.svh_scales(N, 20 + 3 * gi + li)).to(dev)
            skg = api.trellis_gemv_skg(K, N, KB)
            while (K // 128) % skg:     # whole 128-blocks per slice (the fused transform's rule)
                skg -= 1
            lin.append(dict(name="+".join(parts) if len(parts) > 1 else parts[0], K=K, N=N,
                            n_split=shape[parts[0]][1] if len(parts) > 1 else N, words=words, suh=suh, svh=svh,
                            x=x, a=a, skg=skg, ws=torch.empty(max(1, skg * M * N), dtype=torch.float32, device=dev),
                            tickets=api.TicketBuffer(N, dev).t,
                            out=torch.empty((M, N), dtype=torch.bfloat16, device=dev)))
        groups.append(g)
        g["lin"] = lin[len(lin) - len(members):]
    out_scale = float(np.float32(1.0 / np.sqrt(128.0)))

    # The same layer with the projections that share an input laid out as one linear (gdn qkv | z, attn q | k | v:
    # pair grids, svh and outputs concatenated along N), one r4dx_gemm_trellis_nt_m64_parts launch per input
    # group: 6 GEMV launches instead of 9, the same weights and the same columns.
    merged = []
    for g in groups:
        ms = g["lin"]
        if len(ms) == 1:
            merged.append(ms[0])
            continue
        K = ms[0]["K"]
        N = sum(L["N"] for L in ms)
        skg = api.trellis_gemv_skg(K, N, KB)
        merged.append(dict(name="|".join(L["name"] for L in ms), K=K, N=N, parts=[L["a"][0] for L in ms],
                           n0=[int(v) for v in np.cumsum([0] + [L["N"] for L in ms[:-1]])],
                           words=[torch.cat([L["words"][c] for L in ms]) for c in range(copies)],
                           svh=torch.cat([L["svh"] for L in ms]), skg=skg,
                           ws=torch.empty(max(1, skg * M * N), dtype=torch.float32, device=dev),
                           tickets=api.TicketBuffer(N, dev).t,
                           out=torch.empty((M, N), dtype=torch.bfloat16, device=dev)))

    # Launches go to the current stream (the capture stream while a graph is being captured). The step is the
    # engine's launches for the layer: 6 input transforms and 9 GEMVs; the fused entry (r4dx_trellis_gemv_xf:
    # each workgroup transforms its own slice of x; 9 launches) is timed beside it.
    def gemv(L, copy):
        api.trellis_gemm_m64(L["a"][0], L["words"][copy], L["svh"], L["K"], L["N"], KB, skg=L["skg"],
                             a1=L["a"][1] if len(L["a"]) > 1 else None, n_split=L["n_split"],
                             out=L["out"], ws=L["ws"], tickets=L["tickets"], out_scale=out_scale)

    def gemv_xf(L, copy):
        api.trellis_gemv_xf(L["x"], L["suh"][0], L["words"][copy], L["svh"], L["K"], L["N"], KB, skg=L["skg"],
                            suh1=L["suh"][1] if len(L["suh"]) > 1 else None, n_split=L["n_split"],
                            out=L["out"], ws=L["ws"], tickets=L["tickets"], out_scale=out_scale)

    def step(c, gemv_only=False):
        if not gemv_only:
            for g in groups:
                api.trellis_input(g["x"], g["suh"], 0, bf16=False, outs=g["outs"])
        for L in lin:
            gemv(L, c)

    def nparts(L):
        return len(L["parts"]) if "parts" in L else len(L["a"])

    def launch(L, c):
        if "parts" in L:
            api.trellis_gemm_m64_parts(L["parts"], L["n0"], L["words"][c], L["svh"], L["K"], L["N"], KB,
                                       skg=L["skg"], out=L["out"], ws=L["ws"], tickets=L["tickets"],
                                       out_scale=out_scale)
        else:
            gemv(L, c)

    def step_merged(c, gemv_only=False):
        if not gemv_only:
            for g in groups:
                api.trellis_input(g["x"], g["suh"], 0, bf16=False, outs=g["outs"])
        for L in merged:
            launch(L, c)

    def step_fused(c):
        for L in lin:
            gemv_xf(L, c)

    # One HIP graph per sweep over the weight copies: a step per copy (Python launch cost out of the
    # timed region; the kernels are what a C++ caller would launch back to back).
    for c in range(copies):   # eager once: A is valid, tickets settle
        step_fused(c)
        step(c)
        step_merged(c)
    torch.cuda.synchronize()
    if args.pmc:
        # calibration: a plain device copy of a known size (the counters' bytes per algorithmic byte)
        src = torch.empty(512 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        for _ in range(2):
            for c in range(copies):
                for L in merged:
                    launch(L, c)
        torch.cuda.synchronize()
        print(json.dumps({"pmc_pass": "done", "copy_bytes": 512 << 20, "launch_order": [
            [L["name"], L["K"], L["N"], nparts(L)] for L in merged]}), flush=True)
        return

    def capture(fn):
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                fn()
        torch.cuda.synchronize()
        return g

    g_step = capture(lambda: [step_merged(c, args.kernel_only) for c in range(copies)])
    reps = max(1, -(-args.steps // copies))
    steps = reps * copies
    # untimed warm-up sweeps right before the timed ones: after the captures the GPU has idled, and the first sweeps
    # after an idle gap run ~5 % slower (the default 240 steps, 40 sweeps, ~4 ms, reach the steady rate)
    for _ in range(max(1, -(-args.warmup // copies))):
        g_step.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(reps):
        g_step.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = e0.elapsed_time(e1) / steps
    # the same graph timed round by round (one round = one sweep over the weight copies): the median of 11 rounds,
    # reported beside the contract's K-step figure
    rounds = []
    for _ in range(11):
        r0, r1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        r0.record(stream)
        g_step.replay()
        r1.record(stream)
        torch.cuda.synchronize()
        rounds.append(r0.elapsed_time(r1) / copies)
    ms_round_med = sorted(rounds)[len(rounds) // 2]
    g_fused = capture(lambda: [step_fused(c) for c in range(copies)])
    _warm(g_fused)
    u0, u1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    u0.record(stream)
    g_fused.replay()
    u1.record(stream)
    torch.cuda.synchronize()
    ms_step_fused = u0.elapsed_time(u1) / copies
    # the same layer as 6 fused launches (r4dx_trellis_gemv_xf_parts: each group's transform inside its GEMV)
    fl, fcopies, _ = config1_layer(api, WL, M, lambda g: KB, gen)
    _, fused_parts = config1_steps(api, fl, fcopies, out_scale)
    ms_step_fparts = _graph_ms(lambda: [fused_parts(c) for c in range(fcopies)], max(1, reps), fcopies)
    del fl
    # the reference engine's launch pattern: one GEMV per projection (9 launches)
    g_proj = capture(lambda: [step(c) for c in range(copies)])
    _warm(g_proj)
    v0, v1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    v0.record(stream)
    for _ in range(reps):
        g_proj.replay()
    v1.record(stream)
    torch.cuda.synchronize()
    ms_step_proj = v0.elapsed_time(v1) / steps

    # The dominant kernel alone: per launch shape of the step, a graph of back-to-back launches over the
    # rotating copies; the per-projection launches beside it.
    R = 4
    gemv_ms, alg_bytes = 0.0, 0.0
    per_shape, per_proj = {}, {}
    mids, lids = {id(L) for L in merged}, {id(L) for L in lin}
    for L in merged + [L for L in lin if id(L) not in mids]:
        g = capture(lambda: [launch(L, c) for _ in range(R) for c in range(copies)])
        _warm(g)
        b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        b0.record(stream)
        g.replay()
        b1.record(stream)
        torch.cuda.synchronize()
        avg_ms = b0.elapsed_time(b1) / (R * copies)
        K, N = L["K"], L["N"]
        ab = K * N * KB / 8 + nparts(L) * M * K * 2 + M * N * 2 + 4 * N
        rec = {"us": round(avg_ms * 1e3, 2), "GBs": round(ab / (avg_ms * 1e-3) / 1e9, 1)}
        if id(L) in mids:
            gemv_ms += avg_ms
            alg_bytes += ab
            per_shape[L["name"]] = rec
        if id(L) in lids:
            per_proj[L["name"]] = rec
    achieved = alg_bytes / (gemv_ms * 1e-3) / 1e9

    # Each leg starts from an idle GPU (a short pause: the prefill legs run the chip at its power limit, and an
    # HBM-bound leg measured right after them read up to 15 % slower); the HBM-bound w4a16 leg runs first.
    def leg(skip, fn, *a):
        if skip:
            return None
        torch.cuda.synchronize()
        time.sleep(1.0)
        return fn(*a)
    rows = leg(args.no_rows, bench_config1_rows, api, WL)
    w4 = leg(args.no_w4, bench_w4a16, api, WL)
    m256 = leg(args.no_m256, bench_m256, api, WL, KB)
    i8 = leg(args.no_i8, bench_int8, api, WL)
    ti8 = leg(args.no_i8, bench_trellis_i8, api, WL, KB)
    try:   # context only: a vendor-library failure must not cost the bench line
        vendor = leg(args.no_vendor, bench_vendor, WL)
    except Exception as e:  # noqa: BLE001
        vendor = {"error": f"{type(e).__name__}: {e}"[:300]}

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(KB)
        cpu["other_legs"] = cpu_baselines_other(KB)

    value = layer_wbytes / (ms_step * 1e-3) / 1e9
    line = {
        "metric": "trellis GEMV effective HBM GB/s @M=1 (27B layer shapes, KB4)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (uniform random trellis words, +-1 Hadamard signs, log-normal svh, N(0,1) x)",
        "config": {"workload": f"config1: the 10 projections of one 27B-class layer, the projections that share an "
                               f"input laid out as one linear (gdn qkv|z, attn q|k|v, mlp gate|up: 6 GEMV launches, "
                               f"r4dx_gemm_trellis_nt_m64_parts / r4d_gemm_trellis_nt_m64), M={M}, KB={KB}, "
                               f"{copies} rotating weight copies ({copies * layer_wbytes / 2**30:.2f} GiB)",
                   "M": M, "KB": KB, "weight_bytes_per_step": layer_wbytes,
                   "step": "6 input transforms (shared by projections with the same input, nout 1-3) + 6 trellis "
                           "GEMV launches (FWHT/svh epilogue, bf16 out); every weight byte of the layer read once",
                   "timing": f"HIP-graph replays (one sweep over the weight copies each), {args.warmup} untimed warm-up "
                             f"steps right before the {steps} timed ones; every other timed graph after "
                             f"{WARM_REPLAYS} warm-up replays",
                   "median_of_11_rounds_ms_per_step": round(ms_round_med, 4),
                   "median_of_11_rounds_GBs": round(layer_wbytes / (ms_round_med * 1e-3) / 1e9, 1),
                   "per_projection_ms_per_step": round(ms_step_proj, 4),
                   "per_projection_GBs": round(layer_wbytes / (ms_step_proj * 1e-3) / 1e9, 1),
                   "per_projection_step": "the reference engine's launch pattern: 6 transforms + 9 GEMVs, one per "
                                          "projection (mlp gate+up fused)",
                   "per_projection_launch_GBs": per_proj,
                   "fused_xf_ms_per_step": round(ms_step_fused, 4),
                   "fused_xf_GBs": round(layer_wbytes / (ms_step_fused * 1e-3) / 1e9, 1),
                   "fused_xf_step": "9 r4dx_trellis_gemv_xf launches (transform inside the GEMV), per projection",
                   "fused_parts_ms_per_step": round(ms_step_fparts, 4),
                   "fused_parts_GBs": round(layer_wbytes / (ms_step_fparts * 1e-3) / 1e9, 1),
                   "fused_parts_step": "6 r4dx_trellis_gemv_xf_parts launches (each group's input transform inside "
                                       "its GEMV)",
                   "rows": rows},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": _traffic("tq_gemv_kernel", KB, M, [L["name"] for L in merged]),
                     "kernel": "tq_gemv_kernel", "avg_launch_us": round(gemv_ms * 1e3 / len(merged), 3),
                     "per_shape_GBs": per_shape},
        "cpu_baseline": cpu,
        "m256": m256,
        "w4a16": w4,
        "int8": i8,
        "trellis_int8": ti8,
        "vendor_gemm": vendor,
        "wall_s": round(wall, 3),
    }
    print(json.dumps(line), flush=True)


# The 4/5-bit mix of the config-1 rows: the GDN and attention projections at KB 5, the MLP at KB 4 (4.41 bits per
# weight over the layer's weights; the reference reports its 4.5 bpw mix beside K4, docs/trellis-kernel.md:1380-1388).
MIX_KB5 = ("gdn.in", "gdn.out", "attn.in", "attn.o")


def config1_layer(api, WL, M, kb_of, gen, min_bytes=1 << 30):
    """One layer of config 1 at M rows, group g's linears at KB kb_of(g): the 6 launch groups (the projections that
    share an input laid out as one linear), each with >= min_bytes of rotating weight copies over the layer.
    Returns (launch list, copies, weight bytes per step)."""
    import numpy as np
    import torch
    dev = torch.device("cuda:0")
    shape = {name: (K, N) for name, K, N in WL.LAYER_SHAPES}
    wbytes = 0
    specs = []
    for gi, (gname, members) in enumerate(WL.LAYER_GROUPS):
        KB = kb_of(gname)
        K = shape[members[0][0]][0]
        widths = [shape[p][1] for lin in members for p in lin]
        N = sum(widths)
        wbytes += K * N * KB // 8
        specs.append((gi, gname, KB, K, N, widths))
    copies = max(2, int(np.ceil(min_bytes / wbytes)) + 1)
    layer = []
    for gi, gname, KB, K, N, widths in specs:
        nw = K * N * KB // 32
        skg = api.trellis_gemv_skg(K, N, KB)
        while (K // 128) % skg:
            skg -= 1
        parts = len(widths)
        layer.append(dict(
            name=gname, K=K, N=N, KB=KB, skg=skg, n0=[int(v) for v in np.cumsum([0] + widths[:-1])],
            x=torch.from_numpy(WL.activations_f16(M, K, 30 + gi, bf16_exact=True)).to(dev),
            suh=[torch.from_numpy(WL.signs(K, 10 + 3 * gi + j)).to(dev) for j in range(parts)],
            a=[torch.empty((M, K), dtype=torch.float16, device=dev) for _ in range(parts)],
            words=[torch.randint(-2**31, 2**31 - 1, (nw,), dtype=torch.int32, device=dev, generator=gen)
                   for _ in range(copies)],
            svh=torch.from_numpy(WL.svh_scales(N, 20 + gi)).to(dev),
            ws=torch.empty(max(1, skg * M * N), dtype=torch.float32, device=dev),
            tickets=api.TicketBuffer(N, dev).t, out=torch.empty((M, N), dtype=torch.bfloat16, device=dev)))
    return layer, copies, wbytes


def config1_steps(api, layer, copies, out_scale):
    """(two-launch step, fused step) closures over weight copy c: the input transforms (nout = parts) then one
    r4dx_gemm_trellis_nt_m64_parts per group; or one r4dx_trellis_gemv_xf_parts per group (the transform inside)."""
    def two(c):
        for L in layer:
            api.trellis_input(L["x"], L["suh"], 0, bf16=False, outs=L["a"])
        for L in layer:
            api.trellis_gemm_m64_parts(L["a"], L["n0"], L["words"][c], L["svh"], L["K"], L["N"], L["KB"],
                                       skg=L["skg"], out=L["out"], ws=L["ws"], tickets=L["tickets"],
                                       out_scale=out_scale)

    def fused(c):
        for L in layer:
            api.trellis_gemv_xf_parts(L["x"], L["suh"], L["n0"], L["words"][c], L["svh"], L["K"], L["N"], L["KB"],
                                      skg=L["skg"], out=L["out"], ws=L["ws"], tickets=L["tickets"],
                                      out_scale=out_scale)
    return two, fused


def bench_config1_rows(api, WL, reps=4):
    """Config 1's other step rows: the layer at M = 2, 4, 8 (KB 4), at KB 5 (M = 1, 8) and at the 4/5 mix (M = 1, 8),
    each as the two-launch step (6 transforms + 6 parts launches) and as the fused step (6 r4dx_trellis_gemv_xf_parts
    launches), replayed from HIP graphs over > 1 GiB of rotating weight copies. GB/s = weight bytes per step / step
    time."""
    import numpy as np
    import torch
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(99)
    out_scale = float(np.float32(1.0 / np.sqrt(128.0)))
    rows = {}
    cases = [("KB4", 2), ("KB4", 4), ("KB4", 8), ("KB5", 1), ("KB5", 8), ("mix", 1), ("mix", 8)]
    for rate, M in cases:
        kb_of = (lambda g: 4) if rate == "KB4" else (lambda g: 5) if rate == "KB5" else (lambda g: 5 if g in MIX_KB5 else 4)
        layer, copies, wbytes = config1_layer(api, WL, M, kb_of, gen)
        two, fused = config1_steps(api, layer, copies, out_scale)
        rec = {"weight_bytes_per_step": wbytes, "copies": copies}
        for form, fn in (("two_launch", two), ("fused", fused)):
            ms = _graph_ms(lambda: [fn(c) for c in range(copies)], reps, copies)
            rec[form + "_us"] = round(ms * 1e3, 2)
            rec[form + "_GBs"] = round(wbytes / (ms * 1e-3) / 1e9, 1)
        rows[f"{rate}_M{M}"] = rec
        del layer
        torch.cuda.empty_cache()
    return {"workload": "config 1 layer, 6 launch groups; two_launch = transforms + parts GEMVs, fused = "
                        "r4dx_trellis_gemv_xf_parts; mix = GDN and attention at KB 5, MLP at KB 4", "rows": rows}


def pmc_w4(api, WL):
    """The w4a16 LM head at config 3 (N = 248 320, K = 5120) for the HBM-traffic passes: a 512 MiB device copy first
    (each counter's bytes per copied byte), then per group and M the fp32 GEMM and the fused argmax entry, each on
    two weight copies (715 / 795 MB each, beyond the 256 MB MALL), so every launch streams its weights."""
    import torch
    dev = torch.device("cuda:0")
    src = torch.empty(512 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    N, K = 248320, 5120
    order = []
    for g in (32, 64):
        copies = []
        for cidx in range(2):
            wq, wsz = WL.w4a16_packed(N, K, g, 100 + cidx)
            copies.append((torch.from_numpy(wq.view("int32")).to(dev), torch.from_numpy(wsz.view("int32")).to(dev)))
        for M in (1, 8):
            a = torch.from_numpy(WL.activations_f16(M, K, 5)).to(dev)
            out = torch.empty((M, N), dtype=torch.float32, device=dev)
            for wq_d, wsz_d in copies:
                api.w4a16_gemm(a, wq_d, wsz_d, K, N, g, out=out, f32=True)
                order.append(f"g{g}_M{M}_gemm")
            for wq_d, wsz_d in copies:
                api.w4a16_gemm_argmax(a, wq_d, wsz_d, K, N, g, out=out)
                order.append(f"g{g}_M{M}_fused")
            torch.cuda.synchronize()
        del copies
        torch.cuda.empty_cache()
    print(json.dumps({"pmc_pass": "done", "copy_bytes": 512 << 20, "launch_order": order}), flush=True)


def pmc_dense_forms(api, WL):
    """The dense int8 GEMM at 5120 x 17408 (row scales) in its two launch forms, three eager launches each on one
    weight copy: SKG 1 (136 workgroups), then stream-K (256)."""
    import torch
    dev = torch.device("cuda:0")
    K, N = 5120, 17408
    x, w8, sw = WL.int8_case(K, N, 3)
    w_d = api.i8_pack_w(torch.from_numpy(w8).to(dev))
    sw_d = torch.from_numpy(sw).to(dev)
    a8, sa = api.i8_quant(torch.from_numpy(x.view("int16")).to(dev), False)
    out = torch.empty((256, N), dtype=torch.float16, device=dev)
    for skg in (1, 0):
        work = api.I8Workspace(N, skg, dev)
        for _ in range(3):
            api.i8_dense_gemm(a8, sa, w_d, sw_d, K, N, scale_mode=0, skg=skg, out=out, work=work)
        torch.cuda.synchronize()
    print(json.dumps({"pmc_pass": "done", "launch_order": ["skg1"] * 3 + ["stream-K"] * 3}), flush=True)


def pmc_prefill(api, WL, KB):
    """Eager launches of the prefill kernels for a counter pass (MFMA busy cycles per dispatch): every config-2
    shape through r4d_gemm_trellis_nt_m256, then config 4 through the dense int8 GEMM (row scales) and the
    trellis int8 GEMM (coarse), each twice. Prints the launch order with the algorithmic ops per launch."""
    import numpy as np
    import torch
    dev = torch.device("cuda:0")
    order = []
    for i, (name, K, N) in enumerate(WL.LAYER_SHAPES):
        words = torch.randint(-2**31, 2**31 - 1, (K * N * KB // 32,), dtype=torch.int32, device=dev)
        a = torch.from_numpy(WL.activations_f16(256, K, 40 + i, outlier_frac=0.01)).to(dev)
        svh = torch.from_numpy(WL.svh_scales(N, 50 + i)).to(dev)
        for _ in range(2):
            api.trellis_gemm_m256(a, words, svh, K, N, KB, out_scale=0.08838834764831845)
        order.append(["tq_m256_kernel", name, K, N, 2 * 256 * K * N])
    # the merged gate | up launch of the 6-launch layer: 272 groups on 256 CUs, the balanced form
    K, N = 5120, 34816
    words = torch.randint(-2**31, 2**31 - 1, (K * N * KB // 32,), dtype=torch.int32, device=dev)
    a = torch.from_numpy(WL.activations_f16(256, K, 60, outlier_frac=0.01)).to(dev)
    svh = torch.from_numpy(WL.svh_scales(N, 61)).to(dev)
    for _ in range(2):
        api.trellis_gemm_m256(a, words, svh, K, N, KB, out_scale=0.08838834764831845)
    order.append(["tq_m256_kernel", "mlp.gate|mlp.up (balanced)", K, N, 2 * 256 * K * N])
    del words
    for K, N in ((5120, 17408), (17408, 5120)):
        x, w8, sw = WL.int8_case(K, N, 3)
        w_d, sw_d = api.i8_pack_w(torch.from_numpy(w8).to(dev)), torch.from_numpy(sw).to(dev)
        a8, sa = api.i8_quant(torch.from_numpy(x.view(np.uint16)).to(dev), False)
        for _ in range(2):
            api.i8_dense_gemm(a8, sa, w_d, sw_d, K, N, scale_mode=0)
        order.append(["ti8_gemm_kernel<4, 0, 1, true>", f"dense {K}x{N}", K, N, 2 * 256 * K * N])
        words = torch.randint(-2**31, 2**31 - 1, (K * N * KB // 32,), dtype=torch.int32, device=dev)
        swc = api.trellis_i8_table(words, K, N, KB, True)
        svh = torch.from_numpy(WL.svh_scales(N, 8)).to(dev)
        for _ in range(2):
            api.trellis_gemm_i8(a8, sa, words, swc, svh, K, N, KB, coarse=True, skg=1 if N > 8192 else 4)
        order.append(["ti8_gemm_kernel<4, 0, 0, false>", f"trellis coarse {K}x{N}", K, N, 2 * 256 * K * N])
        # the per-128 form: per (row, 128 k) activation scales, per (column, 128 k) weight scales
        a8b, sab = api.i8_quant(torch.from_numpy(x.view(np.uint16)).to(dev), True)
        swb = api.trellis_i8_table(words, K, N, KB, False)
        for _ in range(2):
            api.trellis_gemm_i8(a8b, sab, words, swb, svh, K, N, KB, coarse=False, skg=1 if N > 8192 else 4)
        order.append(["ti8_gemm_kernel<4, 2, 0, false>", f"trellis per-128 {K}x{N}", K, N, 2 * 256 * K * N])
    torch.cuda.synchronize()
    print(json.dumps({"pmc_prefill": "done", "launches_each": 2, "order": order}), flush=True)


def bench_m256(api, WL, KB, R=3):
    """the M = 256 prefill trellis GEMM over the ten projections, fp16 MFMA with fp32
    accumulate, bf16 out; TFLOP/s = 2 * 256 * K * N per launch over the launch's average duration
    (back-to-back launches over rotating weight copies in a HIP graph, HIP events on its stream)."""
    import numpy as np
    import torch
    dev = torch.device("cuda:0")
    M = 256
    per_shape, tot_flop, tot_ms = {}, 0.0, 0.0
    for i, (name, K, N) in enumerate(WL.LAYER_SHAPES):
        nw = K * N * KB // 32
        copies = max(2, int(np.ceil(1.0e9 / (nw * 4))))
        words = [torch.randint(-2**31, 2**31 - 1, (nw,), dtype=torch.int32, device=dev) for _ in range(copies)]
        a = torch.from_numpy(WL.activations_f16(M, K, 40 + i, outlier_frac=0.01)).to(dev)
        svh = torch.from_numpy(WL.svh_scales(N, 50 + i)).to(dev)
        skg = api.trellis_m256_skg(K, N, KB)
        ws = torch.empty(api.lib().r4d_gemm_trellis_nt_m256_ws_bytes(M, N, skg) // 4, dtype=torch.float32, device=dev)
        tk = api.TicketBuffer(N, dev).t
        out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

        def run():
            for c in range(copies):
                api.trellis_gemm_m256(a, words[c], svh, K, N, KB, skg=skg, out=out, ws=ws, tickets=tk,
                                      out_scale=0.08838834764831845)
        run()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                for _ in range(R):
                    run()
        torch.cuda.synchronize()
        _warm(g)
        st = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        g.replay()
        e1.record(st)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / (R * copies)
        flop = 2.0 * M * K * N
        per_shape[name] = {"us": round(ms * 1e3, 2), "TFLOPs": round(flop / (ms * 1e-3) / 1e12, 1), "skg": skg}
        tot_flop += flop
        tot_ms += ms
        del words
        torch.cuda.empty_cache()
    per_proj = tot_flop / (tot_ms * 1e-3) / 1e12

    # The layer as 6 launches: the projections that share an input as one linear (gdn qkv | z, attn q | k | v
    # through r4dx_gemm_trellis_nt_m256_parts; mlp gate | up through the two-part r4d_gemm_trellis_nt_m256).
    # kb_of(group name) gives each group's rate: KB 4 throughout for the headline, then the rows at KB 5 and at
    # config 1's 4/5 mix.
    shape = {name: (K, N) for name, K, N in WL.LAYER_SHAPES}

    def layer(kb_of, Mr=M):
        per_launch, tot_flop, tot_ms = {}, 0.0, 0.0
        for i, (gname, members) in enumerate(WL.LAYER_GROUPS):
            KBg = kb_of(gname)
            names = [p for m in members for p in m]
            K = shape[names[0]][0]
            widths = [shape[p][1] for p in names]
            N = sum(widths)
            n0 = [int(v) for v in np.cumsum([0] + widths[:-1])]
            nw = K * N * KBg // 32
            copies = max(2, int(np.ceil(1.0e9 / (nw * 4))))
            words = [torch.randint(-2**31, 2**31 - 1, (nw,), dtype=torch.int32, device=dev) for _ in range(copies)]
            a = [torch.from_numpy(WL.activations_f16(Mr, K, 60 + 4 * i + j, outlier_frac=0.01)).to(dev)
                 for j in range(len(names))]
            svh = torch.from_numpy(WL.svh_scales(N, 70 + i)).to(dev)
            skg = api.trellis_m256_skg(K, N, KBg)
            ws = torch.empty(api.lib().r4d_gemm_trellis_nt_m256_ws_bytes(Mr, N, skg) // 4, dtype=torch.float32,
                             device=dev)
            tk = api.TicketBuffer(N, dev).t
            out = torch.empty((Mr, N), dtype=torch.bfloat16, device=dev)

            def run():
                for c in range(copies):
                    if len(names) == 1:
                        api.trellis_gemm_m256(a[0], words[c], svh, K, N, KBg, skg=skg, out=out, ws=ws, tickets=tk,
                                              out_scale=0.08838834764831845)
                    else:
                        api.trellis_gemm_m256_parts(a, n0, words[c], svh, K, N, KBg, skg=skg, out=out, ws=ws,
                                                    tickets=tk, out_scale=0.08838834764831845)
            run()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                with torch.cuda.graph(g, stream=s):
                    for _ in range(R):
                        run()
            torch.cuda.synchronize()
            _warm(g)
            st = torch.cuda.current_stream()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(st)
            g.replay()
            e1.record(st)
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / (R * copies)
            flop = 2.0 * Mr * K * N
            per_launch["|".join(names)] = {"us": round(ms * 1e3, 2), "TFLOPs": round(flop / (ms * 1e-3) / 1e12, 1),
                                           "skg": skg, "KB": KBg}
            tot_flop += flop
            tot_ms += ms
            del words, g
            torch.cuda.empty_cache()
        return per_launch, tot_flop, tot_ms

    per_launch, tot_flop, tot_ms = layer(lambda g: KB)
    rows = {}
    if KB == 4:
        for rate, kb_of, mr in (("KB5", lambda g: 5, M), ("mix", lambda g: 5 if g in MIX_KB5 else 4, M),
                                ("M128", lambda g: 4, 128)):
            pl, fl, t = layer(kb_of, mr)
            rows[rate] = {"layer_us": round(t * 1e3, 1), "TFLOPs": round(fl / (t * 1e-3) / 1e12, 1),
                          "per_launch_us": {k: v["us"] for k, v in pl.items()}}
    achieved = tot_flop / (tot_ms * 1e-3) / 1e12
    return {"metric": "M=256 trellis GEMM TFLOP/s (27B layer shapes, KB4)", "value": round(achieved, 1),
            "unit": "TFLOP/s", "roofline": {"bound": "mfma", "achieved": round(achieved, 1),
                                            "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                            "frac": round(achieved / FP16_PEAK_TFLOPS, 4)},
            "kernel": "tq_m256_kernel",
            "workload": "config2: the layer's 10 projections as 6 launches (same-input projections as one linear)",
            "layer_us": round(tot_ms * 1e3, 1), "per_launch": per_launch,
            "per_projection_TFLOPs": round(per_proj, 1), "per_shape": per_shape,
            "rows": {"workload": "the same 6-launch layer at KB 5, at config 1's 4/5 mix (GDN and attention at "
                                 "KB 5, the MLP at KB 4), and at M = 128 (KB 4; the 128-row form)", "rows": rows}}


def bench_w4a16(api, WL, R=8):
    """the w4a16 LM head (N = 248 320, K = 5120) at groups 32 / 64 and M = 1 / 8, fp32
    logits + per-row argmax. GB/s = (N K / 2 + N K / g * 4) bytes over the GEMM's average launch time
    (back-to-back in a HIP graph over 2 weight copies, > the 256 MB MALL)."""
    import torch
    dev = torch.device("cuda:0")
    N, K = 248320, 5120
    res = {}
    # HBM bytes over algorithmic bytes per case, from the committed summary of the two rocprofv3 --pmc passes
    # (bench.py --pmc-w4, counters calibrated on a copy of known size); empty when absent
    try:
        with open(os.path.join(ROOT, "profiles", "w4a16_traffic_config3.json")) as f:
            traffic = json.load(f).get("per_case", {})
    except (OSError, ValueError):
        traffic = {}
    for g in (32, 64):
        copies = []
        for cidx in range(2):
            wq, wsz = WL.w4a16_packed(N, K, g, 100 + cidx)
            copies.append((torch.from_numpy(wq.view("int32")).to(dev), torch.from_numpy(wsz.view("int32")).to(dev)))
        for M in (1, 8):
            a = torch.from_numpy(WL.activations_f16(M, K, 5)).to(dev)
            out = torch.empty((M, N), dtype=torch.float32, device=dev)
            idx = torch.empty(M, dtype=torch.int32, device=dev)
            val = torch.empty(M, dtype=torch.float32, device=dev)

            def run(with_argmax):
                for wq_d, wsz_d in copies:
                    if with_argmax == "fused":
                        api.w4a16_gemm_argmax(a, wq_d, wsz_d, K, N, g, out=out, out_idx=idx, out_val=val)
                        continue
                    api.w4a16_gemm(a, wq_d, wsz_d, K, N, g, out=out, f32=True)
                    if with_argmax:
                        api.argmax_rows(out, idx, val)
            # the argmax alone (one launch over the logits the GEMM left), the GEMM, the GEMM with the argmax, and the
            # fused entry (r4d_gemm_w4a16_nt_m64_f32_argmax): four graphs, each replayed in three interleaved rounds
            # (the median per graph), so that clock drift between measurements does not land on one of them
            def run_am():
                for _ in copies:
                    api.argmax_rows(out, idx, val)
            graphs = {}
            for with_am in (None, False, True, "fused"):
                gr = torch.cuda.CUDAGraph()
                s = torch.cuda.Stream()
                s.wait_stream(torch.cuda.current_stream())
                fn = run_am if with_am is None else (lambda wa=with_am: run(wa))
                with torch.cuda.stream(s):
                    fn()   # eager once on the capture stream: the argmax allocates its scratch there
                    torch.cuda.synchronize()
                    with torch.cuda.graph(gr, stream=s):
                        for _ in range(R):
                            fn()
                torch.cuda.synchronize()
                _warm(gr)
                torch.cuda.synchronize()
                graphs[with_am] = gr
            samples = {k: [] for k in graphs}
            st = torch.cuda.current_stream()
            for _ in range(3):
                for k, gr in graphs.items():
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record(st)
                    gr.replay()
                    e1.record(st)
                    torch.cuda.synchronize()
                    samples[k].append(e0.elapsed_time(e1) / (R * len(copies)))
            times = {k: sorted(v)[1] for k, v in samples.items()}
            nbytes = N * K / 2 + N * K / g * 4
            res[f"g{g}_M{M}"] = {"gemm_us": round(times[False] * 1e3, 2),
                                 "GBs": round(nbytes / (times[False] * 1e-3) / 1e9, 1),
                                 "frac": round(nbytes / (times[False] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                 "gemm_plus_argmax_us": round(times[True] * 1e3, 2),
                                 "argmax_alone_us": round(times[None] * 1e3, 2),
                                 "gemm_fused_argmax_us": round(times["fused"] * 1e3, 2),
                                 "traffic_over_alg": traffic.get(f"g{g}_M{M}_gemm", {}).get("traffic_over_alg")}
        del copies
        torch.cuda.empty_cache()
    return {"metric": "w4a16 LM head (N=248320, K=5120) effective HBM GB/s", "kernel": "w4_kernel",
            "peak_GBs": HBM_PEAK_GBS, "cases": res}


def bench_vendor(WL, R=4):
    """Context for the prefill legs, not a product path: the vendor library's plain GEMMs (hipBLASLt through
    torch.matmul, f16 weights, no decode; torch._int_mm, int8 weights) on the same launch shapes. f16: the config-2
    layer's 6 launches (same-input projections concatenated along N) at M = 256; int8: the two config-4 shapes.
    Best of the two weight layouts ([N][K] read transposed, [K][N]); rotating weight copies (> 1 GB per shape);
    back-to-back launches in a HIP graph (eager if the capture fails)."""
    import numpy as np
    import torch
    dev = torch.device("cuda:0")
    M = 256

    def timed(fn, n):
        try:
            fn()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                with torch.cuda.graph(g, stream=s):
                    for _ in range(R):
                        fn()
            torch.cuda.synchronize()
            _warm(g)
            run = g.replay
            reps = 1
        except RuntimeError:
            run, reps = fn, R
        torch.cuda.synchronize()
        st = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(reps):
            run()
        e1.record(st)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / (R * n)

    shape = {name: (K, N) for name, K, N in WL.LAYER_SHAPES}
    f16, tot_flop, tot_ms = {}, 0.0, 0.0
    for gname, members in WL.LAYER_GROUPS:
        names = [p for m in members for p in m]
        K, N = shape[names[0]][0], sum(shape[p][1] for p in names)
        a = torch.randn((M, K), dtype=torch.float16, device=dev)
        copies = max(2, int(np.ceil(1.0e9 / (K * N * 2))))
        best = None
        for layout in ("nk", "kn"):
            w = [torch.randn((N, K) if layout == "nk" else (K, N), dtype=torch.float16, device=dev)
                 for _ in range(copies)]
            ms = timed(lambda: [a @ (x.t() if layout == "nk" else x) for x in w], copies)
            best = ms if best is None else min(best, ms)
            del w
        torch.cuda.empty_cache()
        flop = 2.0 * M * K * N
        f16["|".join(names)] = {"us": round(best * 1e3, 2), "TFLOPs": round(flop / (best * 1e-3) / 1e12, 1)}
        tot_flop += flop
        tot_ms += best
    i8 = {}
    for K, N in ((5120, 17408), (17408, 5120)):
        a = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev)
        copies = max(2, int(np.ceil(1.0e9 / (K * N))))
        best = None
        for layout in ("nk", "kn"):
            w = [torch.randint(-127, 128, (N, K) if layout == "nk" else (K, N), dtype=torch.int8, device=dev)
                 for _ in range(copies)]
            ms = timed(lambda: [torch._int_mm(a, x.t() if layout == "nk" else x) for x in w], copies)
            best = ms if best is None else min(best, ms)
            del w
        torch.cuda.empty_cache()
        i8[f"K{K}_N{N}"] = {"us": round(best * 1e3, 2), "TOPs": round(2.0 * M * K * N / (best * 1e-3) / 1e12, 1)}
    return {"what": "vendor library plain GEMMs on the same shapes (context, no decode): torch.matmul f16 "
                    "(hipBLASLt) and torch._int_mm int8",
            "f16_layer_us": round(tot_ms * 1e3, 1), "f16_layer_TFLOPs": round(tot_flop / (tot_ms * 1e-3) / 1e12, 1),
            "f16_per_launch": f16, "int8": i8}


def _traffic(kernel, KB, M, names):
    """HBM bytes per launch of `kernel` (mean over the step's launch shapes `names`), from the committed summary
    of the two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE), each scaled by the same counter's reading for a
    copy of known size; None when no summary matches this configuration."""
    path = os.path.join(ROOT, "profiles", "gemv_traffic_config1.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("kernel") != kernel or t.get("KB") != KB or t.get("M") != M or set(t.get("per_shape", {})) != set(names):
        return None
    return t.get("hbm_bytes_per_launch")


def _graph_ms(fn, R, per):
    """Average ms of one of `per` launches inside fn, replayed R times in a HIP graph (events on the
    graph's launch stream)."""
    import torch
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for _ in range(R):
                fn()
    torch.cuda.synchronize()
    _warm(g)
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    g.replay()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (R * per)


def bench_int8(api, WL, R=4):
    """the int8 x int8 prefill GEMM at M = 256, (K, N) = (5120, 17408) and (17408, 5120),
    int8 weights (W8 block layout) with an fp32 scale per column, activations quantized per row (scale mode 0)
    or per (row, 128) (mode 1). TOP/s = 2 M K N over the GEMM's average launch time (12 weight copies back to
    back in a HIP graph); the roofline floor is the larger of the int8 MFMA time (5.0 POP/s) and the HBM time of
    the algorithmic bytes (N K weight bytes + M K + 2 M N + 4 N + the activation scales); the activation
    quantizer is timed beside it."""
    import torch
    dev = torch.device("cuda:0")
    M = 256
    res = {}
    for K, N in ((5120, 17408), (17408, 5120)):
        x, w8, sw = WL.int8_case(K, N, 3)
        copies = 12
        w_d = api.i8_pack_w(torch.from_numpy(w8).to(dev))
        ws_ = [w_d] + [w_d.clone() for _ in range(copies - 1)]
        sw_d = torch.from_numpy(sw).to(dev)
        x_d = torch.from_numpy(x.view("int16")).to(dev)
        for mode in (0, 1):
            skg = api.i8_dense_skg(K, N, mode)
            a8, sa = api.i8_quant(x_d, mode != 0)
            out = torch.empty((M, N), dtype=torch.float16, device=dev)
            work = api.I8Workspace(N, skg, dev)

            def gemm():
                for w in ws_:
                    api.i8_dense_gemm(a8, sa, w, sw_d, K, N, scale_mode=mode, skg=skg, out=out, work=work)
            ms = _graph_ms(gemm, R, copies)
            qms = _graph_ms(lambda: [api.i8_quant(x_d, mode != 0) for _ in range(4)], R, 4)
            ops = 2.0 * M * K * N
            nbytes = N * K + M * K + 2 * M * N + 4 * N + 4 * sa.numel()
            floor_ms = max(ops / 5.0e15, nbytes / (HBM_PEAK_GBS * 1e9)) * 1e3
            res[f"K{K}_N{N}_{'blk' if mode else 'row'}"] = {
                "gemm_us": round(ms * 1e3, 2), "TOPs": round(ops / (ms * 1e-3) / 1e12, 1),
                "GBs": round(nbytes / (ms * 1e-3) / 1e9, 1), "roofline_frac": round(floor_ms / ms, 4),
                "quant_us": round(qms * 1e3, 2), "skg": skg}
        del ws_, w_d
        torch.cuda.empty_cache()
    return {"metric": "int8 x int8 prefill GEMM TOP/s (M=256)", "kernel": "i8_gemm_kernel",
            "peak_TOPs": 5000.0, "peak_GBs": HBM_PEAK_GBS, "cases": res}


def bench_trellis_i8(api, WL, KB, R=4):
    """The int8 x int8 TRELLIS prefill GEMM (r4d_gemm_trellis_nt_i8 per-128 scales, _i8c coarse) at the MLP shapes
    of BASELINE config 4, weights as trellis words (decoded and quantized in the kernel). TOP/s = 2 M K N per
    launch (back to back over rotating word copies in a HIP graph)."""
    import numpy as np
    import torch
    dev = torch.device("cuda:0")
    M = 256
    res = {}
    for K, N in ((5120, 17408), (17408, 5120)):
        nw = K * N * KB // 32
        copies = max(2, int(np.ceil(1.0e9 / (nw * 4))))
        words = [torch.randint(-2**31, 2**31 - 1, (nw,), dtype=torch.int32, device=dev) for _ in range(copies)]
        x = torch.from_numpy(WL.activations_f16(M, K, 7, outlier_frac=0.01).view("int16")).to(dev)
        svh = torch.from_numpy(WL.svh_scales(N, 8)).to(dev)
        out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        skg = 1 if N > 8192 else 4
        ws = torch.empty(api.lib().r4d_gemm_trellis_nt_m256_ws_bytes(M, N, skg) // 4, dtype=torch.float32, device=dev)
        xb = torch.from_numpy(WL.activations_f16(M, K, 7, outlier_frac=0.01).astype("float32")).to(dev) \
            .to(torch.bfloat16).view(torch.int16)
        suh = torch.from_numpy(WL.signs(K, 9)).to(dev)
        for coarse in (False, True):
            a8, sa = api.i8_quant(x, blk=not coarse, ref_layout=True)
            # the fused input transform + quantizer that feeds this GEMM (bf16 x -> a8, sa)
            in_ms = _graph_ms(lambda: api.trellis_input_i8(xb, [suh], 0, coarse, outs=[(a8, sa)]), 8, 1)
            sws = [api.trellis_i8_table(w, K, N, KB, coarse) for w in words]

            def gemm():
                for w, sw in zip(words, sws):
                    api.trellis_gemm_i8(a8, sa, w, sw, svh, K, N, KB, coarse=coarse, skg=skg, out=out, ws=ws,
                                        out_scale=0.08838834764831845)
            ms = _graph_ms(gemm, R, copies)
            ops = 2.0 * M * K * N
            res[f"K{K}_N{N}_{'coarse' if coarse else 'per128'}"] = {
                "gemm_us": round(ms * 1e3, 2), "TOPs": round(ops / (ms * 1e-3) / 1e12, 1),
                "frac_int8_peak": round(ops / (ms * 1e-3) / 5.0e15, 4), "skg": skg,
                "input_i8_us": round(in_ms * 1e3, 2)}
        del words
        torch.cuda.empty_cache()
    return {"metric": "int8 x int8 trellis prefill GEMM TOP/s (M=256, KB4)", "kernel": "ti8_gemm_kernel",
            "peak_TOPs": 5000.0, "cases": res}


def cpu_baseline(KB):
    """The reference's own CPU path for config 0 (K = N = 5120, M = 1): input transform, pair-grid decode, fp64 linear
    (trellis_ref.hpp compiled into oracle/_ref, single-threaded as written), beside the oracle's port of the same work
    on all host cores; each the median of at least 5 runs. x is the GPU leg's kind of input: f16 ~N(0,1) with values
    exact in bf16, because the reference's CPU TransformInput reads bf16 x (trellis_ref.hpp:150) -- both forms then
    read the same numbers."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    from r4dx_amd import workloads as WL
    K = N = 5120
    words, suh, svh = WL.trellis_linear(K, N, KB, 1)
    x = WL.activations_f16(1, K, 2, bf16_exact=True).view(np.uint16)
    lib = O.lib()
    cores = lib.r4o_max_threads()

    def med(fn, budget_s, nmax):
        ts = []
        t_all = time.perf_counter()
        while len(ts) < 5 or (time.perf_counter() - t_all < budget_s and len(ts) < nmax):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts)), len(ts)

    def port_run():
        a = O.transform_input(x, False, suh, 0)
        q = O.decode_pair_grid(words, K, N, KB, 0)
        O.linear_from_a(a, q, svh, 0, nthreads=0)
    dt, n = med(port_run, 5.0, 20)
    port = {"value": round(K * N * KB / 8 / dt / 1e9, 4), "unit": "GB/s", "cores": cores,
            "kind": "port", "sample": f"config0 K=N=5120 KB={KB} M=1 (f16 x, values exact in bf16): transform + "
                                      f"decode + fp64 linear, median of {n} runs, {dt * 1e3:.1f} ms"}
    ref = O.ref()
    if ref is None:
        return port
    from oracle_lib import ptr
    xb = O.f32_to_bf16_bits(O.f16_bits_to_f32(x))
    assert np.array_equal(O.bf16_bits_to_f32(xb), O.f16_bits_to_f32(x)), "x must be exact in bf16"
    a = np.empty((1, K), np.uint16)
    q = np.empty((K, N), np.uint16)
    y = np.empty((1, N), np.float64)
    svh32 = np.ascontiguousarray(svh, np.float32)
    suh32 = np.ascontiguousarray(suh, np.float32)

    def ref_run():
        ref.ref_transform_input_bf16(ptr(xb), 1, K, ptr(suh32), 0, ptr(a))
        ref.ref_decode_pair_grid(ptr(words), K, N, KB, ptr(q))
        ref.ref_linear_from_a(ptr(a), None, N, 1, K, N, ptr(q), ptr(svh32), 0, ptr(y))
    dt, n = med(ref_run, 10.0, 10)
    return {"value": round(K * N * KB / 8 / dt / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "reference",
            "sample": f"config0 K=N=5120 KB={KB} M=1 (the same x as bf16): the reference's trellis_ref.hpp transform + "
                      f"pair-grid decode + fp64 linear, single-threaded as written, median of {n} runs, "
                      f"{dt * 1e3:.1f} ms", "port_all_cores": port}


def cpu_baselines_other(KB):
    """CPU rows beside the other legs, each on a bounded sample of its workload, median of 5 runs: decode alone and
    decode + matmul for the trellis linear (config 0) and the M = 256 GEMM (config 2, a 1024-column sample), the int8
    GEMM (config 4, a 256-column sample) and the w4a16 LM head (config 3, an 8192-row sample at g = 64, dequant alone
    and dequant + matmul). The oracle's C restatement on all host cores ("port"); where oracle/_ref is built, the
    reference's own single-threaded code ("reference": trellis_ref.hpp decode, int8_gemm_proto_ref.h RefGemmInt8)."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    from oracle_lib import ptr
    from r4dx_amd import workloads as WL
    lib, ref = O.lib(), O.ref()
    cores = lib.r4o_max_threads()

    def med(fn, n=5):
        ts = []
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))

    rows = {"cores_port": cores, "cores_reference": 1}
    # config 0 / 2: decode alone, and decode + matmul at M = 1 (config 0) and M = 256 (a 1024-column sample)
    K = N = 5120
    words, suh, svh = WL.trellis_linear(K, N, KB, 1)
    wbytes = K * N * KB / 8
    t = med(lambda: O.decode_pair_grid(words, K, N, KB, 0))
    rows["trellis_decode_only"] = {"value": round(wbytes / t / 1e9, 4), "unit": "GB/s", "kind": "port", "cores": cores,
                                   "sample": f"config0 K=N=5120 KB={KB}: pair-grid decode to f16, {t * 1e3:.1f} ms"}
    if ref is not None:
        q = np.empty((K, N), np.uint16)
        t = med(lambda: ref.ref_decode_pair_grid(ptr(words), K, N, KB, ptr(q)), 3)
        rows["trellis_decode_only_reference"] = {
            "value": round(wbytes / t / 1e9, 4), "unit": "GB/s", "kind": "reference", "cores": 1,
            "sample": f"config0 K=N=5120 KB={KB}: trellis_ref.hpp DecodePairGrid, {t * 1e3:.1f} ms"}
    Ns = 1024
    w_s, _, _ = WL.trellis_linear(K, Ns, KB, 3)
    a = WL.activations_f16(256, K, 4, outlier_frac=0.01).view(np.uint16)
    t_dec = med(lambda: O.decode_pair_grid(w_s, K, Ns, KB, 0))
    qs = O.decode_pair_grid(w_s, K, Ns, KB, 0)
    t_mm = med(lambda: O.raw_sums(a, qs, nthreads=0), 3)
    flop = 2.0 * 256 * K * Ns
    rows["m256_decode_plus_matmul"] = {
        "value": round(flop / (t_dec + t_mm) / 1e12, 5), "unit": "TFLOP/s", "kind": "port", "cores": cores,
        "sample": f"config2 M=256 K=5120, {Ns} of the columns, KB={KB}: decode {t_dec * 1e3:.1f} ms + fp64 matmul "
                  f"{t_mm * 1e3:.1f} ms"}
    # config 4: the int8 GEMM, row scales, a 256-column sample
    Ni = 256
    x, w8, sw = WL.int8_case(K, Ni, 3)
    sa = np.empty(256, np.float32)
    a8 = np.empty((256, K), np.int8)
    lib.r4o_i8_quant_act_row(ptr(np.ascontiguousarray(x.view(np.uint16))), 256, K, ptr(sa), ptr(a8))
    c = np.empty((256, Ni), np.float64)
    ops = 2.0 * 256 * K * Ni
    t = med(lambda: lib.r4o_i8_gemm_ref(ptr(a8), ptr(sa), ptr(w8), ptr(sw), 256, Ni, K, 3, ptr(c), 0))
    rows["int8_gemm"] = {"value": round(ops / t / 1e12, 5), "unit": "TOP/s", "kind": "port", "cores": cores,
                         "sample": f"config4 M=256 K=5120, {Ni} of the columns, row scales: {t * 1e3:.1f} ms"}
    if ref is not None:
        t = med(lambda: ref.ref_i8_gemm(ptr(a8), ptr(sa), ptr(w8), ptr(sw), 256, Ni, K, 3, ptr(c)), 3)
        rows["int8_gemm_reference"] = {"value": round(ops / t / 1e12, 5), "unit": "TOP/s", "kind": "reference",
                                       "cores": 1, "sample": f"the same sample through int8_gemm_proto_ref.h "
                                                             f"RefGemmInt8: {t * 1e3:.1f} ms"}
    # config 3: the w4a16 LM head at g = 64, M = 1, an 8192-row sample: dequant alone, dequant + fp64 matmul
    Nw, g = 8192, 64
    wq, wsz = WL.w4a16_packed(Nw, K, g, 100)
    xa = WL.activations_f16(1, K, 5).view(np.uint16)
    wf = np.empty((Nw, K), np.float32)
    y = np.empty((1, Nw), np.float64)
    wb = Nw * K / 2 + Nw * K / g * 4
    t = med(lambda: lib.r4o_w4_dequant(ptr(wq), ptr(wsz), Nw, K, g, ptr(wf)))
    rows["w4a16_dequant_only"] = {"value": round(wb / t / 1e9, 4), "unit": "GB/s", "kind": "port", "cores": 1,
                                  "sample": f"config3 K=5120 g=64, {Nw} of the vocab rows: dequant to fp32, "
                                            f"{t * 1e3:.1f} ms"}
    t = med(lambda: lib.r4o_w4_gemm_ref(ptr(xa), ptr(wq), ptr(wsz), 1, Nw, K, g, ptr(y), 0))
    rows["w4a16_dequant_plus_matmul"] = {"value": round(wb / t / 1e9, 4), "unit": "GB/s", "kind": "port",
                                         "cores": cores, "sample": f"the same sample, M=1: dequant + fp64 matmul, "
                                                                   f"{t * 1e3:.1f} ms"}
    return rows


if __name__ == "__main__":
    main()
