"""Benchmark: FP8 MoE grouped-GEMM TFLOP/s and % of dense-FP8 MFMA peak on 1 MI355X.

One step = one full MoE layer forward through the native path
(route -> scatter -> grouped GEMM1 + SiLU*up -> requant -> grouped GEMM2 ->
combine) on inputs already resident in HBM.  ``value`` = the layer's GEMM
FLOPs (2*rows*2I*H + 2*rows*H*I, rows = T*k) / measured step time, i.e. the
routing, permute, requant and combine kernels count against the number.

Default workload: the DeepSeek-V3-shape layer (T=8192, H=7168, I=2048, E=256,
top-8, Zipf-skewed routing, 128x128 weight / 1x128 activation block scales).
Synthetic inputs: token rows x and router logits come from numpy's PCG64
(``default_rng(seed)``) in the order the path's frozen generator draws them
(x, logits, the Zipf bias permutation), so the benched routing is the
specification's draw; expert weights are drawn on the GPU (torch generator,
N(0,1)).  Everything is quantised by the path's own device quantisers.

``--config dense2048|tp_local|mx8192`` runs one dense GEMM per step instead:
configs 1 and 4 (per-tensor scales, bf16 out) and the reference MXFP8
harness's 8192^3 shape with 1x32 e8m0 scales (fp32 out); ``value`` is then that
GEMM's TFLOP/s.

Timing: W warm-up calls, then ``settle`` (at least --settle-s seconds of
back-to-back layer calls, recorded), then the K timed steps (wall clock,
synchronised on both sides), then K more one-call layers with the library's
per-dispatch timing events (hkmoe_kernel_timing) in the same steady state.

Extra JSON fields: ``roofline`` (dominant kernel: the 256x256 grouped GEMM 1,
its average duration from the per-dispatch events), ``kernels_ms`` (average
duration of each kernel of the one-call layer) and ``kernel_timing`` (the
layer's mean timeline, its span, the main-stream chain of kernels and the gaps
between them), ``settle``, and ``cpu_baseline``: bench.py's own PyTorch CPU
port of the layer (route, dequantise to fp32, per-expert x_e . W_e^T, SiLU*up,
bf16, requantise, . W2_e^T, combine; kind "port", it does not use the oracle)
timed on the host's cores over a bounded, size-stratified sample of experts.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "distributed-hipkittens_amd"))

METRIC = "fp8 MoE grouped-GEMM TFLOP/s + % of FP8 MFMA peak on 1 MI355X"
PEAK_FP8_TFLOPS = 5000.0
PEAK_HBM_GBS = 8000.0

CONFIGS = {
    "dsv3": dict(T=8192, H=7168, I=2048, E=256, k=8, block=True, skew=True),
    "mixtral": dict(T=4096, H=4096, I=14336, E=8, k=2, block=False, skew=False),
    "decode": dict(T=64, H=4096, I=1536, E=128, k=8, block=True, skew=False),
    # config 3's shapes and routing with MX operands (1x32 e8m0 exponents applied
    # inside the MFMA) instead of fp32 block scales
    "dsv3_mx": dict(T=8192, H=7168, I=2048, E=256, k=8, block=False, skew=True, mx=True),
}
# Dense single-GEMM workloads: configs 1 and 4 (per-tensor scales, bf16 out) and
# the reference MXFP8 harness's shape (kernels/cdna4/gemm/mxfp8/MXFP8_4wave/
# 4_wave.cu:23, 386-388: M = N = K = 8192, N(0, 0.5), 1x32 e8m0, fp32 out).
DENSE = {
    "dense2048": dict(M=2048, N=2048, K=2048, mx=False, sigma=1.0, out="bf16"),
    "tp_local": dict(M=8192, N=8192, K=2048, mx=False, sigma=1.0, out="bf16"),
    "mx8192": dict(M=8192, N=8192, K=8192, mx=True, sigma=0.5, out="f32"),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--settle-s", type=float, default=1.0,
                    help="MoE workloads: seconds of back-to-back layer calls between the warm-up and the "
                         "timed steps (recorded as `settle`)")
    ap.add_argument("--config", default="dsv3", choices=sorted(CONFIGS) + sorted(DENSE))
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="unused (kept for older command lines): the CPU baseline samples a fixed size-stratified share of the experts")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "traffic.json"),
                    help="measured HBM bytes per launch (rocprofv3 --pmc summary)")
    ap.add_argument("--weights", default="packed", choices=["packed", "rows"],
                    help="expert weight layout: packed once at layer construction (default) or row-major")
    ap.add_argument("--graph", action="store_true",
                    help="MoE workloads: capture one layer call in a HIP graph and time its replays")
    ap.add_argument("--rotate-mb", type=int, default=512,
                    help="dense workloads: rotate over copies of A and B totalling at least this many MB "
                         "so that no launch finds its operands in L2/MALL (0: one copy)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run one 1 GiB device-to-device copy (counter calibration)")
    ap.add_argument("--other-configs", default="mixtral,decode,dense2048,tp_local",
                    help="default dsv3 run only: also measure these workloads (each in a child process, "
                         "10 steps, no CPU baseline) and attach their results as `other_configs`; "
                         "'' to skip")
    ap.add_argument("--summarize-counters", metavar="DIR", default=None,
                    help="no GPU work: turn the rocprofv3 --pmc output under DIR (mfma/, lds/) of this config "
                         "into profiles/*_counters.md")
    ap.add_argument("--summarize-profile", metavar="DIR", default=None,
                    help="no GPU work: turn the rocprofv3 output under DIR (trace/, FETCH_SIZE/, "
                         "WRITE_SIZE/) of this config into profiles/*.md and profiles/traffic.json")
    return ap.parse_args()


def host_draw(cfg, seed):
    """Token rows x [T, H] and router logits [T, E] (fp32, numpy PCG64), drawn
    in the order of the path's frozen synthetic generator: x, logits, then for
    skewed routing a permutation rank of 1..E and the Zipf(1.1) bias
    -1.1 * ln(rank) added to every token's logits."""
    import numpy as np
    rng = np.random.default_rng(seed)
    T, H, E = cfg["T"], cfg["H"], cfg["E"]
    x = rng.standard_normal((T, H), dtype=np.float32)
    logits = rng.standard_normal((T, E), dtype=np.float32)
    if cfg["skew"]:
        rank = rng.permutation(E).astype(np.float32) + np.float32(1.0)
        logits = (logits + (-np.float32(1.1) * np.log(rank)).astype(np.float32)[None, :]).astype(np.float32)
    return x, logits


def make_inputs(cfg, seed, dev):
    import torch
    import hkmoe
    T, H, I, E, k = cfg["T"], cfg["H"], cfg["I"], cfg["E"], cfg["k"]
    x_np, logits_np = host_draw(cfg, seed)
    x = torch.from_numpy(x_np).to(dev)
    logits = torch.from_numpy(logits_np).to(dev)
    del x_np, logits_np
    # expert weights: seeded on the device (an independent stream)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    F8 = torch.float8_e4m3fn
    if cfg.get("mx"):
        x_q, x_e = hkmoe.quant_mx(x)
        del x
        w13_q = torch.empty((E, 2 * I, H), dtype=F8, device=dev)
        w2_q = torch.empty((E, H, I), dtype=F8, device=dev)
        w13_e = torch.empty((E, 2 * I, H // 32), dtype=torch.uint8, device=dev)
        w2_e = torch.empty((E, H, I // 32), dtype=torch.uint8, device=dev)
        chunk = max(1, int(2e9 // (2 * I * H * 4)))
        for e0 in range(0, E, chunk):
            e1 = min(E, e0 + chunk)
            for wq, we, shape in ((w13_q, w13_e, (2 * I, H)), (w2_q, w2_e, (H, I))):
                w = torch.randn(((e1 - e0) * shape[0], shape[1]), generator=g, device=dev, dtype=torch.float32)
                q, s = hkmoe.quant_mx(w)
                wq[e0:e1].copy_(q.view(e1 - e0, *shape))
                we[e0:e1].copy_(s.view(e1 - e0, shape[0], shape[1] // 32))
                del w, q, s
        torch.cuda.synchronize()
        return dict(x_q=x_q, x_scale=x_e, logits=logits, w13_q=w13_q, w13_scale=w13_e, w2_q=w2_q,
                    w2_scale=w2_e, top_k=k)
    w13_q = torch.empty((E, 2 * I, H), dtype=F8, device=dev)
    w2_q = torch.empty((E, H, I), dtype=F8, device=dev)
    if cfg["block"]:
        x_q, x_s = hkmoe.quant_group(x)
        w13_s = torch.empty((E, 2 * I // 128, H // 128), dtype=torch.float32, device=dev)
        w2_s = torch.empty((E, H // 128, I // 128), dtype=torch.float32, device=dev)
    else:
        x_q, x_s = hkmoe.quant_tensor(x)
        w13_s = torch.empty(E, dtype=torch.float32, device=dev)
        w2_s = torch.empty(E, dtype=torch.float32, device=dev)
    del x
    chunk = max(1, int(2e9 // (2 * I * H * 4)))
    for e0 in range(0, E, chunk):
        e1 = min(E, e0 + chunk)
        for wq, ws, shape in ((w13_q, w13_s, (2 * I, H)), (w2_q, w2_s, (H, I))):
            w = torch.randn((e1 - e0, *shape), generator=g, device=dev, dtype=torch.float32)
            if cfg["block"]:
                q, s = hkmoe.quant_block(w)
                wq[e0:e1].copy_(q)
                ws[e0:e1].copy_(s)
            else:
                for e in range(e0, e1):
                    q, s = hkmoe.quant_tensor(w[e - e0])
                    wq[e].copy_(q)
                    ws[e:e + 1].copy_(s)
            del w
    torch.cuda.synchronize()
    return dict(x_q=x_q, x_scale=x_s, logits=logits, w13_q=w13_q, w13_scale=w13_s, w2_q=w2_q,
                w2_scale=w2_s, top_k=k)


def gemm_flops(cfg):
    rows = cfg["T"] * cfg["k"]
    return 2.0 * rows * (2 * cfg["I"]) * cfg["H"] + 2.0 * rows * cfg["H"] * cfg["I"]


def kernel_breakdown_mx(inp, layer, iters=10):
    """kernel_breakdown for the MX layer (its own GEMM entry points and the
    activation-exponent gather)."""
    import torch
    import tk_kernel
    import hkmoe
    pk = layer.packed
    r = hkmoe.moe_forward_mx_steps(inp["x_q"], inp["x_scale"], inp["logits"], layer.w13_q, layer.w13_words,
                                   layer.w2_q, layer.w2_words, inp["top_k"], packed=pk)
    T = inp["x_q"].shape[0]
    k = inp["top_k"]
    rows = T * k
    calls = [
        ("route_topk", lambda: tk_kernel.dispatch_route_topk(inp["logits"], r["topk_idx"], r["topk_w"], r["block_counts"])),
        ("expert_offsets", lambda: tk_kernel.dispatch_expert_offsets(r["block_counts"], T, r["counts"], r["offsets"], r["block_base"], r["mtile_offsets"], r["amax"], r["tile_ctr"], r["mtile_list"])),
        ("scatter", lambda: tk_kernel.dispatch_scatter(r["topk_idx"], r["offsets"], r["block_base"], r["perm"], r["inv_perm"], None, None, None, None)),
        ("mx_gather_words", lambda: tk_kernel.dispatch_mx_gather_scales(inp["x_scale"], r["perm"], k, r["offsets"], r["mtile_offsets"], rows, r["xw"])),
        ("grouped_gemm1", lambda: tk_kernel.dispatch_grouped_gemm1_mx(inp["x_q"], r["xw"], r["perm"], k, layer.w13_q, layer.w13_words, r["offsets"], r["mtile_offsets"], r["hq"], r["hw"], r["tile_ctr"][:8], packed=pk, mtile_list=r["mtile_list"])),
        ("grouped_gemm2", lambda: tk_kernel.dispatch_grouped_gemm2_mx(r["hq"], r["hw"], layer.w2_q, layer.w2_words, r["offsets"], r["mtile_offsets"], r["y"], r["tile_ctr"][8:], packed=pk, mtile_list=r["mtile_list"])),
        ("combine", lambda: tk_kernel.dispatch_combine(r["y"], r["topk_w"], r["inv_perm"], r["out"])),
    ]
    ev = {name: [] for name, _ in calls}
    torch.cuda.synchronize()
    for _ in range(iters):
        for name, fn in calls:
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record()
            fn()
            e.record()
            ev[name].append((s, e))
    torch.cuda.synchronize()
    ms = {name: sum(s.elapsed_time(e) for s, e in lst) / len(lst) for name, lst in ev.items()}
    return ms, r


def kernel_breakdown(inp, layer, iters=10):
    """Average ms of each kernel of the stepwise layer, events on torch's current
    stream (the stream every dispatch_* call launches on)."""
    import torch
    import tk_kernel
    import hkmoe
    if hasattr(layer, "w13_words"):
        return kernel_breakdown_mx(inp, layer, iters)
    pk = layer.packed
    w13, w2 = layer.w13_q, layer.w2_q
    block = inp["x_scale"].dim() == 2
    narrow = narrow_setting(inp)
    if narrow is not None:
        return kernel_breakdown_narrow(inp, layer, narrow, iters)
    r = hkmoe.moe_forward_steps(inp["x_q"], inp["x_scale"], inp["logits"], w13,
                                inp["w13_scale"], w2, inp["w2_scale"], inp["top_k"], packed=pk)
    T = inp["x_q"].shape[0]
    k = inp["top_k"]
    calls = [
        ("route_topk", lambda: tk_kernel.dispatch_route_topk(inp["logits"], r["topk_idx"], r["topk_w"], r["block_counts"])),
        ("expert_offsets", lambda: tk_kernel.dispatch_expert_offsets(r["block_counts"], T, r["counts"], r["offsets"], r["block_base"], r["mtile_offsets"], r["amax"], r["tile_ctr"], r["mtile_list"])),
        ("scatter", lambda: tk_kernel.dispatch_scatter(r["topk_idx"], r["offsets"], r["block_base"], r["perm"], r["inv_perm"], None, None, None, None)),
    ]
    if block:
        calls.append(("grouped_gemm1", lambda: tk_kernel.dispatch_grouped_gemm1(inp["x_q"], inp["x_scale"], r["perm"], k, w13, inp["w13_scale"], r["offsets"], r["mtile_offsets"], r["hq"], r["hs"], r["tile_ctr"][:8], packed=pk, mtile_list=r["mtile_list"])))
    else:
        calls.append(("grouped_gemm1", lambda: tk_kernel.dispatch_grouped_gemm1(inp["x_q"], inp["x_scale"], r["perm"], k, w13, inp["w13_scale"], r["offsets"], r["mtile_offsets"], r["h"], r["amax"], r["tile_ctr"][:8], packed=pk, mtile_list=r["mtile_list"])))
        calls.append(("requant", lambda: tk_kernel.dispatch_requant(r["h"], r["amax"], r["hq"], r["hs"])))
    calls += [
        ("grouped_gemm2", lambda: tk_kernel.dispatch_grouped_gemm2(r["hq"], r["hs"], w2, inp["w2_scale"], r["offsets"], r["mtile_offsets"], r["y"], r["tile_ctr"][8:], packed=pk, mtile_list=r["mtile_list"])),
        ("combine", lambda: tk_kernel.dispatch_combine(r["y"], r["topk_w"], r["inv_perm"], r["out"])),
    ]
    ev = {name: [] for name, _ in calls}
    torch.cuda.synchronize()
    for _ in range(iters):
        for name, fn in calls:
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record()
            fn()
            e.record()
            ev[name].append((s, e))
    torch.cuda.synchronize()
    ms = {name: sum(s.elapsed_time(e) for s, e in lst) / len(lst) for name, lst in ev.items()}
    return ms, r


def narrow_setting(inp):
    """(cus, max_rows, share) of the layer's narrow path, or None when the
    layer runs without it (per-tensor scales, odd K-step counts, turned off)."""
    import tk_kernel
    cus, max_rows, share = tk_kernel.get_narrow()
    hidden = inp["x_q"].shape[1]
    inter = inp["w2_q"].shape[2]
    steps = (hidden // 128, inter // 128)
    if inp["x_scale"].dim() != 2 or cus <= 0 or max_rows <= 0 or any(n % 2 or n > 64 for n in steps):
        return None
    return cus, max_rows, share


def kernel_breakdown_narrow(inp, layer, narrow, iters=10):
    """Per-kernel average ms of the split layer: the 256x256 GEMMs on the current
    stream and the narrow GEMMs on a side stream, enqueued as hkmoe_moe_forward
    does (events on the stream each kernel runs on), plus GEMM 1's span over
    both of its kernels."""
    import torch
    import tk_kernel
    import hkmoe
    cus, max_rows, share = narrow
    pk = layer.packed
    w13, w2 = layer.w13_q, layer.w2_q
    k = inp["top_k"]
    T = inp["x_q"].shape[0]
    r = hkmoe.moe_forward_steps(inp["x_q"], inp["x_scale"], inp["logits"], w13, inp["w13_scale"], w2,
                                inp["w2_scale"], k, packed=pk, narrow=narrow)
    dev = inp["x_q"].device
    main = torch.cuda.current_stream(dev)
    side = r["side"]
    n_cu = torch.cuda.get_device_properties(dev).multi_processor_count
    cus = hkmoe.layer.narrow_cus(cus, n_cu)
    grid = cus
    split = dict(packed=pk, mtile_list=r["mtile_list"], narrow_info=r["narrow_info"])
    ev = lambda: torch.cuda.Event(enable_timing=True)
    route = [
        ("route_topk", lambda: tk_kernel.dispatch_route_topk(inp["logits"], r["topk_idx"], r["topk_w"], r["block_counts"])),
        ("expert_offsets", lambda: tk_kernel.dispatch_expert_offsets(r["block_counts"], T, r["counts"], r["offsets"], r["block_base"], r["mtile_offsets"], r["amax"], r["tile_ctr"], r["mtile_list"], narrow_max=max_rows, narrow_info=r["narrow_info"])),
        ("scatter", lambda: tk_kernel.dispatch_scatter(r["topk_idx"], r["offsets"], r["block_base"], r["perm"], r["inv_perm"], None, None, None, None)),
    ]
    acc = {n: [] for n in ("route_topk", "expert_offsets", "scatter", "grouped_gemm1", "narrow_gemm1",
                           "gemm1_span", "grouped_gemm2", "narrow_gemm2", "combine")}
    torch.cuda.synchronize()
    for _ in range(iters):
        marks = {}
        for name, fn in route:
            a, b = ev(), ev()
            a.record(main)
            fn()
            b.record(main)
            marks[name] = (a, b)
        e0, e1, e2, s0, s1, s2 = ev(), ev(), ev(), ev(), ev(), ev()
        e0.record(main)
        side.wait_stream(main)
        with torch.cuda.stream(side):
            s0.record(side)
            tk_kernel.dispatch_grouped_gemm1(inp["x_q"], inp["x_scale"], r["perm"], k, w13, inp["w13_scale"], r["offsets"], r["mtile_offsets"], r["hq"], r["hs"], None, part=1, grid=grid, **split)
            s1.record(side)
            tk_kernel.dispatch_grouped_gemm2(r["hq"], r["hs"], w2, inp["w2_scale"], r["offsets"], r["mtile_offsets"], r["y"], None, part=1, grid=grid, **split)
            s2.record(side)
        tk_kernel.dispatch_grouped_gemm1(inp["x_q"], inp["x_scale"], r["perm"], k, w13, inp["w13_scale"], r["offsets"], r["mtile_offsets"], r["hq"], r["hs"], r["tile_ctr"][:8], part=0, grid=n_cu - cus if share else 0, **split)
        e1.record(main)
        tk_kernel.dispatch_grouped_gemm2(r["hq"], r["hs"], w2, inp["w2_scale"], r["offsets"], r["mtile_offsets"], r["y"], r["tile_ctr"][8:], part=0, grid=0, **split)
        e2.record(main)
        main.wait_stream(side)
        c0, c1 = ev(), ev()
        c0.record(main)
        tk_kernel.dispatch_combine(r["y"], r["topk_w"], r["inv_perm"], r["out"])
        c1.record(main)
        marks.update(grouped_gemm1=(e0, e1), narrow_gemm1=(s0, s1), grouped_gemm2=(e1, e2),
                     narrow_gemm2=(s1, s2), combine=(c0, c1), gemm1_span=(e0, (e1, s1)))
        acc_marks = marks
        for n in acc:
            acc[n].append(acc_marks[n])
    torch.cuda.synchronize()
    ms = {}
    for n, lst in acc.items():
        if n == "gemm1_span":
            ms[n] = sum(max(a.elapsed_time(b1), a.elapsed_time(b2)) for a, (b1, b2) in lst) / len(lst)
        else:
            ms[n] = sum(a.elapsed_time(b) for a, b in lst) / len(lst)
    return ms, r


def settle_run(step, seconds):
    """Back-to-back layer calls for at least `seconds` (synchronised at the
    end), run between the warm-up and the timed steps so that the timed steps
    start in the clock and power state that sustained calls settle into."""
    import torch
    calls = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            step()
        calls += 10
        torch.cuda.synchronize()
    el = time.perf_counter() - t0
    return {"seconds": round(el, 3), "calls": calls, "ms_per_call": round(el / calls * 1e3, 4) if calls else None}


# Layer roles on the main stream, in launch order (the critical path when the
# narrow kernels run on the auxiliary stream beside the 256x256 GEMM 1).
CHAIN = ("route_topk", "expert_block_scan", "expert_offsets", "scatter", "mx_gather_words", "grouped_gemm1",
         "requant", "grouped_gemm2", "combine")


def layer_kernel_timing(step, calls):
    """Per-kernel times of `calls` one-call layers, measured by the library's
    per-dispatch events (hkmoe_kernel_timing: each kernel's own start and end
    timestamps, no marker packets between kernels).  Returns the mean duration
    of each kernel role, the mean start/end of each role from the start of the
    call's first kernel (timeline), the mean span of a call (first kernel start
    to last kernel end) and the wall-clock ms per call of these timed calls."""
    import torch
    import tk_kernel
    roles = tk_kernel.TIMING_ROLES
    torch.cuda.synchronize()
    tk_kernel.kernel_timing(calls)
    try:
        t0 = time.perf_counter()
        for _ in range(calls):
            step()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / calls * 1e3
        per = [tk_kernel.kernel_timing_read(i) for i in range(calls)]
    finally:
        tk_kernel.kernel_timing(0)
    dur, beg, end = {}, {}, {}
    for i, name in enumerate(roles):
        got = [c[i] for c in per if c[i][0] >= 0]
        if got:
            dur[name] = sum(e - b for b, e in got) / len(got)
            beg[name] = sum(b for b, _ in got) / len(got)
            end[name] = sum(e for _, e in got) / len(got)
    span = sum(max(e for _, e in c) for c in per) / calls
    # with the one-stream schedule the narrow kernels follow the 256x256 ones on
    # the caller's stream and belong to the chain
    one_stream = "narrow_gemm1" in dur and beg["narrow_gemm1"] >= end.get("grouped_gemm1", 0.0)
    chain = sum(dur[n] for n in CHAIN + (("narrow_gemm1", "narrow_gemm2") if one_stream else ()) if n in dur)
    res = {"kernels_ms": dur, "calls": calls, "wall_ms_per_call": round(wall, 4), "span_ms": round(span, 4),
           "chain_sum_ms": round(chain, 4), "chain_gaps_ms": round(span - chain, 4),
           "timeline_ms": {n: [round(beg[n], 4), round(end[n], 4)] for n in dur}}
    if "narrow_gemm1" in dur and "grouped_gemm1" in dur:
        res["gemm1_span_ms"] = (max(end["grouped_gemm1"], end["narrow_gemm1"]) -
                                min(beg["grouped_gemm1"], beg["narrow_gemm1"]))
    return res


def route_counts(inp):
    """Rows per expert of the benched routing (the path's own routing kernels)."""
    import torch
    import tk_kernel
    logits, k = inp["logits"], inp["top_k"]
    T, E = logits.shape
    dev = logits.device
    nblk = tk_kernel.route_blocks(T)
    idx = torch.empty((T, k), dtype=torch.int32, device=dev)
    w = torch.empty((T, k), dtype=torch.float32, device=dev)
    bc = torch.empty((nblk, E), dtype=torch.int32, device=dev)
    tk_kernel.dispatch_route_topk(logits, idx, w, bc)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offs = torch.empty(E + 1, dtype=torch.int32, device=dev)
    mto = torch.empty(E + 1, dtype=torch.int32, device=dev)
    tk_kernel.dispatch_expert_offsets(bc, T, counts, offs, torch.empty_like(bc), mto, None)
    return counts.cpu()


def cpu_threads():
    """Host threads of the CPU baseline: the machine's cores (os.cpu_count()),
    capped by OMP_NUM_THREADS when the environment sets it (the GPU boxes give
    one GPU's job a share of the host's cores)."""
    n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(env))) if env.isdigit() and int(env) > 0 else n


def _torch_dequant_rows(q, s, mode):
    """e4m3 rows [R, C] (torch float8) -> fp32 with per-tensor s ([1]), 1x128
    group scales s [R, C/128] or MX exponents s uint8 [R, C/32]."""
    import torch
    x = q.float()
    r, c = x.shape
    if mode == "tensor":
        return x * s.reshape(())
    if mode == "mx":
        return (x.view(r, c // 32, 32) * torch.pow(2.0, s.float() - 127.0)[..., None]).view(r, c)
    return (x.view(r, c // 128, 128) * s[..., None]).view(r, c)


def _torch_dequant_weight(q, s, mode):
    """e4m3 expert weight [N, K] with per-tensor s (scalar), 128x128 block
    scales s [N/128, K/128] or MX exponents s [N, K/32]."""
    import torch
    if mode != "block":
        return _torch_dequant_rows(q, s.reshape(1) if mode == "tensor" else s, mode)
    x = q.float()
    n, k = x.shape
    return (x.view(n // 128, 128, k // 128, 128) * s[:, None, :, None]).view(n, k)


def _torch_requant(h, mode):
    """bf16-rounded h -> dequantised e4m3 values as the spec requantises them:
    1x128 groups (s = max(amax/448, 2^-126), 1 for an all-zero group),
    one per-tensor scale, or MX (1x32 e8m0)."""
    import torch
    f8 = torch.float8_e4m3fn
    r, c = h.shape
    if mode == "mx":
        g = h.view(r, c // 32, 32)
        e = torch.clamp(torch.floor(torch.log2(g.abs().amax(-1))), -127, 127)
        sc = torch.pow(2.0, e)[..., None]
        return ((g / sc).to(f8).float() * sc).view(r, c)
    if mode == "tensor":
        a = h.abs().max()
        sc = torch.clamp(a / 448.0, min=2.0 ** -126) if a > 0 else torch.tensor(1.0)
        return (h / sc).to(f8).float() * sc
    g = h.view(r, c // 128, 128)
    a = g.abs().amax(-1, keepdim=True)
    sc = torch.where(a > 0, torch.clamp(a / 448.0, min=2.0 ** -126), torch.ones_like(a))
    return ((g / sc).to(f8).float() * sc).view(r, c)


def cpu_baseline(inp, cfg, budget_s):
    """The path's PyTorch CPU version of the layer, timed on the host: route
    (top-k + softmax over the selected logits), dequantise to fp32, per expert
    x_e . W13_e^T -> SiLU(gate)*up -> bf16 -> requantise as specified ->
    . W2_e^T -> bf16, then the top-k weighted combine.

    A bounded, size-stratified sample: the active experts sorted by row count,
    every m-th of them (m = ceil(active / 24), so small, median and large
    experts are all in it), best of 3 runs.  Per-expert time is fitted as
    a + b * rows (dequantisation is per expert, the matmuls per row) and summed
    over every active expert; adding the measured combine over all T tokens
    gives the extrapolated full-layer time.  ``value`` = layer GEMM FLOPs /
    that time."""
    import math
    import numpy as np
    import torch
    threads = cpu_threads()
    torch.set_num_threads(threads)
    T, H, I, E, k = cfg["T"], cfg["H"], cfg["I"], cfg["E"], cfg["k"]
    mode = "mx" if cfg.get("mx") else "block" if cfg["block"] else "tensor"
    logits = inp["logits"].cpu()
    x_q = inp["x_q"].cpu()
    x_s = inp["x_scale"].cpu()
    t0 = time.perf_counter()
    top_v, top_i = torch.topk(logits, k, dim=1)
    top_w = torch.softmax(top_v, dim=1)
    t_route = time.perf_counter() - t0
    counts = torch.bincount(top_i.reshape(-1), minlength=E).numpy()
    active = np.flatnonzero(counts)
    order = active[np.argsort(counts[active], kind="stable")]
    m = max(1, math.ceil(len(order) / 24))
    sample = order[::m]
    flat = top_i.reshape(-1).numpy()
    w13, w2 = inp["w13_q"], inp["w2_q"]
    s13, s2 = inp["w13_scale"], inp["w2_scale"]
    per_expert = {}
    for rep in range(3):
        for e in sample:
            slots = np.flatnonzero(flat == e)
            tok = torch.from_numpy(slots // k)
            wq, wqs = w13[e].cpu(), s13[e].cpu()
            vq, vqs = w2[e].cpu(), s2[e].cpu()
            xq = x_q[tok]
            xs = x_s if mode == "tensor" else x_s[tok]
            t1 = time.perf_counter()
            xa = _torch_dequant_rows(xq, xs, mode)
            z = xa @ _torch_dequant_weight(wq, wqs, mode).T
            g, u = z[:, :I], z[:, I:]
            h = (g / (1.0 + torch.exp(-g)) * u).to(torch.bfloat16).float()
            y = (_torch_requant(h, mode) @ _torch_dequant_weight(vq, vqs, mode).T).to(torch.bfloat16)
            dt = time.perf_counter() - t1
            per_expert[int(e)] = min(per_expert.get(int(e), float("inf")), dt)
            del xa, z, h, y
    # combine over all tokens (bf16 y rows in expert order, gathered per slot)
    y_all = torch.zeros((T * k, H), dtype=torch.bfloat16)
    inv = torch.from_numpy(np.argsort(np.argsort(flat, kind="stable"), kind="stable"))
    t_comb = float("inf")
    for rep in range(3):
        t1 = time.perf_counter()
        yv = y_all[inv].view(T, k, H).float()
        out = (yv * top_w[..., None]).sum(1).to(torch.bfloat16)
        t_comb = min(t_comb, time.perf_counter() - t1)
        del yv, out
    del y_all
    rows_s = np.array([counts[e] for e in sample], np.float64)
    t_s = np.array([per_expert[int(e)] for e in sample], np.float64)
    if len(sample) >= 2 and np.ptp(rows_s) > 0:
        b, a = np.polyfit(rows_s, t_s, 1)
        a = max(a, 0.0)
    else:
        a, b = 0.0, float(t_s.sum() / rows_s.sum())
    t_experts = float(sum(a + b * counts[e] for e in active)) if m > 1 else float(t_s.sum())
    t_full = t_route + t_experts + t_comb
    flops = gemm_flops(cfg)
    return {"value": flops / t_full / 1e12, "unit": "TFLOP/s", "cores": int(threads), "kind": "port",
            "full_layer_s": round(t_full, 3),
            "sample": (f"torch CPU path ({mode} scales), {threads} threads (os.cpu_count()={os.cpu_count()}); "
                       f"{len(sample)} of {len(active)} active experts (every {m}-th by row count, "
                       f"{int(rows_s.sum())} rows), best of 3: {t_s.sum():.2f} s; "
                       + (f"full layer extrapolated with t_e = {a * 1e3:.1f} ms + {b * 1e6:.2f} us/row over all "
                          f"experts" if m > 1 else "all experts measured")
                       + f", + routing {t_route:.2f} s + combine {t_comb:.2f} s = {t_full:.1f} s")}


# ----------------------------------------------------------------------------
# rocprofv3 summaries (host only)
# ----------------------------------------------------------------------------
PROF_TRACE_CMD = ("rocprofv3 --kernel-trace --stats --output-format csv -d {d}/trace -o run -- "
                  "python3 bench.py --config {c} --steps 5 --warmup 2 --no-cpu --other-configs '' > {d}/bench.json")
PROF_TRACE_CMD_DENSE = ("rocprofv3 --kernel-trace --stats --output-format csv -d {d}/trace -o run -- "
                        "python3 bench.py --config {c} --steps 40 --warmup 5 --no-cpu > {d}/bench.json")
PROF_PMC_CMD = ("rocprofv3 --pmc {ctr} --output-format csv -d {d}/{ctr} -o run -- "
                "python3 bench.py --config {c} --steps 2 --warmup 1 --settle-s 0 --no-cpu --other-configs '' "
                "--calibrate-copy")
CALIB_BYTES = 1 << 30


def _kernel_label(name, dense=False):
    """Short label of a kernel of this library (None for other kernels)."""
    if "gemm_fp8_persistent" in name:
        if dense:
            return "gemm"
        epi = name.split("Epi)")[1][0] if "Epi)" in name else "?"
        return "grouped_gemm1" if epi in "234" else "grouped_gemm2"
    if "gemm_fp8_narrow" in name:
        epi = name.split("Epi)")[1][0] if "Epi)" in name else "?"
        return "narrow_gemm1" if epi == "3" else "narrow_gemm2"
    if "gemm_fp8_small" in name:  # the dense GEMM's 128x128-tile kernel
        return "gemm"
    n = name[len("void "):] if name.startswith("void ") else name  # template kernels
    if n.startswith("hkmoe::"):
        return n[len("hkmoe::"):].split("(")[0].split("<")[0].replace("_kernel", "")
    return None


def _algorithmic_bytes(cfg, active, narrow=None):
    """Compulsory HBM bytes per launch (inputs read once, outputs written once;
    weights of the `active` experts only).  With the narrow split (``narrow`` =
    the bench line's narrow object) the 256x256 GEMMs count the other experts and
    rows, the narrow GEMMs the narrow ones."""
    if "M" in cfg:  # dense GEMM: A, B, their scales, C
        M, N, K = cfg["M"], cfg["N"], cfg["K"]
        sc = (M + N) * (K // 32) if cfg["mx"] else 8
        return {"gemm": M * K + N * K + sc + M * N * (4 if cfg["out"] == "f32" else 2)}
    T, H, I, k = cfg["T"], cfg["H"], cfg["I"], cfg["k"]
    rows = T * k
    if cfg.get("mx"):  # one e8m0 byte per 32 elements (packed 4 per word)
        sc_x, sc_h = rows * (H // 32), rows * (I // 32)
        sw1, sw2 = active * 2 * I * (H // 32), active * H * (I // 32)
    else:
        sc_x = rows * (H // 128) * 4 if cfg["block"] else 4
        sc_h = rows * (I // 128) * 4 if cfg["block"] else 4
        sw1 = sw2 = 0
    comb = rows * H * 2 + T * H * 2 + rows * 8
    if narrow:
        ne, nr = narrow["experts"], narrow["rows"]
        we, wr = active - ne, rows - nr
        per_row_x = H + (H // 128) * 4
        per_row_h = I + (I // 128) * 4
        return {"grouped_gemm1": we * 2 * I * H + min(T, wr) * per_row_x + wr * per_row_h,
                "narrow_gemm1": ne * 2 * I * H + nr * per_row_x + nr * per_row_h,
                "grouped_gemm2": we * H * I + wr * per_row_h + wr * H * 2,
                "narrow_gemm2": ne * H * I + nr * per_row_h + nr * H * 2,
                "combine": comb}
    g1 = active * 2 * I * H + sw1 + T * H + sc_x + rows * I + sc_h
    g2 = active * H * I + sw2 + rows * I + sc_h + rows * H * 2
    return {"grouped_gemm1": g1, "grouped_gemm2": g2, "combine": comb}


def _write_timeline(f, path, n_calls):
    """The last timed one-call layer of a kernel trace (the n_calls-th routing
    launch opens it, the next one closes it): each kernel's start and end
    relative to the layer's first launch, and the CUs' idle windows it shows."""
    import csv
    if not os.path.exists(path):
        return
    with open(path) as tf:
        ks = sorted(csv.DictReader(tf), key=lambda r: int(r["Start_Timestamp"]))
    starts = [i for i, r in enumerate(ks) if "route_topk" in r["Kernel_Name"]]
    if len(starts) < n_calls:
        return
    i0 = starts[n_calls - 1]
    i1 = starts[n_calls] if len(starts) > n_calls else len(ks)
    t0 = int(ks[i0]["Start_Timestamp"])
    f.write("\nTimeline of the last timed layer call (one `MoELayer` call: with block scales the narrow "
            "kernels run on the library's auxiliary stream beside the 256x256 GEMMs, or, for decode-like "
            "shapes with T*k <= E*64, on the same stream after each of them; per-tensor layers have no "
            "narrow kernels):\n\n")
    f.write("| kernel | start us | end us | duration us |\n|---|---|---|---|\n")
    for r in ks[i0:i1]:
        lab = _kernel_label(r["Kernel_Name"], False)
        if lab is None:  # torch's own kernels between calls
            continue
        s0 = (int(r["Start_Timestamp"]) - t0) / 1e3
        s1 = (int(r["End_Timestamp"]) - t0) / 1e3
        f.write(f"| {lab} | {s0:.1f} | {s1:.1f} | {s1 - s0:.1f} |\n")


def summarize_profile(args):
    import csv
    import collections
    dense = args.config in DENSE
    cfg = DENSE[args.config] if dense else CONFIGS[args.config]
    d = args.summarize_profile
    out_dir = os.path.join(ROOT, "profiles")
    os.makedirs(out_dir, exist_ok=True)
    stats = os.path.join(d, "trace", "run_kernel_stats.csv")
    rows = []
    with open(stats) as f:
        for r in csv.DictReader(f):
            lab = _kernel_label(r["Name"], dense)
            if lab is None:
                continue
            rows.append((lab, int(r["Calls"]), float(r["AverageNs"]) / 1e3, float(r["MinNs"]) / 1e3,
                         float(r["MaxNs"]) / 1e3, float(r["TotalDurationNs"]) / 1e6))
    tot = sum(r[5] for r in rows)
    name = f"gemm_{args.config}" if dense else f"moe_layer_{args.config}"
    what = "dense GEMM" if dense else "MoE layer"
    with open(os.path.join(out_dir, f"{name}_kernels.md"), "w") as f:
        f.write(f"# rocprofv3 kernel trace: {what}, workload `{args.config}`\n\n")
        f.write(f"Config: {json.dumps(cfg)}\n\n")
        with open(os.path.join(d, "bench.json")) as bj:
            b = json.loads([ln for ln in bj if ln.startswith("{")][-1])
        if dense:
            f.write(f"bench line of the traced run: value {b['value']} {b['unit']}, "
                    f"{b['ms_per_step']} ms/step, event-timed kernel average "
                    f"{b['roofline']['avg_ms']} ms\n\n")
        else:
            f.write(f"bench line of the traced run: value {b['value']} {b['unit']}, "
                    f"{b['ms_per_step']} ms/step, weights {b['config'].get('weights')}, "
                    f"active experts {b['config']['active_experts']}, kernel averages from per-dispatch events (ms): "
                    f"{json.dumps(b['kernels_ms'])}\n\n")
        if dense:
            f.write("Command (repo root; the GEMM's call count includes the warmup calls):\n\n")
            f.write("    " + PROF_TRACE_CMD_DENSE.format(d="<out>", c=args.config) + "\n\n")
        else:
            f.write("Command (repo root; bench.py runs warm-up calls, the settle calls, the timed steps and "
                    "as many calls with per-dispatch timing events, so call counts include all of them):\n\n")
            f.write("    " + PROF_TRACE_CMD.format(d="<out>", c=args.config) + "\n\n")
        f.write("| kernel | calls | avg us | min us | max us | share of library time |\n|---|---|---|---|---|---|\n")
        for lab, n, avg, mn, mx, t in sorted(rows, key=lambda r: -r[5]):
            f.write(f"| {lab} | {n} | {avg:.1f} | {mn:.1f} | {mx:.1f} | {100 * t / tot:.1f}% |\n")
        if not dense:
            _write_timeline(f, os.path.join(d, "trace", "run_kernel_trace.csv"),
                            b["warmup"] + b.get("settle", {}).get("calls", 0) + b["steps"])
    # traffic passes
    per = {}
    calib = {}
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        path = os.path.join(d, ctr, "run_counter_collection.csv")
        agg = collections.defaultdict(lambda: collections.defaultdict(float))
        copies = collections.defaultdict(float)
        with open(path) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] != ctr:
                    continue
                if r["Kernel_Name"] == "__amd_rocclr_copyBuffer":
                    copies[r["Dispatch_Id"]] += float(r["Counter_Value"])
                lab = _kernel_label(r["Kernel_Name"], dense)
                if lab is not None:
                    agg[lab][r["Dispatch_Id"]] += float(r["Counter_Value"])
        big = max(copies.values())  # the 1 GiB calibration copy is the largest copy
        calib[ctr] = (big, CALIB_BYTES / (big * 1024.0))
        for lab, disp in agg.items():
            per.setdefault(lab, {})[ctr] = sum(disp.values()) / len(disp)
    with open(os.path.join(d, "bench.json")) as f:
        line = [ln for ln in f if ln.startswith("{")][-1]
    bench = json.loads(line)
    active = bench["config"].get("active_experts", 1)
    algo = _algorithmic_bytes(cfg, active, bench.get("narrow"))
    traffic = {}
    with open(os.path.join(out_dir, f"{name}_traffic.md"), "w") as f:
        f.write(f"# HBM traffic per launch: {what}, workload `{args.config}`\n\n")
        f.write("Two counter passes, one counter each (repo root):\n\n")
        for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
            f.write("    " + PROF_PMC_CMD.format(d="<out>", ctr=ctr, c=args.config) + "\n")
        f.write("\nCalibration: `--calibrate-copy` runs one 1 GiB device-to-device copy "
                "(`__amd_rocclr_copyBuffer`, reads and writes 1 GiB).  Factor = 1 GiB / counter "
                "reading of that copy:\n\n")
        for ctr, (raw, fac) in calib.items():
            f.write(f"- {ctr}: {raw:,.0f} KiB for the 1 GiB copy -> factor {fac:.3f}\n")
        f.write("\n| kernel | FETCH KiB (raw) | WRITE KiB (raw) | HBM read GB | HBM write GB | "
                "algorithmic GB | measured / algorithmic |\n|---|---|---|---|---|---|---|\n")
        for lab in sorted(per, key=lambda x: -per[x].get("FETCH_SIZE", 0)):
            fe = per[lab].get("FETCH_SIZE", 0.0)
            wr = per[lab].get("WRITE_SIZE", 0.0)
            rd_b = fe * 1024 * calib["FETCH_SIZE"][1]
            wr_b = wr * 1024 * calib["WRITE_SIZE"][1]
            traffic[f"{args.config}:{lab}"] = round(rd_b + wr_b)
            a = algo.get(lab)
            f.write(f"| {lab} | {fe:,.0f} | {wr:,.0f} | {rd_b / 1e9:.3f} | {wr_b / 1e9:.3f} | "
                    + (f"{a / 1e9:.3f} | {(rd_b + wr_b) / a:.2f} |\n" if a else "- | - |\n"))
        if dense:
            f.write("\nAlgorithmic bytes: A and B (e4m3) and their scales read once, C written once.\n")
        else:
            f.write(f"\nAlgorithmic bytes: operands read once, outputs written once, weights of the "
                    f"{active} active experts only (activations e4m3, intermediates e4m3 + fp32 group "
                    f"scales, y and out bf16).\n")
            if bench.get("narrow"):
                nw = bench["narrow"]
                f.write(f"The narrow kernels count the {nw['experts']} experts of at most {nw['max_rows']} rows "
                        f"({nw['rows']} rows, gathered x rows read once each); the 256x256 GEMMs the other "
                        f"{active - nw['experts']} experts (GEMM 1: x read once, at most T rows).\n")
    tj = os.path.join(out_dir, "traffic.json")
    old = {}
    if os.path.exists(tj):
        with open(tj) as f:
            old = json.load(f)
    # this config's entries are replaced as a whole: kernels the path no longer
    # launches drop out
    old = {k: v for k, v in old.items() if not k.startswith(args.config + ":")}
    old.update(traffic)
    with open(tj, "w") as f:
        json.dump(old, f, indent=1, sort_keys=True)
    print(json.dumps({"written": [f"{name}_kernels.md", f"{name}_traffic.md", "traffic.json"],
                      "traffic": traffic}))


# Counter passes (one rocprofv3 run each; every pass stays within one run's
# hardware counter limits).  MfmaUtil = MFMA-busy cycles of all SIMDs / (GPU
# active cycles x SIMDs); LDSBankConflict = LDS bank-conflict stall cycles as a
# share of GPU time; LdsBankConflict = conflict cycles per conflict-free LDS cycle.
PMC_PASSES = {
    "mfma": "MfmaUtil VALUBusy SQ_VALU_MFMA_COEXEC_CYCLES SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F8 "
            "SQ_BUSY_CYCLES",
    "lds": "LDSBankConflict LdsBankConflict SQ_INSTS_LDS SQ_WAIT_INST_LDS SQ_LDS_IDX_ACTIVE",
    "mem": "TCP_TCC_READ_REQ_LATENCY_sum TCP_TCC_READ_REQ_sum TCP_PENDING_STALL_CYCLES_sum GRBM_GUI_ACTIVE",
}
PROF_PMC_PASS_CMD = ("rocprofv3 --pmc {ctrs} --output-format csv -d {d}/{p} -o run -- "
                     "python3 bench.py --config {c} --steps 2 --warmup 1 --settle-s 0 --no-cpu --other-configs ''")


def summarize_counters(args):
    """profiles/<workload>_counters.md from the two counter passes under DIR:
    per kernel, the average over its dispatches of each metric."""
    import csv
    import collections
    dense = args.config in DENSE
    cfg = DENSE[args.config] if dense else CONFIGS[args.config]
    d = args.summarize_counters
    vals = collections.defaultdict(lambda: collections.defaultdict(list))
    for p in PMC_PASSES:
        path = os.path.join(d, p, "run_counter_collection.csv")
        per = collections.defaultdict(lambda: collections.defaultdict(float))
        names = {}
        with open(path) as f:
            for r in csv.DictReader(f):
                lab = _kernel_label(r["Kernel_Name"], dense)
                if lab is None:
                    continue
                per[(lab, r["Dispatch_Id"])][r["Counter_Name"]] += float(r["Counter_Value"])
                names[r["Counter_Name"]] = 1
        for (lab, _), ctrs in per.items():
            for c, v in ctrs.items():
                vals[lab][c].append(v)
    avg = {lab: {c: sum(v) / len(v) for c, v in cs.items()} for lab, cs in vals.items()}
    ndisp = {lab: max(len(v) for v in cs.values()) for lab, cs in vals.items()}
    name = f"gemm_{args.config}" if dense else f"moe_layer_{args.config}"
    out = os.path.join(ROOT, "profiles", f"{name}_counters.md")
    with open(out, "w") as f:
        f.write(f"# rocprofv3 counters: {'dense GEMM' if dense else 'MoE layer'}, workload `{args.config}`\n\n")
        f.write(f"Config: {json.dumps(cfg)}\n\n")
        f.write(f"{len(PMC_PASSES)} counter passes, one rocprofv3 run each (repo root):\n\n")
        for p, ctrs in PMC_PASSES.items():
            f.write("    " + PROF_PMC_PASS_CMD.format(ctrs=ctrs, d="<out>", p=p, c=args.config) + "\n")
        f.write("\nCounter collection serialises the dispatches, so every kernel runs alone on the GPU "
                "here (the narrow kernels do not overlap the 256x256 GEMMs as they do in the timed layer). "
                "MfmaUtil is MFMA-busy cycles summed over all 1024 SIMDs / (GPU-active cycles x 1024); a "
                "kernel that leaves CUs idle (the first 256x256 GEMM yields 64 CUs to the narrow kernel while "
                "narrow experts exist) is charged for them.  MFMA FLOPs = SQ_INSTS_VALU_MFMA_MOPS_F8 x 512, "
                "the FLOPs the matrix cores executed (padded rows of partial tiles included).  "
                "LDSBankConflict: bank-conflict stall cycles as % of GPU time per CU; LdsBankConflict: "
                "conflict cycles per conflict-free LDS cycle.\n\n")
        f.write("| kernel | dispatches | MfmaUtil % | VALUBusy % | MFMA-VALU co-exec / MFMA busy | MFMA TFLOP per "
                "dispatch | LDSBankConflict % | LdsBankConflict | LDS instr. per dispatch |\n"
                "|---|---|---|---|---|---|---|---|---|\n")
        for lab in sorted(avg, key=lambda x: -avg[x].get("SQ_VALU_MFMA_BUSY_CYCLES", 0)):
            a = avg[lab]
            busy = a.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0)
            co = a.get("SQ_VALU_MFMA_COEXEC_CYCLES", 0.0)

            def g(k, fmt):
                return fmt.format(a[k]) if k in a else "-"
            f.write(f"| {lab} | {ndisp[lab]} | {g('MfmaUtil', '{:.1f}')} | {g('VALUBusy', '{:.1f}')} | "
                    + (f"{co / busy:.2f}" if busy > 0 else "-") + " | "
                    + (f"{a['SQ_INSTS_VALU_MFMA_MOPS_F8'] * 512 / 1e12:.3f}" if "SQ_INSTS_VALU_MFMA_MOPS_F8" in a
                       else "-")
                    + f" | {g('LDSBankConflict', '{:.2f}')} | {g('LdsBankConflict', '{:.4f}')} | "
                    + f"{g('SQ_INSTS_LDS', '{:,.0f}')} |\n")
        if any("TCP_TCC_READ_REQ_sum" in a for a in avg.values()):
            f.write("\nMemory side (pass `mem`): L2 read latency = TCP_TCC_READ_REQ_LATENCY_sum / "
                    "TCP_TCC_READ_REQ_sum, in cycles as the CU's L1 (TCP) sees them; requests are 128 B. GPU "
                    "cycles = GRBM_GUI_ACTIVE / 8 (one count per XCD). In flight = requests per GPU cycle x "
                    "latency (Little's law), per CU of the kernel. TCP pending stall = "
                    "TCP_PENDING_STALL_CYCLES_sum / (GPU cycles x CUs of the kernel): the share of cycles an "
                    "L1 waits on data from L2.\n\n")
            f.write("| kernel | CUs | L2 read requests | L2 read latency (cycles) | GPU cycles | requests in flight "
                    "per CU | TCP pending stall % |\n|---|---|---|---|---|---|---|\n")
            ncu = {} if dense else layer_cus(cfg)
            for lab in sorted(avg, key=lambda x: -avg[x].get("TCP_TCC_READ_REQ_sum", 0)):
                a = avg[lab]
                req, lat = a.get("TCP_TCC_READ_REQ_sum", 0.0), a.get("TCP_TCC_READ_REQ_LATENCY_sum", 0.0)
                cyc = a.get("GRBM_GUI_ACTIVE", 0.0) / 8
                if req < 1e5 or cyc <= 0:
                    continue
                cus = ncu.get(lab, 256) if not dense else 256
                f.write(f"| {lab} | {cus} | {req:,.0f} | {lat / req:.0f} | {cyc:,.0f} | "
                        f"{req / cyc / cus * lat / req:.0f} | "
                        f"{100 * a.get('TCP_PENDING_STALL_CYCLES_sum', 0.0) / (cyc * cus):.0f} |\n")
    print(json.dumps({"written": [os.path.relpath(out, ROOT)]}))


def layer_cus(cfg, device_cus=256, narrow_cus=64, max_rows=64):
    """CUs each kernel of a layer runs on, under the default narrow setting:
    with narrow experts (at most max_rows rows) beside larger ones and T*k >
    2*E*max_rows (two-stream schedule) the first 256x256 GEMM keeps
    device_cus - narrow_cus and the narrow GEMMs take narrow_cus; otherwise
    (no narrow expert, the one-stream schedule, or the MX layer, which has no
    narrow path) every kernel has every CU.  The routing is the benched one
    (host_draw), its top-k taken on the host (ties cannot occur on the drawn
    floats)."""
    import numpy as np
    if cfg.get("mx") or not cfg["block"]:
        return {}
    _, logits = host_draw(cfg, 0)
    k, E = cfg["k"], cfg["E"]
    top = np.argpartition(-logits, k - 1, axis=1)[:, :k]
    counts = np.bincount(top.ravel(), minlength=E)
    narrow = int(((counts > 0) & (counts <= max_rows)).sum())
    if narrow == 0 or cfg["T"] * k <= 2 * E * max_rows:
        return {}
    return {"grouped_gemm1": device_cus - narrow_cus, "narrow_gemm1": narrow_cus, "narrow_gemm2": narrow_cus}


def dense_cpu_baseline(a_q, sa, b_q, sb, cfg, budget_s):
    """The path's PyTorch CPU version of the dense GEMM: dequantise A and B to
    fp32 (per-tensor scales, or 1x32 e8m0 for the MX shape), one fp32
    torch.matmul, best of 3 runs, timed on the host."""
    import torch
    threads = cpu_threads()
    torch.set_num_threads(threads)
    mode = "mx" if cfg["mx"] else "tensor"
    aq, bq = a_q.cpu(), b_q.cpu()
    sac, sbc = sa.cpu(), sb.cpu()
    best = float("inf")
    for rep in range(3):
        t0 = time.perf_counter()
        _ = _torch_dequant_rows(aq, sac, mode) @ _torch_dequant_rows(bq, sbc, mode).T
        best = min(best, time.perf_counter() - t0)
    flops = 2.0 * cfg["M"] * cfg["N"] * cfg["K"]
    return {"value": flops / best / 1e12, "unit": "TFLOP/s", "cores": int(threads), "kind": "port",
            "sample": f"the whole GEMM: torch dequantisation ({'1x32 e8m0' if cfg['mx'] else 'per-tensor'}) "
                      f"+ fp32 torch.matmul, {threads} threads (os.cpu_count()={os.cpu_count()}), best of 3: "
                      f"{best:.2f} s"}


def dense_main(args):
    """One step = one dense GEMM launch on resident operands."""
    import torch
    import hkmoe
    import tk_kernel
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = DENSE[args.config]
    M, N, K = cfg["M"], cfg["N"], cfg["K"]
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)
    a = torch.randn((M, K), generator=g, device=dev) * cfg["sigma"]
    b = torch.randn((N, K), generator=g, device=dev) * cfg["sigma"]
    if cfg["mx"]:
        a_q, sa = hkmoe.quant_mx(a)
        b_q, sb = hkmoe.quant_mx(b)
        pa, pb = hkmoe.mx_pack_scales(sa), hkmoe.mx_pack_scales(sb)
    else:
        a_q, sa = hkmoe.quant_tensor(a)
        b_q, sb = hkmoe.quant_tensor(b)
    del a, b
    c = torch.empty((M, N), dtype=torch.float32 if cfg["out"] == "f32" else torch.bfloat16, device=dev)
    # The reference times rotating input buffers (4_wave.cu:517-571): copies of
    # the operands at distinct addresses, used in turn, so no launch finds its
    # A and B in L2/MALL from the launch before.
    opnd_mb = (M + N) * K / 2**20
    n_rot = max(1, -(-args.rotate_mb // max(1, int(opnd_mb)))) if args.rotate_mb > 0 else 1
    if cfg["mx"]:
        ops = [(a_q, pa, b_q, pb)] + [(a_q.clone(), pa.clone(), b_q.clone(), pb.clone()) for _ in range(n_rot - 1)]
        run = lambda o: tk_kernel.dispatch_gemm_mx(o[0], o[1], o[2], o[3], c)
    else:
        ops = [(a_q, b_q, sa, sb)] + [(a_q.clone(), b_q.clone(), sa.clone(), sb.clone()) for _ in range(n_rot - 1)]
        run = lambda o: tk_kernel.dispatch_gemm_fp8(o[0], o[1], c, o[2], o[3])
    it = [0]

    def step():
        run(ops[it[0] % n_rot])
        it[0] += 1
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # Eager launches from Python: for a kernel of tens of microseconds the host
    # issue rate, not the GPU, sets this time; reported beside the value.
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) / args.steps * 1e3
    # The timed steps: the same launches, captured once into a HIP graph and
    # replayed, so they run back to back on the GPU (the wall time of one replay
    # of `steps` launches, synchronised on both sides).
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(args.steps):
            step()
    graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    kern_ms = e0.elapsed_time(e1) / args.steps  # one kernel per step, back to back on this stream
    flops = 2.0 * M * N * K
    if args.calibrate_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    traffic = None
    if os.path.exists(args.traffic):
        try:
            with open(args.traffic) as f:
                traffic = json.load(f).get(f"{args.config}:gemm")
        except Exception:
            traffic = None
    value = flops / dt / 1e12
    ach = flops / (kern_ms * 1e-3) / 1e12
    res = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "e4m3",
        "data": "synthetic (seeded torch normal on device, quantised by the path's quantisers)",
        "config": {"workload": f"{args.config}_gemm", "M": M, "N": N, "K": K,
                   "scales": "1x32 e8m0 (MX)" if cfg["mx"] else "per-tensor", "out": cfg["out"],
                   "operand_copies": n_rot, "launch": "graph"},
        "eager_ms_per_step": round(eager_ms, 4),
        "pct_fp8_peak": round(100.0 * value / PEAK_FP8_TFLOPS, 2),
        "roofline": {"bound": "mfma", "kernel": "gemm_mx" if cfg["mx"] else "gemm_fp8",
                     "achieved": round(ach, 2), "peak": PEAK_FP8_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(ach / PEAK_FP8_TFLOPS, 4), "traffic": traffic,
                     "avg_ms": round(kern_ms, 4), "flops_per_launch": flops},
    }
    if not args.no_cpu:
        res["cpu_baseline"] = dense_cpu_baseline(a_q, sa, b_q, sb, cfg, min(args.cpu_seconds, 10.0))
    print(json.dumps(res), flush=True)


def main():
    args = parse()
    if args.summarize_profile:
        summarize_profile(args)
        return
    if args.summarize_counters:
        summarize_counters(args)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: run with --gpus 1 "
                                   "(multi-GPU sharding is a design note, not a measured path)"}))
        sys.exit(2)
    if args.config in DENSE:
        dense_main(args)
        return
    import torch
    import hkmoe
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = CONFIGS[args.config]
    inp = make_inputs(cfg, args.seed, dev)
    if cfg.get("mx"):
        layer = hkmoe.MoELayerMX(inp["w13_q"], inp["w13_scale"], inp["w2_q"], inp["w2_scale"], inp["top_k"],
                                 pack=args.weights == "packed")
    else:
        layer = hkmoe.MoELayer(inp["w13_q"], inp["w13_scale"], inp["w2_q"], inp["w2_scale"], inp["top_k"],
                               pack=args.weights == "packed")
    out = torch.empty((cfg["T"], cfg["H"]), dtype=torch.bfloat16, device=dev)
    step = lambda: layer(inp["x_q"], inp["x_scale"], inp["logits"], out=out)
    if args.graph:
        # one eager call sizes the workspace; the captured call is replayed
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        step = graph.replay
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    settle = settle_run(step, args.settle_s)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    flops = gemm_flops(cfg)
    value = flops / dt / 1e12
    # the same steady state: the next `steps` one-call layers (eager) with
    # per-dispatch timing events
    eager = lambda: layer(inp["x_q"], inp["x_scale"], inp["logits"], out=out)
    kt = layer_kernel_timing(eager, max(args.steps, 1))
    ms = kt["kernels_ms"]

    if args.calibrate_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    rows = cfg["T"] * cfg["k"]
    counts = route_counts(inp)
    narrow = "narrow_gemm1" in ms
    narrow_rows = 0
    if narrow:
        _, max_rows, _ = narrow_setting(inp)
        small = (counts > 0) & (counts <= max_rows)
        narrow_rows = int(counts[small].sum())
        n_narrow = int(small.sum())
    # the dominant kernel is the 256x256 GEMM 1 over the rows it processes
    g1_flops = 2.0 * (rows - narrow_rows) * 2 * cfg["I"] * cfg["H"]
    g1_tflops = g1_flops / (ms["grouped_gemm1"] * 1e-3) / 1e12 if "grouped_gemm1" in ms else 0.0
    traffic = None
    if os.path.exists(args.traffic):
        try:
            with open(args.traffic) as f:
                traffic = json.load(f).get(f"{args.config}:grouped_gemm1")
        except Exception:
            traffic = None
    res = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "e4m3",
        "data": ("synthetic: x and logits numpy PCG64 N(0,1) in the spec generator's order, weights seeded "
                 "torch N(0,1) on device; quantised by the path's quantisers"),
        "config": {"workload": f"{args.config}_moe_layer", "T": cfg["T"], "hidden": cfg["H"],
                   "inter": cfg["I"], "experts": cfg["E"], "top_k": cfg["k"],
                   "scales": ("1x32 e8m0 (MX) weights and activations" if cfg.get("mx") else
                              "128x128 weight / 1x128 activation blocks" if cfg["block"] else "per-tensor"),
                   "routing": "zipf(1.1) skew" if cfg["skew"] else "N(0,1) logits",
                   "weights": args.weights, "launch": "hip_graph" if args.graph else "eager",
                   "active_experts": int((counts > 0).sum()), "max_rows": int(counts.max())},
        "pct_fp8_peak": round(100.0 * value / PEAK_FP8_TFLOPS, 2),
        "roofline": {"bound": "mfma",
                     "kernel": ("grouped_gemm1 256x256 (gate/up + SiLU*up), experts above the narrow "
                                "threshold" if narrow else "grouped_gemm1 (gate/up + SiLU*up)"),
                     "achieved": round(g1_tflops, 2), "peak": PEAK_FP8_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(g1_tflops / PEAK_FP8_TFLOPS, 4), "traffic": traffic,
                     "avg_ms": round(ms.get("grouped_gemm1", 0.0), 4), "flops_per_launch": g1_flops},
        "settle": settle,
        "kernels_ms": {k: round(v, 4) for k, v in ms.items()},
        "kernel_timing": {k: v for k, v in kt.items() if k != "kernels_ms"},
    }
    if "grouped_gemm1" in ms and "grouped_gemm2" in ms:
        res["gemm_only_tflops"] = round(flops / ((ms["grouped_gemm1"] + ms["grouped_gemm2"]) * 1e-3) / 1e12, 2)
    if narrow:
        # narrow kernels stream the small experts' weights: HBM-bound
        cus, max_rows, share = narrow_setting(inp)
        # with every expert narrow (T <= max_rows) no 256x256 GEMM is launched:
        # GEMM 1's span is the narrow kernel's
        g1_span = kt.get("gemm1_span_ms", ms["narrow_gemm1"])
        nb1 = n_narrow * 2 * cfg["I"] * cfg["H"]
        nb2 = n_narrow * cfg["H"] * cfg["I"]
        res["narrow"] = {
            "experts": n_narrow, "rows": narrow_rows, "max_rows": max_rows, "cus": cus, "wide_share": share,
            "gemm1": {"ms": round(ms["narrow_gemm1"], 4), "weight_bytes": nb1,
                      "GB_s": round(nb1 / ms["narrow_gemm1"] / 1e6, 1)},
            "gemm2": {"ms": round(ms["narrow_gemm2"], 4), "weight_bytes": nb2,
                      "GB_s": round(nb2 / ms["narrow_gemm2"] / 1e6, 1)},
            "gemm1_span_ms": round(g1_span, 4),
            "gemm1_span_tflops": round(2.0 * rows * 2 * cfg["I"] * cfg["H"] / (g1_span * 1e-3) / 1e12, 2),
        }
        if narrow_rows == rows:
            # every expert is narrow (decode-like): the dominant kernel is the
            # narrow GEMM 1, bound by streaming the experts' weights from HBM
            ntraffic = None
            if os.path.exists(args.traffic):
                try:
                    with open(args.traffic) as f:
                        ntraffic = json.load(f).get(f"{args.config}:narrow_gemm1")
                except Exception:
                    ntraffic = None
            res["roofline"] = {"bound": "hbm", "kernel": "narrow grouped_gemm1 (gate/up + SiLU*up)",
                               "achieved": round(nb1 / ms["narrow_gemm1"] / 1e6, 1), "peak": PEAK_HBM_GBS,
                               "unit": "GB/s", "frac": round(nb1 / ms["narrow_gemm1"] / 1e6 / PEAK_HBM_GBS, 4),
                               "traffic": ntraffic, "avg_ms": round(ms["narrow_gemm1"], 4), "bytes_per_launch": nb1}
        res.pop("gemm_only_tflops", None)
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(inp, cfg, args.cpu_seconds)
    if args.config == "dsv3" and args.other_configs:
        res["other_configs"] = other_configs(args)
    print(json.dumps(res), flush=True)


def other_configs(args):
    """Configs 1, 2, 4 and 5 (parity-test cases, not the headline): each runs as
    `bench.py --config <w>` in a child process (its own GPU memory, 10 timed
    steps after 3 warm-up steps, no CPU baseline); the fields that describe
    the result are kept."""
    import subprocess
    out = {}
    for name in [c for c in args.other_configs.split(",") if c]:
        cmd = [sys.executable, os.path.abspath(__file__), "--config", name, "--steps", "10", "--warmup", "3",
               "--no-cpu", "--other-configs", ""]
        try:
            p = subprocess.run(cmd, capture_output=True, text=True, timeout=240)
            line = [ln for ln in p.stdout.splitlines() if ln.startswith("{")]
            if p.returncode != 0 or not line:
                out[name] = {"error": f"exit {p.returncode}: {p.stderr.strip()[-300:]}"}
                continue
            d = json.loads(line[-1])
        except subprocess.TimeoutExpired:
            out[name] = {"error": "timed out"}
            continue
        keep = {k: d[k] for k in ("value", "unit", "ms_per_step", "pct_fp8_peak", "eager_ms_per_step") if k in d}
        keep["workload"] = d["config"]["workload"]
        rf = d.get("roofline", {})
        keep["roofline"] = {k: rf[k] for k in ("kernel", "bound", "achieved", "peak", "unit", "frac", "traffic", "avg_ms")
                            if k in rf}
        out[name] = keep
    return out


if __name__ == "__main__":
    main()
