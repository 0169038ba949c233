#!/usr/bin/env python3
"""Benchmark of the EXL3 grouped routed-expert MoE prefill on one MI355X.

Workload (the shape the metric is quoted on): one TP rank's share of a 288-expert layer,
H=4096, I=768, 4 bpw trellis, an 8192-token chunk, top-8 routing skewed by a Zipf(1.1) prior; synthetic seeded
inputs resident in HBM before timing starts. A step is one full grouped_prefill call (route sort, block table,
gather + input Hadamard, gate|up GEMM, SwiGLU + down Hadamard, down GEMM and its output by token: at this size the
runtime's default picks per-route fp32 rows summed per token in a fixed order, below 16384 routes the fp32 atomic
scatter; --scatter overrides). Python's garbage
collector runs, and its surviving objects are frozen, before every warm-up and timed region (quiet_gc): a full
collection inside the timed steps would stall the launching thread for 30-40 ms.

Prints ONE JSON line: value = routed tokens/s (T*topk / step time); ms_per_step = per-layer MoE ms; stage_ms = the
median over the timed steps of each stage's HIP-event time on the launch stream (stage_ms_mean beside it); roofline of
the dominant stage (the gate|up grouped GEMM: full expert tiles on the main kernel, each expert's last tile of <= 64
rows on the thin kernel; MFMA-bound: algorithmic 4*R*H*I flop per stage call over its median duration) and
roofline_down for the down GEMM and its output stages (2*R*H*I flop). From the committed rocprofv3 summaries of the same workload
(profiles/grouped_prefill_headline_*.md): traffic (calibrated FETCH_SIZE + WRITE_SIZE bytes per stage call),
stage_hbm_gbs (those bytes over this run's stage time) and counters (matrix-pipe and VALU busy fractions from
SQ_VALU_MFMA_BUSY_CYCLES / SQ_ACTIVE_INST_VALU over GRBM_GUI_ACTIVE). cpu_baseline = a PyTorch CPU expert loop (the
reference's prototype loop: dequantised fp16 weights, per-expert matmuls, index_add_ scatter) on a bounded sample of
the active experts, dequant and loop timed apart and extrapolated to the layer.

  python bench.py [--steps K] [--warmup W] [--tokens T] [--bits B] [--routing R] [--no-cpu-baseline]
  python bench.py --sweep          (extra lines for T = 1024, 2048, 4096, 8192; not the driver's contract line)
  python bench.py --decode         (the decode path, moe_decode, at small batches of the same layer: one line per
                                    batch, eager and graph-replayed; not the driver's contract line)
  python bench.py --fat            (the per-expert fat GEMM per call: config 2 and the reference's published shapes)
  python bench.py --config repro --tokens T   (the reference's published grouped-path shape; vs_baseline = its GB10
                                    per-layer ms / this run's)
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "glm53-exl3-prefill_amd")]

MFMA_F16_PEAK_TFLOPS = 2500.0      # MI355X dense fp16 (no sparsity)
# The reference's published per-layer ms of its grouped path on GB10 at the `repro` shape (288 experts, H=4096,
# I=1024 per rank, routing_skewed(hot=12, share=0.55), real checkpoint layer 3): reference README.md:41-44.
REFERENCE_GB10_MS = {1024: 11.4, 2048: 13.7, 4096: 20.2, 8192: 33.2}
HBM_PEAK_GBS = 8000.0
# The kernels of each stage of grouped_prefill as rocprofv3 names them (namespaces and parameter lists stripped; the keys
# of the committed profile summaries): the GEMMs run full expert tiles on the main kernel and each expert's last tile
# of <= 64 rows on the thin one.
STAGE_KERNELS = {
    "sort_routes": ("sort_hist_kernel", "sort_scatter_tiles_kernel"),         # + the tile tables
    "row_had": ("row_had_t16_kernel<true>",),
    "gemm_gate_up": ("trellis_gemm_kernel<{bits}, 0, false, 4, 4, false>", "trellis_gemm_kernel<{bits}, 0, false, 1, 4, true>"),
    "act_had": ("act_had_t16_kernel<false, true>",),
}
# The down projection's stages by output method: the fp32 atomic scatter by token (mode 1), or per-route fp32 rows
# (mode 2) and their fixed-order sum per token.
DOWN_STAGE_KERNELS = {
    "atomic": {"gemm_down_scatter": ("trellis_gemm_kernel<{bits}, 1, false, 4, 4, false>",
                                     "trellis_gemm_kernel<{bits}, 1, false, 1, 4, false>")},
    "combine": {"gemm_down_routes": ("trellis_gemm_kernel<{bits}, 3, false, 4, 4, false>",
                                     "trellis_gemm_kernel<{bits}, 3, false, 1, 4, true>"),
                "combine": ("combine_routes_cols_kernel<8, 0>",)},
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--tokens", type=int, default=None)
    ap.add_argument("--bits", type=int, default=None)
    ap.add_argument("--config", default="headline")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-seconds", type=float, default=20.0)
    ap.add_argument("--sweep", action="store_true")
    ap.add_argument("--decode", action="store_true", help="time the decode path (moe_decode) at small batches")
    ap.add_argument("--fat", action="store_true", help="time the per-expert fat GEMM (config 2 and the reference's "
                    "published per-call shapes)")
    ap.add_argument("--decode-tokens", default="1,4,16,32,64,128")
    ap.add_argument("--decode-no-compare", action="store_true",
                    help="with --decode: skip the prefill-path comparison (clean kernel traces of the decode path)")
    ap.add_argument("--stages", action="store_true", help="print per-stage ms to stderr")
    ap.add_argument("--scatter", choices=["atomic", "combine", "auto"], default=None,
                    help="down-projection output method (default: the runtime's, EXL3_GROUPED_SCATTER or auto)")
    ap.add_argument("--atomic-probe", action="store_true",
                    help="only time fp32 atomic adds of the down scatter's volume (65536 rows x 4096 floats into 8192 "
                         "token rows, torch index_add_) against a plain copy of the same rows, and exit")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB a few times (calibrates rocprofv3 FETCH_SIZE / "
                         "WRITE_SIZE against known bytes) and exit")
    return ap.parse_args()


def quiet_gc():
    """Run Python's cyclic garbage collector now and exempt the objects that exist so far from later collections.
    In this process a full (generation 2) collection takes ~30-40 ms of host time; one that lands inside a timed region
    stalls the launch stream (the GPU idles until the host resumes), which the per-step events show as one step of
    ~30 ms. Serving processes freeze their start-up objects the same way. Called before every warm-up (not between
    the warm-up and the timed steps: the collection leaves the GPU idle for its duration)."""
    import gc
    gc.collect()
    gc.freeze()


def copy_probe(mib: int):
    """A plain copy kernel of known size: reads and writes exactly mib MiB per launch."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.randn(n, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_per_launch": n * 4, "launches": 5}), flush=True)


def atomic_probe():
    """The scatter's fp32 atomic volume alone: out[token[r]] += src[r] for 65536 rows of 4096 floats (1.07 GB of fp32
    adds, the down scatter at the headline shape) with torch's index_add_ (one hardware fp32 atomic per element), and a
    plain device copy of the same 1.07 GB for comparison (it also reads them: twice the bytes). HIP events, median of
    5."""
    import torch
    g = torch.Generator(device="cuda:0").manual_seed(0)
    rows, width, tokens = 65536, 4096, 8192
    src = torch.randn(rows, width, device="cuda:0", generator=g)
    idx = torch.randint(0, tokens, (rows,), device="cuda:0", generator=g)
    out = torch.zeros(tokens, width, device="cuda:0")
    dst = torch.empty_like(src)
    res = {}
    for name, fn in (("atomic_add", lambda: out.index_add_(0, idx, src)), ("copy", lambda: dst.copy_(src))):
        ts = []
        for _ in range(7):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1))
        ms = statistics.median(ts[2:])
        res[name] = {"ms": round(ms, 4), "fp32_elements_per_s": round(rows * width / (ms * 1e-3), 1),
                     "bytes_per_s": round(rows * width * 4 / (ms * 1e-3), 1)}
    print(json.dumps({"atomic_probe": res, "elements": rows * width}), flush=True)


def profile_json(name: str):
    """The fenced JSON block of a committed profile summary (profiles/<name>.md), or None if it is missing."""
    try:
        text = open(os.path.join(ROOT, "profiles", f"{name}.md")).read()
        return json.loads(text.split("```json", 1)[1].split("```", 1)[0])
    except (OSError, IndexError, ValueError):
        return None


def traffic_from_profiles(workload: str, kernels):
    """HBM bytes per call of the stage made of `kernels` (one launch each) from the committed rocprofv3 --pmc summary
    of `workload` (profiles/grouped_prefill_<workload>_traffic.md: FETCH_SIZE and WRITE_SIZE passes scaled by a
    copy-kernel calibration, in its fenced JSON block), or None if the summary or one of the kernels is missing."""
    j = profile_json(f"grouped_prefill_{workload}_traffic")
    try:
        per = j["bytes_per_launch"]
        return sum(per[k] for k in kernels)
    except (TypeError, KeyError):
        return None


def mfma_busy_from_profiles(workload: str, kernels):
    """Matrix-pipe busy fraction of a stage's launches from the committed SQ counter summary: sum of
    SQ_VALU_MFMA_BUSY_CYCLES over the launches / (their GRBM_GUI_ACTIVE cycles per XCD x SIMDs), and the shader clock
    the same counters imply; None if missing."""
    j = profile_json(f"grouped_prefill_{workload}_sq_counters")
    try:
        ks = [j["kernels"][k] for k in kernels]
        busy = sum(k["SQ_VALU_MFMA_BUSY_CYCLES"] for k in ks)
        cycles = sum(k["GRBM_GUI_ACTIVE"] / j["xcds"] for k in ks)
        return {"mfma_busy": round(busy / (cycles * j["simds"]), 4),
                "valu_busy": round(sum(k["SQ_ACTIVE_INST_VALU"] for k in ks) * 4 / (cycles * j["simds"]), 4),
                "clock_mhz": j.get("clock_mhz", {}).get(kernels[0])}
    except (TypeError, KeyError, ZeroDivisionError):
        return None


def run(args, T=None, emit=True):
    import numpy as np
    import torch

    import exl3_grouped_runtime as rt
    from exl3_grouped import synth

    dev = torch.device("cuda:0")
    cfg_name = args.config
    L, x, ids, w, cfg = synth.make_config(cfg_name, seed=args.seed, T=T or args.tokens, bits=args.bits)
    TL = synth.to_device(L, dev)
    xt = torch.from_numpy(x).to(dev)
    it = torch.from_numpy(ids).to(dev)
    wt = torch.from_numpy(w).to(dev)
    T_, k, E, H, I, bits = cfg["T"], cfg["topk"], cfg["E"], cfg["H"], cfg["I"], cfg["bits"]
    R = T_ * k
    limit = 10.0

    scatter = rt.resolve_scatter(args.scatter, R)
    quiet_gc()                          # before the warm-up, whose steps then bring the clocks back up
    for _ in range(args.warmup):
        rt.grouped_prefill(xt, it, wt, TL, limit, scatter=scatter)
    torch.cuda.synchronize()

    # timed region: exactly `steps` full steps, bracketed by device synchronisation
    events = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ev = []
        out = rt.grouped_prefill(xt, it, wt, TL, limit, stage_events=ev, scatter=scatter)
        events.append(ev)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps

    stage_ms = {}
    for ev in events:
        for (name, e1), (_, e0) in zip(ev[1:], ev[:-1]):
            stage_ms.setdefault(name, []).append(e0.elapsed_time(e1))
    # per-stage medians (a host stall that starves the launch stream -- e.g. a garbage collection the freeze above
    # missed -- shows as one long step of one stage, which a mean over 20 steps misreports); the means beside them
    stage_avg = {n: statistics.median(v) for n, v in stage_ms.items()}
    stage_mean = {n: statistics.mean(v) for n, v in stage_ms.items()}
    gemm_ms = stage_avg["gemm_gate_up"]
    gate_up_flop = 4.0 * R * H * I
    down_flop = 2.0 * R * H * I
    achieved = gate_up_flop / (gemm_ms * 1e-3) / 1e12
    down_stages = list(DOWN_STAGE_KERNELS[scatter])
    down_ms = sum(stage_avg[st] for st in down_stages)
    both_gemm_tflops = (gate_up_flop + down_flop) / ((gemm_ms + down_ms) * 1e-3) / 1e12
    layer_tflops = (gate_up_flop + down_flop) / (ms_per_step * 1e-3) / 1e12
    if args.stages or not emit:
        print(json.dumps({"T": T_, "bits": bits, "scatter": scatter, "ms_per_step": round(ms_per_step, 4),
                          "stage_ms": {n: round(v, 4) for n, v in stage_avg.items()},
                          "gemm_tflops_both": round(both_gemm_tflops, 1),
                          "layer_tflops": round(layer_tflops, 1)}), file=sys.stderr, flush=True)
    workload = f"{cfg_name}: E={E} H={H} I={I} {bits}bpw T={T_} top{k} {cfg['routing']}"
    thin = rt.thin_tiles_enabled()
    kernels_of = {st: [kn.format(bits=bits) for kn in (ks if thin or not st.startswith("gemm") else ks[:1])]
                  for st, ks in {**STAGE_KERNELS, **DOWN_STAGE_KERNELS[scatter]}.items()}
    gate_up_kernels = kernels_of["gemm_gate_up"]
    down_gemm_kernels = kernels_of[down_stages[0]]
    down_kernels = [kn for st in down_stages for kn in kernels_of[st]]
    down_achieved = down_flop / (down_ms * 1e-3) / 1e12
    stage_bytes = {st: traffic_from_profiles(cfg_name, ks) for st, ks in kernels_of.items()}
    down_bytes = (sum(stage_bytes[st] for st in down_stages)
                  if all(stage_bytes[st] is not None for st in down_stages) else None)
    stage_gbs = {st: (round(b / (stage_avg[st] * 1e-3) / 1e9, 1) if b and st in stage_avg else None)
                 for st, b in stage_bytes.items()}
    result = {
        "metric": "per-layer MoE ms + routed tok/s, 288 experts @8192 tok; % MFMA peak",
        "value": round(R / (ms_per_step * 1e-3), 1),
        "unit": "routed tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": (round(REFERENCE_GB10_MS[T_] / ms_per_step, 2)
                        if cfg_name == "repro" and T_ in REFERENCE_GB10_MS else None),
        "dtype": "f16",
        "data": "synthetic (seeded random trellis codes, signs, scales, N(0,1) activations, Zipf-skewed router)",
        "config": {"workload": workload, "experts": E, "hidden": H, "intermediate": I, "bits": bits,
                   "tokens": T_, "topk": k, "routing": cfg["routing"], "routed_rows": R, "scatter": scatter,
                   "tile_rows": rt.tile_rows()},
        "tokens_per_s": round(T_ / (ms_per_step * 1e-3), 1),
        "stage_ms": {n: round(v, 4) for n, v in stage_avg.items()},
        "stage_ms_mean": {n: round(v, 4) for n, v in stage_mean.items()},
        # HBM bytes per stage call from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary of this workload
        # (calibrated against a copy kernel) over this run's stage time, against the 8 TB/s peak
        "stage_hbm_gbs": stage_gbs,
        "stage_hbm_frac": {st: (round(v / HBM_PEAK_GBS, 4) if v else None) for st, v in stage_gbs.items()},
        # matrix-pipe and VALU busy fractions of the GEMM stages from the committed SQ counter summary (against the
        # clock the counters measured, not the datasheet's)
        "counters": {"gemm_gate_up": mfma_busy_from_profiles(cfg_name, gate_up_kernels),
                     down_stages[0]: mfma_busy_from_profiles(cfg_name, down_gemm_kernels)},
        "gemm_tflops_gate_up_and_down": round(both_gemm_tflops, 1),
        "mfma_frac_layer": round(layer_tflops / MFMA_F16_PEAK_TFLOPS, 4),
        "roofline": {"kernel": "grouped_gemm gate|up stage (" + " + ".join(gate_up_kernels) + ")", "bound": "mfma",
                     "achieved": round(achieved, 1), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4),
                     "traffic": traffic_from_profiles(cfg_name, gate_up_kernels),
                     "work_per_launch": f"4*R*H*I = {gate_up_flop:.4g} flop (R={R} routed rows) per stage call",
                     "peak_source": "MI355X dense fp16 MFMA, AMD datasheet (256 CUs x 2.4 GHz x 4096 flop/clk)"},
        "roofline_down": {"kernel": ("grouped_gemm down + fp32 atomic scatter stage (" if scatter == "atomic" else
                                     "grouped_gemm down to per-route fp32 rows + combine_routes stages (")
                          + " + ".join(down_kernels) + ")",
                          "bound": "mfma", "achieved": round(down_achieved, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                          "unit": "TFLOP/s", "frac": round(down_achieved / MFMA_F16_PEAK_TFLOPS, 4),
                          "traffic": down_bytes,
                          "work_per_launch": f"2*R*H*I = {down_flop:.4g} flop per stage call"},
        "device": device_info(),
    }
    return result, (L, x, ids, w, cfg), out


def device_info():
    """Name, CU count and peak engine clock of cuda:0. The clock comes from hipDeviceGetAttribute in the HIP runtime
    the extension already loaded (dlopen by soname returns that copy); None if the query fails."""
    import ctypes

    import torch

    props = torch.cuda.get_device_properties(0)
    clock_mhz = None
    try:
        hip = ctypes.CDLL("libamdhip64.so.7")
        v = ctypes.c_int(0)
        if hip.hipDeviceGetAttribute(ctypes.byref(v), 5, 0) == 0:          # hipDeviceAttributeClockRate, kHz
            clock_mhz = round(v.value / 1e3)
    except OSError:
        pass
    return {"name": props.name, "arch": getattr(props, "gcnArchName", None), "cus": props.multi_processor_count,
            "peak_clock_mhz": clock_mhz}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(inputs, seconds: float, gpu_out=None):
    """The reference's expert loop as a PyTorch CPU loop (harness/proto_fp8.py:123-134, weights per :66-76 in the
    real domain W = diag(suh) H128 W' H128 diag(svh), W' from the CPU trellis decode): per expert gather the routed
    rows, gate = fp16(h W_g), up = fp16(h W_u), act = fp16(silu(min(gate, L)) clamp(up, -L, L)), down = act W_d,
    out.index_add_(token, down * fp16(w)); fp32 arithmetic. A bounded sample (experts largest first, about `seconds`
    of CPU work) extrapolated to the layer: dequant time per expert x active experts + loop time per routed row x
    routed rows. Also the GPU output's rel L2 against the loop on the tokens whose routes all fall in the sample."""
    import numpy as np
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import exl3_oracle as O

    L, x, ids, w, cfg = inputs
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    limit = 10.0
    H128 = torch.from_numpy(O.sylvester(128).astype(np.float32)) / np.sqrt(128.0)

    def full_weight(trellis, suh, svh):
        wp = torch.from_numpy(O.reconstruct(trellis).astype(np.float32))                # W' [K, N]
        K, N = wp.shape
        wr = (H128 @ wp.view(-1, 128, N)).view(K, N) * torch.from_numpy(suh.astype(np.float32))[:, None]
        wr = (wr.view(K, -1, 128) @ H128).view(K, N) * torch.from_numpy(svh.astype(np.float32))[None, :]
        return wr

    x16 = torch.from_numpy(np.asarray(x)).to(torch.float16).float()
    ids_t = torch.from_numpy(ids)
    w16 = torch.from_numpy(np.asarray(w, dtype=np.float32)).to(torch.float16).float()
    out = torch.zeros(x16.shape[0], cfg["H"], dtype=torch.float32)
    counts = np.bincount(ids.ravel(), minlength=cfg["E"])
    order = [int(e) for e in np.argsort(-counts, kind="stable") if counts[e] > 0]
    t_deq = t_loop = 0.0
    rows = 0
    used = []
    for e in order:
        t0 = time.perf_counter()
        wg = full_weight(L.w13_trellis[e, 0], L.w13_suh[e, 0], L.w13_svh[e, 0])
        wu = full_weight(L.w13_trellis[e, 1], L.w13_suh[e, 1], L.w13_svh[e, 1])
        wd = full_weight(L.w2_trellis[e], L.w2_suh[e], L.w2_svh[e])
        t1 = time.perf_counter()
        tok, kpos = (ids_t == e).nonzero(as_tuple=True)
        h = x16.index_select(0, tok)
        gate = (h @ wg).half().float()
        up = (h @ wu).half().float()
        act = (torch.nn.functional.silu(gate.clamp(max=limit)) * up.clamp(min=-limit, max=limit)).half().float()
        down = act @ wd
        out.index_add_(0, tok, down * w16[tok, kpos].unsqueeze(-1))
        t2 = time.perf_counter()
        t_deq += t1 - t0
        t_loop += t2 - t1
        rows += int(counts[e])
        used.append(e)
        if t_deq + t_loop >= seconds:
            break
    n_active = int((counts > 0).sum())
    R = int(counts.sum())
    layer_s = t_deq / len(used) * n_active + t_loop / rows * R
    res = {"value": round(rows / (t_deq + t_loop), 1), "unit": "routed tok/s", "cores": threads, "kind": "port",
           "cpu_model": cpu_model(),
           "sample": f"PyTorch CPU expert loop on {len(used)} of {n_active} active experts (largest first), {rows} of "
                     f"{R} routed rows, one run: dequant {t_deq:.2f} s + loop {t_loop:.2f} s; host {os.cpu_count()} "
                     "cpus visible",
           "dequant_s_per_expert": round(t_deq / len(used), 4), "loop_us_per_routed_row": round(t_loop / rows * 1e6, 2),
           "ms_per_layer_extrapolated": round(layer_s * 1e3, 1),
           "routed_tok_s_extrapolated": round(R / layer_s, 1)}
    if gpu_out is not None:
        covered = np.isin(ids, np.array(used)).all(axis=1)
        if covered.any():
            g = gpu_out[covered]
            c = out.numpy()[covered]
            res["gpu_rel_l2_vs_cpu_loop"] = float(np.linalg.norm(g - c) / max(np.linalg.norm(c), 1e-30))
            res["gpu_rel_l2_tokens"] = int(covered.sum())
    return res


# The reference's published per-call ms of its per-expert fat GEMM on GB10 (variant K64/2-stage): gate|up
# M x 4096 x 2048 and down M x 1024 x 4096 (reference docs/BASELINE.md:105-106).
REFERENCE_FAT_GB10_MS = {128: (0.093, 0.032), 256: (0.093, 0.050), 512: (0.159, 0.075), 1024: (0.239, 0.146),
                         2048: (0.457, 0.272)}


def fat_bench(args):
    """Per-call time of fat_gemm_v2 (fp32 store) with HIP events: config 2 (M=4096, K=4096, N=1536), then the shapes
    the reference published per-call times for. One JSON line per shape."""
    import torch

    import exl3_grouped as gp
    from exl3_grouped import synth

    dev = torch.device("cuda:0")

    def timed(M, K, N, variant=1):
        a, packed, svh = synth.make_fat(0, M=M, K=K, N=N)
        at, pt, st = (torch.from_numpy(v).to(dev) for v in (a, packed, svh))
        out = torch.empty(M, N, dtype=torch.float32, device=dev)
        quiet_gc()
        for _ in range(args.warmup):
            gp.fat_gemm_v2(at, pt, out, st, 4, True, False, variant)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = max(args.steps, 10)
        e0.record()
        for _ in range(n):
            gp.fat_gemm_v2(at, pt, out, st, 4, True, False, variant)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    def line(name, M, K, N, ref_ms=None):
        ms = timed(M, K, N)
        tflops = 2.0 * M * K * N / (ms * 1e-3) / 1e12
        print(json.dumps({"metric": "fat GEMM ms per call", "shape": name, "M": M, "K": K, "N": N, "bits": 4,
                          "ms": round(ms, 4), "tflops": round(tflops, 1),
                          "mfma_frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                          "reference_gb10_ms": ref_ms,
                          "vs_reference": round(ref_ms / ms, 2) if ref_ms else None}), flush=True)

    line("config 2 (gate|up of one expert, N = 2 x 768)", 4096, 4096, 1536)
    for M, (gu_ms, dn_ms) in REFERENCE_FAT_GB10_MS.items():
        line("gate|up, I = 1024", M, 4096, 2048, gu_ms)
        line("down, I = 1024", M, 1024, 4096, dn_ms)


GRAPH_CALLS = 10          # decode-path calls captured in one graph for graph_in_step_us


def decode_bench(args):
    """moe_decode on the config-3 layer (E=288, H=4096, I=768) at small batches with softmax top-8 routing: HIP-event
    time per call, eager, replayed from a captured graph of one call (graph_us), and per call from a graph of
    GRAPH_CALLS calls (graph_in_step_us: a decode step's graph holds every layer, so its launch is paid once per
    step), beside the prefill path at the same batch. Its bound is
    the trellis stream of the active experts (HBM) and their decode (VALU): bytes = active experts x 3 H I bits / 8
    plus their sign / scale vectors, x and out."""
    import numpy as np
    import torch
    import exl3_grouped as gp
    import exl3_grouped_runtime as rt
    from exl3_grouped import synth

    dev = torch.device("cuda:0")
    L, _, _, _, cfg = synth.make_config("layer1k", seed=args.seed, T=1, bits=args.bits)
    TL = synth.to_device(L, dev)
    E, H, I, k, bits = cfg["E"], cfg["H"], cfg["I"], cfg["topk"], cfg["bits"]
    for T in [int(t) for t in args.decode_tokens.split(",")]:
        ids_np, w_np = synth.make_routing("softmax", T, E, k, seed=args.seed + T)
        x = torch.from_numpy(synth.make_x(T, H, args.seed + T)).to(dev).half()
        ids = torch.from_numpy(ids_np).to(dev)
        w = torch.from_numpy(w_np).to(dev)
        out = torch.empty(T, H, dtype=torch.float32, device=dev)
        ws = torch.empty(gp.moe_decode_workspace_bytes(T, k, E, H, I), dtype=torch.uint8, device=dev)

        def call():
            gp.moe_decode(x, ids, w, TL.w13_trellis, TL.w13_suh, TL.w13_svh, TL.w2_trellis, TL.w2_suh, TL.w2_svh,
                          10.0, out=out, workspace=ws)

        def timed(fn, n):
            quiet_gc()
            for _ in range(args.warmup):
                fn()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(n):
                fn()
            b.record()
            torch.cuda.synchronize()
            return a.elapsed_time(b) * 1e3 / n

        n = max(args.steps, 20)
        eager_us = timed(call, n)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            call()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            call()
        graph_us = timed(g.replay, n)
        # A decode step's graph holds every layer's call, so the graph launch is paid once per step, not per layer:
        # GRAPH_CALLS back-to-back calls in one graph, time per call.
        g_n = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_n):
            for _ in range(GRAPH_CALLS):
                call()
        graph_step_us = timed(g_n.replay, max(n // GRAPH_CALLS, 4)) / GRAPH_CALLS
        prefill_us = None if args.decode_no_compare else round(timed(lambda: rt.grouped_prefill(x, ids, w, TL, 10.0),
                                                                         n), 2)
        active = int(np.unique(ids_np).size)
        nbytes = active * (3 * H * I * bits // 8 + (H + 2 * I + I + H) * 2) + T * H * 2 + T * H * 4
        print(json.dumps({"metric": "decode-path MoE us per layer", "tokens": T, "topk": k, "active_experts": active,
                          "eager_us": round(eager_us, 2), "graph_us": round(graph_us, 2),
                          "graph_in_step_us": round(graph_step_us, 2), "graph_calls_per_step": GRAPH_CALLS,
                          "prefill_path_us": prefill_us, "bytes": nbytes,
                          "hbm_frac_graph": round(nbytes / (graph_us * 1e-6) / (HBM_PEAK_GBS * 1e9), 4),
                          "config": {"workload": f"layer1k weights: E={E} H={H} I={I} {bits}bpw top{k} softmax"}}),
              flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the path would shard "
              "as TP (an all-reduce of the fp32 outputs) or EP (an all-to-all of routed rows) across GPUs",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.atomic_probe:
        atomic_probe()
        return
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.decode:
        decode_bench(args)
        return
    if args.fat:
        fat_bench(args)
        return
    if args.sweep:
        for T in (1024, 2048, 4096, 8192):
            torch.cuda.synchronize()
            torch.cuda.empty_cache()        # each size starts from a fresh allocator pool, as in its own process
            r, _, _ = run(args, T=T, emit=False)
            r.pop("cpu_baseline", None)
            print(json.dumps(r), flush=True)
        return
    result, inputs, out = run(args)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(inputs, args.cpu_sample_seconds, gpu_out=out.cpu().numpy())
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
