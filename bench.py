"""Benchmark of the quantized matvec hot path on one MI355X.

Workload (config 1, the headline): the Qwen3-8B per-layer 4-bit decode matvec set
    q 4096->4096, k/v 4096->1024, o 4096->4096, gate/up 4096->12288, down 12288->4096
MLX-affine W4, group 64, bf16 scale/bias planes in the converter's group-output
layout, bf16 activations N(0,1), M=1. One step = one pass over the set, issued
as one stark_qmm_encode_many call (one kernel launch; argument structs are
marshalled once per layer copy, as a compiled caller holds them). Steps rotate through 36
distinct copies of the layer weights (a Qwen3-8B has 36 layers; 3.9 GB), so
every step streams its weights from HBM as a decode step does, never from the
256 MB MALL.

value = algorithmic bytes of the timed steps / wall time between HIP events on
the launch stream. roofline.achieved = algorithmic bytes per launch / mean
launch duration (per-launch HIP events). cpu_baseline = the oracle's
single-thread restatement of MatmulCpuKernel on a bounded sample of the same
layer set (weights quantized by the same rule).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
SHAPES = [("q_proj", 4096, 4096), ("k_proj", 1024, 4096), ("v_proj", 1024, 4096), ("o_proj", 4096, 4096),
          ("gate_proj", 12288, 4096), ("up_proj", 12288, 4096), ("down_proj", 4096, 12288)]
GROUP = 64
LAYERS = 36
SEED = 20261201



# Secondary lines: printed one per line when a config is run on its own; in the
# default run they are collected and attached to the headline line instead
# (bench.py prints one JSON line).
SINK = None


def emit(d):
    if SINK is not None:
        SINK.append(d)
    else:
        print(json.dumps(d))

def quantize_gpu(w, group=GROUP):
    """MLX affine quantization on the GPU (data generation only): per group
    scale=(max-min)/15, bias=min as bf16; q=clamp(round((w-bias)/scale)).
    Returns (codes u8 [N, K/2], scales/biases int16 bits [G, N] group-output)."""
    import torch
    n, k = w.shape
    g = w.view(n, k // group, group)
    mn = g.amin(dim=2)
    mx = g.amax(dim=2)
    s = ((mx - mn) / 15.0).to(torch.bfloat16)
    b = mn.to(torch.bfloat16)
    sf, bf = s.float().unsqueeze(2), b.float().unsqueeze(2)
    q = torch.where(sf > 0, torch.round((g - bf) / torch.where(sf > 0, sf, torch.ones_like(sf))),
                    torch.zeros_like(g)).clamp(0, 15).to(torch.uint8).view(n, k)
    codes = (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous()
    return codes, s.t().contiguous().view(torch.int16), b.t().contiguous().view(torch.int16)


def quantize_gpu_bits(torch, w, bits, group=GROUP):
    """MLX affine at `bits` (4 or 8): scale=(max-min)/(2^bits-1),
    bias=min as bf16; codes little-endian (low nibble first for 4-bit)."""
    if bits == 4:
        return quantize_gpu(w, group)
    n, k = w.shape
    g = w.view(n, k // group, group)
    mn, mx = g.amin(dim=2), g.amax(dim=2)
    s = ((mx - mn) / 255.0).to(torch.bfloat16)
    b = mn.to(torch.bfloat16)
    sf, bf = s.float().unsqueeze(2), b.float().unsqueeze(2)
    q = torch.where(sf > 0, torch.round((g - bf) / torch.where(sf > 0, sf, torch.ones_like(sf))),
                    torch.zeros_like(g)).clamp(0, 255).to(torch.uint8).view(n, k).contiguous()
    return q, s.t().contiguous().view(torch.int16), b.t().contiguous().view(torch.int16)


def quantize_gguf_gpu(torch, w, kind):
    """GGUF blocks for row-major w [N, K] (data generation on the GPU):
    Q8_0: d = amax/127 (f16), q = round(x/d) int8, 34-byte blocks;
    Q4_K: per 32-value sub-block scale (max-min)/15 and min, quantised to 6 bits
    against the super-block's d/dmin (f16), 144-byte super-blocks laid out as
    ggml's block_q4_K (d, dmin, 12 packed scale/min bytes, 128 nibble bytes)."""
    n, k = w.shape
    if kind == 8:
        g = w.view(n, k // 32, 32)
        d = (g.abs().amax(dim=2) / 127.0).to(torch.float16)
        df = d.float().unsqueeze(2)
        q = torch.where(df > 0, torch.round(g / torch.where(df > 0, df, torch.ones_like(df))),
                        torch.zeros_like(g)).clamp(-127, 127).to(torch.int8)
        out = torch.empty(n, k // 32, 34, dtype=torch.uint8, device=w.device)
        out[:, :, 0:2] = d.view(torch.uint8).view(n, k // 32, 2)
        out[:, :, 2:] = q.view(torch.uint8)
        return out.view(-1)
    g = w.view(n, k // 256, 8, 32)
    mn = torch.clamp(g.amin(dim=3), max=0.0)
    sc = (g.amax(dim=3) - mn) / 15.0
    m = -mn
    d = (sc.amax(dim=2) / 63.0).to(torch.float16)
    dmin = (m.amax(dim=2) / 63.0).to(torch.float16)
    dfl, dmf = d.float().unsqueeze(2), dmin.float().unsqueeze(2)
    scq = torch.where(dfl > 0, torch.round(sc / torch.where(dfl > 0, dfl, torch.ones_like(dfl))),
                      torch.zeros_like(sc)).clamp(0, 63)
    mq = torch.where(dmf > 0, torch.round(m / torch.where(dmf > 0, dmf, torch.ones_like(dmf))),
                     torch.zeros_like(m)).clamp(0, 63)
    step = (dfl * scq).unsqueeze(3)
    q = torch.where(step > 0, torch.round((g + (dmf * mq).unsqueeze(3)) / torch.where(step > 0, step, torch.ones_like(step))),
                    torch.zeros_like(g)).clamp(0, 15).to(torch.int32)
    sci, mi = scq.to(torch.int32), mq.to(torch.int32)
    scales = torch.empty(n, k // 256, 12, dtype=torch.int32, device=w.device)
    scales[..., 0:4] = (sci[..., 0:4] & 63) | ((sci[..., 4:8] >> 4) << 6)
    scales[..., 4:8] = (mi[..., 0:4] & 63) | ((mi[..., 4:8] >> 4) << 6)
    scales[..., 8:12] = (sci[..., 4:8] & 15) | ((mi[..., 4:8] & 15) << 4)
    # element part*64 + half*32 + l sits in qs[part*32 + l] at shift 4*half (sub-block 2*part + half)
    qv = q.view(n, k // 256, 4, 2, 32)
    qs = (qv[:, :, :, 0, :] | (qv[:, :, :, 1, :] << 4)).reshape(n, k // 256, 128)
    out = torch.empty(n, k // 256, 144, dtype=torch.uint8, device=w.device)
    out[:, :, 0:2] = d.view(torch.uint8).view(n, k // 256, 2)
    out[:, :, 2:4] = dmin.view(torch.uint8).view(n, k // 256, 2)
    out[:, :, 4:16] = scales.to(torch.uint8)
    out[:, :, 16:] = qs.to(torch.uint8)
    return out.view(-1)


def algorithmic_bytes(m=1):
    total = 0
    for _, n, k in SHAPES:
        n4 = (n + 3) // 4 * 4
        total += n * k // 2 + 2 * (k // GROUP) * n4 * 2 + m * k * 2 + m * n * 2
    return total


def build_layer_set(torch, Q, gen):
    """One layer's matrices (quantized on the GPU) + activations."""
    mats = []
    for name, n, k in SHAPES:
        w = torch.randn(n, k, generator=gen, device="cuda") * 0.02
        codes, s, b = quantize_gpu(w)
        del w
        mats.append(dict(name=name, n=n, k=k, codes=codes, scales=s, biases=b))
    return mats


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(torch, layer, xs, budget_s=12.0):
    """The oracle (MatmulCpuKernel::encode restated) on the host over whole
    layer-set passes, for about budget_s of wall time per mode:
      A: one thread, the reference CPU backend's single worker
         (crates/stark-engine/src/backends/cpu/context.rs:26-30);
      B: OpenMP over the output rows on every host core this process may use
         (per-output arithmetic order unchanged, so bit-identical to A).
    Returns GB/s of algorithmic bytes; mode B is the reported value."""
    import numpy as np
    from oracle import oracle as O
    O.lib()
    host = []
    for mat, x in zip(layer, xs):
        host.append(dict(n=mat["n"], k=mat["k"], codes=mat["codes"].cpu().numpy(),
                         s=mat["scales"].cpu().numpy().view(np.uint16), b=mat["biases"].cpu().numpy().view(np.uint16),
                         x=x.view(torch.int16).cpu().numpy().view(np.uint16)))

    def run(threads):
        passes, bytes_done, t0 = 0, 0, time.perf_counter()
        outs = []
        while True:
            outs = []
            for h in host:
                st, y = O.matmul(a=h["x"], m=1, n=h["n"], k=h["k"], codes=h["codes"], scales=h["s"],
                                 correction_data=h["b"], layout=O.GROUP_OUTPUT, bits=4, group_size=GROUP,
                                 output_dt=O.BF16, threads=threads)
                assert st == 0
                outs.append(np.asarray(y).copy())
            passes += 1
            bytes_done += algorithmic_bytes(1)
            el = time.perf_counter() - t0
            if el >= budget_s or passes >= 400:
                return bytes_done / el / 1e9, passes, el, outs

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    cores = max(1, min(cores, int(os.environ.get("OMP_NUM_THREADS", cores))))
    a_gbs, a_passes, a_el, a_out = run(0)
    b_gbs, b_passes, b_el, b_out = run(cores)
    assert all(np.array_equal(u, v) for u, v in zip(a_out, b_out)), "mode B must be bit-identical to mode A"
    return dict(value=round(b_gbs, 4), unit="GB/s", cores=cores, kind="port",
                cpu_model=_cpu_model(),
                single_thread=dict(value=round(a_gbs, 4), cores=1,
                                   sample=f"{a_passes} passes, {a_el:.1f} s"),
                sample=f"mode B: {b_passes} full passes over one Qwen3-8B W4 layer matvec set (M=1) with OpenMP "
                       f"over output rows on {cores} threads, {b_el:.1f} s; oracle restatement of "
                       f"MatmulCpuKernel::encode, bit-identical to the single-thread mode A")


def copy_calibration(torch, mib=256):
    """A plain device pass of known size (reads `mib` MiB, writes `mib` MiB),
    run under rocprofv3 --pmc to scale FETCH_SIZE / WRITE_SIZE to bytes."""
    src = torch.full(((mib << 20) // 4,), 1, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        torch.bitwise_not(src, out=dst)
    torch.cuda.synchronize()


def config1(args, torch, Q):
    """Config 1: the Qwen3-8B W4 layer matvec set at M=1 (the headline line)."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED)

    layer0 = build_layer_set(torch, Q, gen)
    xs = {}
    for name, n, k in SHAPES:
        key = {"k_proj": "q_proj", "v_proj": "q_proj", "up_proj": "gate_proj"}.get(name, name)
        if key not in xs:
            xs[key] = torch.randn(k, generator=gen, device="cuda").to(torch.bfloat16)
        xs[name] = xs[key]
    x_list = [xs[name] for name, _, _ in SHAPES]
    # 36 distinct weight copies (same values, distinct memory) so that every
    # step reads HBM, as successive decode layers do.
    layers = [layer0] + [[{**m, "codes": m["codes"].clone(), "scales": m["scales"].clone(),
                           "biases": m["biases"].clone()} for m in layer0] for _ in range(args.copies - 1)]
    outs = [torch.empty(n, dtype=torch.int16, device="cuda") for _, n, _ in SHAPES]

    def layer_args(layer):
        return [Q.MatmulArguments(a=x.view(torch.int16), m=1, n=mat["n"], k=mat["k"], d=out,
                                  b=Q.QuantizedB(codes=mat["codes"], scales=mat["scales"],
                                                 params=Q.QuantParams(Q.GROUP_OUTPUT, mat["n"], mat["k"] // GROUP),
                                                 correction_data=mat["biases"]))
                for mat, x, out in zip(layer, x_list, outs)]

    kern = Q.MatmulKernel(Q.BF16, Q.BF16, Q.BF16)
    # argument structs marshalled once per layer copy (a compiled caller keeps them)
    all_args = [kern.prepare_many(layer_args(l)) for l in layers]
    stream = torch.cuda.current_stream()

    if args.calibrate_copy:
        copy_calibration(torch)

    # setup, outside the timed region: one pass over every copy (first touch of
    # all 3.9 GB), checking the property that copies of the same weights give
    # bit-identical outputs
    ref = None
    for i in range(args.copies):
        kern.encode_prepared(all_args[i], stream)
        got = torch.cat([o.clone() for o in outs])
        if ref is None:
            ref = got
        elif not torch.equal(got, ref):
            raise SystemExit(f"bench: layer copy {i} gave different outputs from copy 0")
    torch.cuda.synchronize()

    clock_ramp(torch, lambda i: kern.encode_prepared(all_args[i % args.copies], stream))
    for i in range(args.warmup):
        kern.encode_prepared(all_args[i % args.copies], stream)
    torch.cuda.synchronize()

    # timed region: K steps between two events on the launch stream
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(args.steps):
        kern.encode_prepared(all_args[i % args.copies], stream)
    stop.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(stop)

    # per-launch durations (events bracket each launch on the same stream)
    n_lat = min(args.steps, 180)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n_lat)]
    for i in range(n_lat):
        evs[i][0].record(stream)
        kern.encode_prepared(all_args[i % args.copies], stream)
        evs[i][1].record(stream)
    torch.cuda.synchronize()
    launch_ms = sorted(a.elapsed_time(b) for a, b in evs)
    mean_launch_ms = sum(launch_ms) / len(launch_ms)

    bytes_step = algorithmic_bytes(1)
    ms_step = total_ms / args.steps
    value = bytes_step / (ms_step * 1e-3) / 1e9
    # one qmv_stream launch per step: its average duration over the timed region
    # is the events' span / K (dispatch gaps included, so it bounds the kernel's
    # own mean from above); the per-launch event pairs above isolate every
    # launch (each waits for the previous one to drain) and are kept as a
    # diagnostic only
    achieved = bytes_step / (ms_step * 1e-3) / 1e9
    traffic = None
    tfile = os.path.join(ROOT, "profiles", "qmv_stream_w4_layerset_pmc.md")
    if os.path.exists(tfile):
        import re
        hit = re.search(r"hbm_bytes_per_launch\s*=\s*(\d+)", open(tfile).read())
        traffic = int(hit.group(1)) if hit else None

    decode = None
    if args.decode_tokens:
        decode = decode_measure(args, torch)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(torch, layer0, x_list)

    line = {
        "metric": "q4 matvec HBM GB/s (% of peak); Qwen3-8B-shape q4 decode tokens/s at 1 GPU",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init N(0,0.02) weights quantized W4 g64 (MLX affine rule), bf16 N(0,1) activations",
        "config": {
            "workload": "Qwen3-8B layer matvec set q,k,v,o,gate,up,down; MLX-affine W4 g64 bf16 planes; M=1; "
                        f"{args.copies} rotating layer copies; one stark_qmm_encode_many launch per step",
            "bytes_per_step": bytes_step,
            "pct_of_peak_hbm": round(100.0 * value / PEAK_HBM_GBS, 2),
            "matvec_only_layer_sets_per_s_over_36": round(1000.0 / (ms_step * LAYERS), 1),
            "isolated_launch_ms_median": round(launch_ms[len(launch_ms) // 2], 5),
            "isolated_launch_ms_mean": round(mean_launch_ms, 5),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "kernel": ("qmv_w4_decode (VALU form, STARK_QMM_FORCE_VALU_DECODE=1)"
                       if os.environ.get("STARK_QMM_FORCE_VALU_DECODE") == "1"
                       else "qmv_stream<false> (one persistent launch per step)"),
            "launch_ms": round(ms_step, 5),
        },
        "cpu_baseline": cpu,
    }
    if decode is not None:
        line["config"]["decode_tokens_per_s"] = decode["tokens_per_s"]
        line["config"]["decode"] = decode
    if args.headline_only:
        print(json.dumps(line))
        if args.verify:
            verify_lines(args, torch, Q, gen, kern, layers, stream)
        return
    # The other configurations, measured in the same run and attached to this
    # line (one line per run): verify M = 2..16 and M = 32, 64, config 2, config 3, config 4
    # prefill (bf16 and int8 activations). Each is summarised; a failure is
    # recorded in place of its figures and does not stop the run.
    global SINK
    SINK = []
    others = []

    def collect(what, fn):
        del SINK[:]
        t0 = time.time()
        try:
            fn()
            for d in SINK:
                rf = d.get("roofline") or {}
                others.append({"metric": d["metric"], "value": d["value"], "unit": d["unit"],
                               "ms_per_step": d.get("ms_per_step"), "steps": d.get("steps"),
                               "workload": d.get("config", {}).get("workload"),
                               "roofline_frac": rf.get("frac"), "wall_s": round(time.time() - t0, 1)})
        except Exception as e:  # recorded, not fatal: the headline figures above stand
            others.append({"metric": what, "error": f"{type(e).__name__}: {e}"[:300]})
        print(f"bench: {what} done in {time.time() - t0:.1f} s", file=sys.stderr, flush=True)

    collect("config 1 verify M=2,4,8,16,32,64,128,256", lambda: verify_lines(args, torch, Q, gen, kern, layers, stream))
    del all_args, layers, outs
    torch.cuda.empty_cache()
    sub = argparse.Namespace(**{**vars(args), "steps": 200, "warmup": 40, "decode_tokens": 0})
    collect("config 2", lambda: config2(sub, torch, Q))
    torch.cuda.empty_cache()
    collect("config 3", lambda: config3(sub, torch, Q))
    torch.cuda.empty_cache()
    collect("config 4 prefill", lambda: config4(argparse.Namespace(**{**vars(sub), "steps": 20, "warmup": 3}),
                                                torch, Q))
    torch.cuda.empty_cache()
    SINK = None
    line["other_configs"] = others
    print(json.dumps(line))


def verify_lines(args, torch, Q, gen, kern, layers, stream):
    """Config 1 at M = 2, 4, 8, 16 (speculative verify), 32, 64 (short
    prefill chunks, the skinny dequant product) and 128, 256 (the
    dequant-GEMM's 128-row tiles): the same layer set and
    rotating copies, M activation rows per product (q/k/v and gate/up share
    theirs), one line each (attached to the default run's line)."""
    for m in (2, 4, 8, 16, 32, 64, 128, 256):
        xs = {}
        for name, n, k in SHAPES:
            key = {"k_proj": "q_proj", "v_proj": "q_proj", "up_proj": "gate_proj"}.get(name, name)
            if key not in xs:
                xs[key] = torch.randn(m * k, generator=gen, device="cuda").to(torch.bfloat16)
            xs[name] = xs[key]
        outs = [torch.empty(m * n, dtype=torch.int16, device="cuda") for _, n, _ in SHAPES]
        all_args = [kern.prepare_many([Q.MatmulArguments(
            a=xs[name].view(torch.int16), m=m, n=mat["n"], k=mat["k"], d=out,
            b=Q.QuantizedB(codes=mat["codes"], scales=mat["scales"],
                           params=Q.QuantParams(Q.GROUP_OUTPUT, mat["n"], mat["k"] // GROUP),
                           correction_data=mat["biases"]))
            for (name, _, _), mat, out in zip(SHAPES, layer, outs)]) for layer in layers]
        ms = timed(torch, lambda i: kern.encode_prepared(all_args[i % args.copies], stream), args.steps,
                   args.warmup, stream)
        nbytes = algorithmic_bytes(m)
        gbs = nbytes / (ms * 1e-3) / 1e9
        what = ("speculative verify" if m <= 16 else "short prefill, bf16-effective weights" if m <= 64
                else "short prefill, dequant-GEMM")
        emit({"metric": f"q4 matvec HBM GB/s at M={m} ({what})", "value": round(gbs, 1),
                          "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
                          "vs_baseline": None, "dtype": "bf16",
                          "data": "synthetic: the config-1 layer set, bf16 N(0,1) activations",
                          "config": {"workload": f"config 1 verify: Qwen3-8B layer matvec set at M={m}, "
                                                 f"{args.copies} rotating layer copies, one launch per step",
                                     "bytes_per_step": nbytes,
                                     "pct_of_peak_hbm": round(100.0 * gbs / PEAK_HBM_GBS, 2),
                                     "tokens_per_s": round(m * 1000.0 / ms, 1),
                                     "tflop_s": round(2.0 * m * sum(n * k for _, n, k in SHAPES) / (ms * 1e-3) / 1e12, 1)},
                          "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                                       "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None}})


def clock_ramp(torch, step, seconds=0.4):
    """Setup, outside the timed region: run step(i) back to back for `seconds`
    so the GPU leaves its idle clock state before the warmup and timed steps
    (a cold GPU runs the first few thousand launches up to 10% slower)."""
    t0 = time.perf_counter()
    i = 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(64):
            step(i)
            i += 1
        torch.cuda.synchronize()


def timed(torch, step, steps, warmup, stream):
    """Warm up, then time `steps` calls of step(i) between two events on the
    launch stream; also the mean of per-call event pairs. Returns ms per step."""
    clock_ramp(torch, step)
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for i in range(steps):
        step(i)
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


EAGER = False  # --eager: graph_timed issues the calls one by one (counter passes under rocprofv3)


def graph_timed(torch, step, count, steps):
    """Capture `count` calls step(i, stream) (each on its own weight copy) in
    one HIP graph, replay it until at least `steps` calls have run after a
    clock ramp and one warm replay, and time the replays between two events.
    Python dispatch is outside the figure. Returns ms per call. With --eager
    the calls are issued one by one instead (Python dispatch included)."""
    if EAGER:
        cur = torch.cuda.current_stream()
        ms = timed(torch, lambda i: step(i % count, cur), steps, count, cur)
        return ms, steps
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(count):  # eager pass: builds the per-shape schedules
            step(i, s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(count):
                step(i, s)
    torch.cuda.synchronize()
    clock_ramp(torch, lambda i: g.replay())
    g.replay()
    torch.cuda.synchronize()
    reps = max(1, -(-steps // count))
    cur = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(cur)
    for _ in range(reps):
        g.replay()
    b.record(cur)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / (reps * count)
    del g
    return ms, reps * count


ROTATION_BYTES = 1.1 * 2 ** 30  # config 2: each format's copies cover more than 1 GiB (4x the MALL)


def config2(args, torch, Q):
    """Config 2: N=12288, K=4096 at M=1 and M=8 in MLX-affine 8-bit g64,
    GGUF Q8_0 and GGUF Q4_K (one line each). Weights N(0,0.02) quantized by
    each format's rule on the GPU; every format rotates distinct copies of more
    than 1 GiB in total (past the 256 MB MALL), and the steps are timed as
    replays of one captured HIP graph over all copies."""
    N, K = 12288, 4096
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED + 2)
    w = torch.randn(N, K, generator=gen, device="cuda") * 0.02
    lines = []
    for m in (1, 8):
        x = torch.randn(m, K, generator=gen, device="cuda").to(torch.bfloat16)
        # -- MLX affine 8-bit through MatmulKernel::encode
        codes, sc, bi = quantize_gpu_bits(torch, w, 8)
        wbytes = N * K + 2 * 2 * (K // GROUP) * N
        copies = int(-(-ROTATION_BYTES // wbytes))
        mats = [(codes.clone(), sc.clone(), bi.clone()) for _ in range(copies)]
        y = torch.empty(m * N, dtype=torch.int16, device="cuda")
        kern = Q.MatmulKernel(Q.BF16, Q.BF16, Q.BF16)
        batches = [kern.prepare_many([Q.MatmulArguments(
            a=x.view(torch.int16), m=m, n=N, k=K, d=y,
            b=Q.QuantizedB(codes=c, scales=s_, correction_data=b_, mode=Q.MODE_U8,
                           params=Q.QuantParams(Q.GROUP_OUTPUT, N, K // GROUP)))]) for c, s_, b_ in mats]
        ms, ran = graph_timed(torch, lambda i, s: kern.encode_prepared(batches[i], s), copies, args.steps)
        lines.append(("mlx_affine_u8_g64", m, ms, wbytes + m * 2 * K + m * 2 * N, copies, wbytes, ran))
        del mats, batches
        # -- GGUF Q8_0 / Q4_K through the hybrid operator (stream-ordered form)
        xf = x.float().contiguous()
        status = torch.zeros(1, dtype=torch.int32, device="cuda")
        for kind, name, block, bsize in ((Q.KIND_Q8_0, "gguf_q8_0", 32, 34), (Q.KIND_Q4_K, "gguf_q4_k", 256, 144)):
            blocks = quantize_gguf_gpu(torch, w, kind)
            wbytes = N * (K // block) * bsize
            copies = int(-(-ROTATION_BYTES // wbytes))
            views = [blocks.clone() for _ in range(copies)]
            preps = []
            for v in views:
                op = Q.MappedOperation(matrices=[Q.MappedMatrix(codes=v)] * m, inputs=xf.view(-1), rows=N, columns=K,
                                       format=("packed", kind))
                preps.append(Q.mapped_prepare([op])[0])
            ms, ran = graph_timed(torch, lambda i, s: Q.mapped_many_async(preps[i], status, s), copies, args.steps)
            assert int(status.item()) == 0
            lines.append((name, m, ms, wbytes + m * 4 * K + m * 4 * N, copies, wbytes, ran))
            del views, preps
    for name, m, ms, nbytes, copies, wbytes, ran in lines:
        gbs = nbytes / (ms * 1e-3) / 1e9
        emit({"metric": f"{name} matvec HBM GB/s", "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1,
                          "steps": ran, "warmup": copies, "ms_per_step": round(ms, 5),
                          "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                          "dtype": "u8" if "u8" in name else "f32",
                          "data": "synthetic: N(0,0.02) weights quantized by the format's rule, N(0,1) activations",
                          "config": {"workload": f"config 2: {name} N={N} K={K} M={m}, {copies} rotating copies "
                                                 f"({copies * wbytes / 2 ** 30:.2f} GiB), one captured HIP graph "
                                                 f"over the copies, replayed",
                                     "bytes_per_step": nbytes, "pct_of_peak_hbm": round(100 * gbs / PEAK_HBM_GBS, 2)},
                          "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                       "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None}})
    # GGUF layer sets: the Qwen3-8B projection set (q, k, v, o, gate, up, down) in Q8_0 and
    # Q4_K as one mapped_many call at M = 8 (the hybrid engine's batched products), rotating
    # more than 1 GiB of copies, graph-timed like the lines above
    m = 8
    for kind, name, block, bsize in ((Q.KIND_Q8_0, "gguf_q8_0", 32, 34), (Q.KIND_Q4_K, "gguf_q4_k", 256, 144)):
        wbytes = sum(n * (k // block) * bsize for _, n, k in SHAPES)
        copies = int(-(-ROTATION_BYTES // wbytes))
        xs = {k: torch.randn(m, k, generator=gen, device="cuda").contiguous() for k in (4096, 12288)}
        status = torch.zeros(1, dtype=torch.int32, device="cuda")
        preps = []
        for _ in range(copies):
            mats = []
            for _, n, k in SHAPES:
                mats.append(quantize_gguf_gpu(torch, torch.randn(n, k, generator=gen, device="cuda") * 0.02, kind))
            ops = [Q.MappedOperation(matrices=[Q.MappedMatrix(codes=v)] * m, inputs=xs[k].view(-1), rows=n, columns=k,
                                     format=("packed", kind)) for (_, n, k), v in zip(SHAPES, mats)]
            preps.append((Q.mapped_prepare(ops)[0], mats))
        ms, ran = graph_timed(torch, lambda i, st: Q.mapped_many_async(preps[i][0], status, st), copies, args.steps)
        assert int(status.item()) == 0
        nbytes = wbytes + sum(m * 4 * (k + n) for _, n, k in SHAPES)
        gbs = nbytes / (ms * 1e-3) / 1e9
        emit({"metric": f"{name} layer-set matvec HBM GB/s at M={m}", "value": round(gbs, 1), "unit": "GB/s",
              "n_gpus": 1, "steps": ran, "warmup": copies, "ms_per_step": round(ms, 5), "higher_is_better": True,
              "scaling": "weak", "vs_baseline": None, "dtype": "f32",
              "data": "synthetic: N(0,0.02) weights quantized by the format's rule, N(0,1) activations",
              "config": {"workload": f"{name} Qwen3-8B projection set (7 products) in one mapped_many call, M={m}, "
                                     f"{copies} rotating copies ({copies * wbytes / 2 ** 30:.2f} GiB), one captured "
                                     f"HIP graph over the copies, replayed",
                         "bytes_per_step": nbytes, "pct_of_peak_hbm": round(100 * gbs / PEAK_HBM_GBS, 2)},
              "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                           "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None}})
        del preps


def config3(args, torch, Q):
    """Config 3: Qwen3-30B-A3B MoE layer decode: router 2048->128 bf16 matvec
    (f32 logits), then stark_qmm_routed_experts (top-8 renormalised, expert
    compaction, grouped W4 g64 gate/up + SiLU and down products, accumulate).
    Tokens 1, 4, 16; 4 rotating layer copies (1.3 GB > the MALL), timed as
    replays of one captured graph over the copies."""
    Hm, E, I, A, copies = 2048, 128, 768, 8, 4
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED + 3)
    stream = torch.cuda.current_stream()
    layers = []
    for _ in range(copies):
        wr = (torch.randn(E, Hm, generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
        up = [quantize_gpu(torch.randn(2 * I, Hm, generator=gen, device="cuda") * 0.02) for _ in range(E)]
        dn = [quantize_gpu(torch.randn(Hm, I, generator=gen, device="cuda") * 0.02) for _ in range(E)]
        # banks: rows of every expert stacked; planes [G, rows] in group-output layout
        ub = (torch.cat([u[0] for u in up]), torch.cat([u[1] for u in up], 1).contiguous(),
              torch.cat([u[2] for u in up], 1).contiguous())
        db = (torch.cat([d[0] for d in dn]), torch.cat([d[1] for d in dn], 1).contiguous(),
              torch.cat([d[2] for d in dn], 1).contiguous())
        del up, dn
        layers.append((wr, ub, db))
    per_expert = 2 * I * Hm // 2 + Hm * I // 2 + 2 * 2 * (Hm // GROUP) * 2 * I + 2 * 2 * (I // GROUP) * Hm
    for T in args.tokens:
        x = torch.randn(T, Hm, generator=gen, device="cuda").to(torch.bfloat16)
        logits = torch.empty(T * E, dtype=torch.float32, device="cuda")
        out = torch.empty(T * Hm, dtype=torch.bfloat16, device="cuda")
        rk = Q.MatmulKernel(Q.BF16, Q.BF16, Q.F32)
        ws = torch.empty(Q.routed_experts_workspace_size(T, Hm, I, E, A), dtype=torch.uint8, device="cuda")
        steps = []
        uniq = []
        for wr, ub, db in layers:
            rb = rk.prepare_many([Q.MatmulArguments(a=x.view(torch.int16), m=T, n=E, k=Hm, d=logits,
                                                    b=Q.FullPrecisionB(values=wr.view(torch.int16)))])
            upb = Q.QuantizedB(codes=ub[0], scales=ub[1].view(-1), correction_data=ub[2].view(-1),
                               params=Q.QuantParams(Q.GROUP_OUTPUT, E * 2 * I, Hm // GROUP))
            dnb = Q.QuantizedB(codes=db[0], scales=db[1].view(-1), correction_data=db[2].view(-1),
                               params=Q.QuantParams(Q.GROUP_OUTPUT, E * Hm, I // GROUP))
            prep = Q.routed_experts(x.view(torch.int16), logits, upb, dnb, T, Hm, I, E, A, workspace=ws,
                                    output=out, prepare_only=True)
            steps.append((rb, prep))
            rk.encode_prepared(rb, stream)
            ids, _ = Q.moe_route(logits, T, E, A)
            torch.cuda.synchronize()
            uniq.append(len(set(ids.cpu().tolist())))

        def step(i, s):
            rb, prep = steps[i]
            rk.encode_prepared(rb, s)
            Q.routed_experts_prepared(prep, s)

        ms, ran = graph_timed(torch, step, copies, args.steps)
        u = sum(uniq) / len(uniq)
        nbytes = u * per_expert + E * Hm * 2 + T * Hm * 2 * 2 + T * E * 4
        gbs = nbytes / (ms * 1e-3) / 1e9
        emit({"metric": "Qwen3-30B-A3B MoE layer decode HBM GB/s", "value": round(gbs, 1), "unit": "GB/s",
                          "n_gpus": 1, "steps": ran, "warmup": copies, "ms_per_step": round(ms, 5),
                          "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
                          "data": "synthetic: N(0,0.02) weights W4 g64 (MLX affine rule), N(0,1) hidden states",
                          "config": {"workload": f"config 3: router + routed experts, tokens={T}, E={E}, top-{A}, "
                                                 f"H={Hm}, I={I}, {copies} rotating layer copies, one captured HIP "
                                                 f"graph over the copies, replayed",
                                     "unique_experts": u, "bytes_per_step": int(nbytes),
                                     "tokens_per_s": round(T * 1000.0 / ms, 1),
                                     "pct_of_peak_hbm": round(100 * gbs / PEAK_HBM_GBS, 2)},
                          "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                       "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None}})


PEAK_MFMA_INT8_TOPS = 5000.0
PEAK_MFMA_BF16_TFLOPS = 2500.0


def config4(args, torch, Q):
    """Config 4 (prefill part): M=2048 tokens through the Qwen3-8B W4 g64
    projection set on the matrix-core dequant-GEMM; one step = the seven
    products (q, k, v, o, gate, up, down) of one layer."""
    Mtok = 2048
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED + 4)
    stream = torch.cuda.current_stream()
    layer = build_layer_set(torch, Q, gen)
    kern = Q.MatmulKernel(Q.BF16, Q.BF16, Q.BF16)
    xs = {k: torch.randn(Mtok, k, generator=gen, device="cuda").to(torch.bfloat16) for k in (4096, 12288)}
    outs = [torch.empty(Mtok * mat["n"], dtype=torch.int16, device="cuda") for mat in layer]
    args_list = [Q.MatmulArguments(a=xs[mat["k"]].view(torch.int16), m=Mtok, n=mat["n"], k=mat["k"], d=out,
                                   b=Q.QuantizedB(codes=mat["codes"], scales=mat["scales"],
                                                  params=Q.QuantParams(Q.GROUP_OUTPUT, mat["n"], mat["k"] // GROUP),
                                                  correction_data=mat["biases"]))
                 for mat, out in zip(layer, outs)]
    batch = kern.prepare_many(args_list)
    ms = timed(torch, lambda i: kern.encode_prepared(batch, stream), args.steps, args.warmup, stream)
    flops = sum(2 * Mtok * n * k for _, n, k in SHAPES)
    tf = flops / (ms * 1e-3) / 1e12
    emit({"metric": "Qwen3-8B W4 prefill dequant-GEMM TFLOP/s", "value": round(tf, 1), "unit": "TFLOP/s",
                      "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
                      "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
                      "data": "synthetic: N(0,0.02) weights W4 g64 (MLX affine rule), N(0,1) bf16 activations",
                      "config": {"workload": f"config 4 prefill: M={Mtok} through q,k,v,o,gate,up,down (one layer)",
                                 "flops_per_step": flops, "prefill_tokens_per_s_36_layers":
                                     round(Mtok * 1000.0 / (ms * LAYERS), 1)},
                      "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": PEAK_MFMA_BF16_TFLOPS,
                                   "unit": "TFLOP/s", "frac": round(tf / PEAK_MFMA_BF16_TFLOPS, 4),
                                   "traffic": None}})
    a8_prefill_line(args, torch, Q, layer, stream)
    if args.decode_tokens:
        decode_line(args, torch)


def a8_prefill_line(args, torch, Q, layer, stream):
    """Config 4 prefill with int8 activations (MatmulA::Int8Symmetric, the
    A8W4 path): M=2048 codes per projection input (activation groups of 128,
    grouped-by-nibble order, made by the library's own quantizing transform),
    the same W4 g64 weights, on the int8 matrix-core GEMM."""
    Mtok, AG = 2048, 128
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED + 5)
    kern = Q.MatmulKernel(Q.BF16, Q.BF16, Q.BF16)
    quant = Q.ActivationTransform.quantize(Q.BF16, Q.ActivationQuantization.new(AG, GROUP, False, Q.GROUPED_BY_NIBBLE))
    acts = {}
    for k in (4096, 12288):
        x = torch.randn(Mtok * k, generator=gen, device="cuda").to(torch.bfloat16)
        f = (torch.randint(0, 2, (k,), generator=gen, device="cuda", dtype=torch.int32) * 2 - 1)
        codes = torch.empty(Mtok * k, dtype=torch.int8, device="cuda")
        scales = torch.empty(Mtok * k // AG, dtype=torch.float32, device="cuda")
        quant.encode_quantize(x.view(torch.int16), codes, scales, None, f, Mtok, k, stream)
        acts[k] = Q.Int8SymmetricA(values=codes, scales=scales, scale_group_size=AG, code_layout=Q.GROUPED_BY_NIBBLE)
    outs = [torch.empty(Mtok * mat["n"], dtype=torch.int16, device="cuda") for mat in layer]
    args_list = [Q.MatmulArguments(a=acts[mat["k"]], m=Mtok, n=mat["n"], k=mat["k"], d=out,
                                   b=Q.QuantizedB(codes=mat["codes"], scales=mat["scales"],
                                                  params=Q.QuantParams(Q.GROUP_OUTPUT, mat["n"], mat["k"] // GROUP),
                                                  correction_data=mat["biases"]))
                 for mat, out in zip(layer, outs)]
    batch = kern.prepare_many(args_list)
    ms = timed(torch, lambda i: kern.encode_prepared(batch, stream), args.steps, args.warmup, stream)
    ops = sum(2 * Mtok * n * k for _, n, k in SHAPES)
    tops = ops / (ms * 1e-3) / 1e12
    emit({"metric": "Qwen3-8B A8W4 prefill int8 GEMM TOP/s", "value": round(tops, 1), "unit": "TOP/s",
                      "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
                      "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
                      "data": "synthetic: N(0,0.02) weights W4 g64, N(0,1) activations RHT-quantized to int8 "
                              "(scale groups of 128)",
                      "config": {"workload": f"config 4 prefill, int8 activations: M={Mtok} through "
                                             "q,k,v,o,gate,up,down (one layer)",
                                 "ops_per_step": ops, "prefill_tokens_per_s_36_layers":
                                     round(Mtok * 1000.0 / (ms * LAYERS), 1)},
                      "roofline": {"bound": "mfma", "achieved": round(tops, 1), "peak": PEAK_MFMA_INT8_TOPS,
                                   "unit": "TOP/s", "frac": round(tops / PEAK_MFMA_INT8_TOPS, 4),
                                   "traffic": None}})


def decode_measure(args, torch):
    """Config 4 (decode part): random-init Qwen3-8B architecture (36 layers,
    32/8 heads of 128, intermediate 12288, vocab 151936; W4 g64 projections,
    W8 g64 lm_head, bf16 KV cache), a 4096-token context whose KV rows are
    synthetic N(0,1), then greedy tokens generated one HIP-graph replay each.
    Returns generated tokens per second over the timed tokens and the bytes."""
    from stark_amd import decode as DEC
    cfg = DEC.Qwen3Config()
    ctx, gen_tokens = 4096, args.decode_tokens
    m = DEC.Qwen3Decoder(cfg, capacity=ctx + gen_tokens + 8, seed=SEED + 40, chain=args.decode_form == "chain")
    m.fill_context(ctx, seed=SEED + 41)
    m.step()  # eager: builds the library's per-shape schedules
    torch.cuda.synchronize()
    graph = m.capture()
    # clocks up (as for the headline): 0.4 s of replays, the position put back
    # every 16 tokens so that the capacity holds
    start = int(m.pos.item())
    t_end = time.time() + 0.4
    while time.time() < t_end:
        for _ in range(16):
            graph.replay()
        m.pos.fill_(start)
        torch.cuda.synchronize()
    warm = 3
    for _ in range(warm):
        graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    timed_tokens = gen_tokens - 1 - warm
    a.record(stream)
    for _ in range(timed_tokens):
        graph.replay()
    b.record(stream)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / timed_tokens
    assert int(m.pos.item()) == ctx + gen_tokens, "device position did not advance once per token"
    tps = 1000.0 / ms
    H, hd = cfg.hidden, cfg.head_dim
    layer_bytes = algorithmic_bytes()
    lm_bytes = cfg.vocab * H * (1 + 4 / GROUP) + H * 2 + cfg.vocab * 4
    mid = ctx + gen_tokens // 2
    kv_bytes = cfg.layers * 2 * cfg.kv_heads * mid * hd * 2
    per_token = cfg.layers * layer_bytes + lm_bytes + kv_bytes + H * 2
    gbs = per_token * tps / 1e9
    del graph, m
    torch.cuda.empty_cache()
    return dict(tokens_per_s=round(tps, 1), ms_per_token=round(ms, 5), timed_tokens=timed_tokens,
                workload=f"config 4 decode: {gen_tokens} greedy tokens after a {ctx}-token context, 36 layers, "
                         "vocab 151936 (W8 lm_head), one HIP graph replay per token; RMS norms and gated SiLU run as "
                         "input prologues of the products"
                         + ("; per layer, o, gate/up, down and the next layer's q/k/v products run as one chained "
                            "launch" if args.decode_form == "chain" else ""),
                form=args.decode_form,
                hbm_bytes_per_token_algorithmic=per_token, achieved_gbs=round(gbs, 1),
                frac_of_hbm_peak=round(gbs / PEAK_HBM_GBS, 4))


def decode_line(args, torch):
    d = decode_measure(args, torch)
    gbs = d["achieved_gbs"]
    emit({"metric": "Qwen3-8B W4 end-to-end greedy decode tokens/s", "value": d["tokens_per_s"],
                      "unit": "tokens/s", "n_gpus": 1, "steps": d["timed_tokens"], "warmup": 4,
                      "ms_per_step": d["ms_per_token"], "higher_is_better": True, "scaling": "weak",
                      "vs_baseline": None, "dtype": "bf16",
                      "data": "synthetic: random-init weights (W4 g64, W8 g64 lm_head), KV of a 4096-token context "
                              "filled N(0,1), uniform random prompt token",
                      "config": {"workload": d["workload"],
                                 "hbm_bytes_per_token_algorithmic": d["hbm_bytes_per_token_algorithmic"]},
                      "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                   "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None}})


def attention_line(args, torch):
    """Diagnostic (--attention): the decode step's attention pair alone -- the
    fused q/k norm + RoPE + KV write + chunk partials launch and the chunk
    combine -- at the Qwen3-8B shape (32 query / 8 KV heads of 128) after a
    4096-token context, over 36 rotating layer caches (past the MALL), timed
    as replays of one captured graph. Bytes: the K and V rows read (the new
    position's included) plus the partials written and read back."""
    import ctypes as C
    from stark_amd import decode as DEC
    D = DEC.lib()
    qh, kvh, hd, ctx, layers = 32, 8, 128, 4096, LAYERS
    cap = ctx + 264
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED + 50)
    nch = D.stark_decode_attn_chunks(cap)
    caches = [((torch.randn(kvh * cap * hd, generator=gen, device="cuda")).to(torch.bfloat16),
               (torch.randn(kvh * cap * hd, generator=gen, device="cuda")).to(torch.bfloat16)) for _ in range(layers)]
    q = torch.randn(qh * hd, generator=gen, device="cuda").to(torch.bfloat16)
    k = torch.randn(kvh * hd, generator=gen, device="cuda").to(torch.bfloat16)
    v = torch.randn(kvh * hd, generator=gen, device="cuda").to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(hd, generator=gen, device="cuda")).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(hd, generator=gen, device="cuda")).to(torch.bfloat16)
    po = torch.empty(qh * nch * hd, dtype=torch.float32, device="cuda")
    pml = torch.empty(qh * nch * 2, dtype=torch.float32, device="cuda")
    out = torch.empty(qh * hd, dtype=torch.bfloat16, device="cuda")
    pos = torch.tensor([ctx], dtype=torch.int32, device="cuda")
    ptr = lambda t: C.c_void_p(t.data_ptr())

    def step(i, s):
        kc, vc = caches[i]
        st = D.stark_decode_attention_fused(ptr(q), ptr(k), ptr(v), ptr(qw), ptr(kw), ptr(kc), ptr(vc), ptr(po),
                                            ptr(pml), ptr(out), ptr(pos), qh, kvh, cap, 1e6, 1e-6,
                                            C.c_void_p(s.cuda_stream))
        if st != 0:
            raise SystemExit(f"attention: status {st}")

    ms, ran = graph_timed(torch, step, layers, args.steps)
    used = (ctx + 1 + 63) // 64
    nbytes = 2 * kvh * (ctx + 1) * hd * 2 + 2 * qh * used * (hd + 2) * 4 + qh * hd * 2 * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    emit({"metric": "decode attention pair (fused partials + combine) HBM GB/s", "value": round(gbs, 1),
                      "unit": "GB/s", "n_gpus": 1, "steps": ran, "warmup": layers, "ms_per_step": round(ms, 5),
                      "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
                      "data": "synthetic: N(0,1) K/V caches and q/k/v rows",
                      "config": {"workload": f"decode attention at position {ctx}: 32/8 heads of 128, "
                                             f"{layers} rotating layer caches, one captured HIP graph over them",
                                 "bytes_per_step": nbytes},
                      "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                   "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None}})


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default 360 for config 1, else 200)")
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--config", type=int, default=1, choices=(1, 2, 3, 4),
                    help="1: Qwen3-8B W4 layer set (headline); 2: 8-bit / Q8_0 / Q4_K; 3: Qwen3-30B-A3B MoE layer; "
                         "4: prefill dequant-GEMM at M=2048")
    ap.add_argument("--tokens", type=int, nargs="+", default=[1, 4, 16], help="config 3 tokens per step")
    ap.add_argument("--decode-tokens", type=int, default=256,
                    help="configs 1 and 4: greedy tokens generated after the 4096-token context in the end-to-end "
                         "decode measurement (0 skips it)")
    ap.add_argument("--decode-only", action="store_true", help="only the end-to-end decode line (config 4)")
    ap.add_argument("--headline-only", action="store_true",
                    help="config 1: print the headline line alone (the default run also measures verify M=2..256, "
                         "configs 2 and 3 and the config-4 prefill and attaches them as other_configs)")
    ap.add_argument("--decode-form", choices=("chain", "fused"), default="fused",
                    help="decode stand-in: products after attention as one chained launch per layer (chain) or one "
                         "launch per product with norm/SiLU prologues (fused)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--verify", action="store_true",
                    help="config 1: also print the M = 2, 4, 8, 16 (speculative verify) and M = 32, 64 (short prefill) lines")
    ap.add_argument("--copies", type=int, default=LAYERS,
                    help="config 1: distinct layer-weight copies the steps rotate through (36 = one Qwen3-8B)")
    ap.add_argument("--eager", action="store_true",
                    help="configs 2 and 3 and --attention: issue the calls one by one instead of graph replays "
                         "(for counter passes)")
    ap.add_argument("--attention", action="store_true",
                    help="diagnostic: time the decode attention pair alone (Qwen3-8B shape, 36 rotating caches)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a 256 MiB bitwise_not pass (byte-counter calibration under rocprofv3)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1).",
              file=sys.stderr)
        sys.exit(2)
    if args.steps is None:
        args.steps = {1: 360, 4: 20}.get(args.config, 200)
    if args.warmup is None:
        args.warmup = {1: 72, 4: 3}.get(args.config, 40)

    import torch
    from stark_amd import qmm as Q
    Q.lib()
    torch.cuda.set_device(torch.device("cuda:0"))
    global EAGER
    EAGER = args.eager
    if args.attention:
        attention_line(args, torch)
        return
    if args.decode_only:
        decode_line(args, torch)
        return
    {1: config1, 2: config2, 3: config3, 4: config4}[args.config](args, torch, Q)


if __name__ == "__main__":
    main()
