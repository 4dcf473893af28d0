"""Benchmark of the quantized matvec hot path on one MI355X.

Workload: the Qwen3-8B per-layer 4-bit decode matvec set
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


def quantize_gpu(w, group=GROUP):
    """BASELINE rule on the GPU (data generation only): per group
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


def cpu_baseline(torch, layer, xs, budget_s=12.0):
    """Single-thread oracle (MatmulCpuKernel restated) over whole layer-set
    passes until ~budget_s of CPU time; returns GB/s of algorithmic bytes."""
    import numpy as np
    from oracle import oracle as O
    O.lib()
    host = []
    for mat, x in zip(layer, xs):
        host.append(dict(n=mat["n"], k=mat["k"], codes=mat["codes"].cpu().numpy(),
                         s=mat["scales"].cpu().numpy().view(np.uint16), b=mat["biases"].cpu().numpy().view(np.uint16),
                         x=x.view(torch.int16).cpu().numpy().view(np.uint16)))
    passes, bytes_done, t0 = 0, 0, time.perf_counter()
    while True:
        for h in host:
            st, _ = O.matmul(a=h["x"], m=1, n=h["n"], k=h["k"], codes=h["codes"], scales=h["s"],
                             correction_data=h["b"], layout=O.GROUP_OUTPUT, bits=4, group_size=GROUP,
                             output_dt=O.BF16)
            assert st == 0
        passes += 1
        bytes_done += algorithmic_bytes(1)
        el = time.perf_counter() - t0
        if el >= budget_s or passes >= 50:
            break
    return dict(value=bytes_done / el / 1e9, unit="GB/s", cores=1, kind="port",
                sample=f"{passes} full passes over one Qwen3-8B W4 layer matvec set (M=1), single thread, "
                       f"oracle restatement of MatmulCpuKernel::encode, {el:.1f} s")


def copy_calibration(torch, mib=256):
    """A plain device pass of known size (reads `mib` MiB, writes `mib` MiB),
    run under rocprofv3 --pmc to scale FETCH_SIZE / WRITE_SIZE to bytes."""
    src = torch.full(((mib << 20) // 4,), 1, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        torch.bitwise_not(src, out=dst)
    torch.cuda.synchronize()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=360)
    ap.add_argument("--warmup", type=int, default=72)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a 256 MiB bitwise_not pass (byte-counter calibration under rocprofv3)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from stark_amd import qmm as Q
    Q.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
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
                           "biases": m["biases"].clone()} for m in layer0] for _ in range(LAYERS - 1)]
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

    for i in range(args.warmup):
        kern.encode_prepared(all_args[i % LAYERS], stream)
    torch.cuda.synchronize()

    # timed region: K steps between two events on the launch stream
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(args.steps):
        kern.encode_prepared(all_args[i % LAYERS], stream)
    stop.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(stop)

    # per-launch durations (events bracket each launch on the same stream)
    n_lat = min(args.steps, 180)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n_lat)]
    for i in range(n_lat):
        evs[i][0].record(stream)
        kern.encode_prepared(all_args[i % LAYERS], stream)
        evs[i][1].record(stream)
    torch.cuda.synchronize()
    launch_ms = sorted(a.elapsed_time(b) for a, b in evs)
    mean_launch_ms = sum(launch_ms) / len(launch_ms)

    bytes_step = algorithmic_bytes(1)
    ms_step = total_ms / args.steps
    value = bytes_step / (ms_step * 1e-3) / 1e9
    achieved = bytes_step / (mean_launch_ms * 1e-3) / 1e9
    traffic = None
    tfile = os.path.join(ROOT, "profiles", "qmv_w4_mfma_layerset_pmc.md")
    if os.path.exists(tfile):
        import re
        hit = re.search(r"hbm_bytes_per_launch\s*=\s*(\d+)", open(tfile).read())
        traffic = int(hit.group(1)) if hit else None

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
        "data": "synthetic: random-init N(0,0.02) weights quantized W4 g64 (BASELINE rule), bf16 N(0,1) activations",
        "config": {
            "workload": "Qwen3-8B layer matvec set q,k,v,o,gate,up,down; MLX-affine W4 g64 bf16 planes; M=1; "
                        "36 rotating layer copies; one stark_qmm_encode_many launch per step",
            "bytes_per_step": bytes_step,
            "pct_of_peak_hbm": round(100.0 * value / PEAK_HBM_GBS, 2),
            "matvec_decode_tokens_per_s_36_layers": round(1000.0 / (ms_step * LAYERS), 1),
            "launch_ms_median": round(launch_ms[len(launch_ms) // 2], 5),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "kernel": "qmv_w4_mfma<1,1,false,true,true> (one launch per step)",
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
