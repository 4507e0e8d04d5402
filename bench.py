#!/usr/bin/env python3
"""Benchmark: batch-1 packed GEMV over every matmul of the 2.2B shape.

Workload: 26 layers x 7 packed matmuls (q, k, v, o:
2560x2560; gate, up: 6912x2560; down: 2560x6912), 3-bit, 8 entries, block
128, random-init weights quantized as the reference does (per-block quantile
codebooks, nearest-entry indices), activations bf16 N(0,1), outputs fp32.
All 182 packed layers (1.29 GB) are resident in HBM, so every step streams
them from HBM (more than the 256 MB Infinity Cache).

A step is one decode token's worth of GEMVs, launched the way the decode step
launches them: per layer q|k|v as one GEMV over the three contiguous packed
matrices (they share x; the reference fuses qkv the same way,
inference/generate_torch.py:68), o, gate|up as one GEMV (shared x), down --
4 launches per layer, 104 per step, captured once in a HIP graph and
replayed.  The JSON line reports total algorithmic bytes / step time.

Usage: python bench.py [--steps K] [--warmup W] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "packed GEMV GB/s (% HBM peak) + decode tok/s, 2.2B-shape 3-bit, batch 1"
HBM_PEAK_GBS = 8000.0
NE, BS, BITS = 8, 128, 3


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--layers", type=int, default=26)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-breakdown", action="store_true")
    p.add_argument("--cpu-reps", type=int, default=3)
    return p.parse_args()


class Launch:
    """One nb_gemv call with its buffers and algorithmic byte count."""

    def __init__(self, name, layers, x, y, packed, cb, N, K):
        from nativebit_amd import _lib, synth
        self.name, self.N, self.K = name, N, K
        self.x, self.y, self.packed, self.cb = x, y, packed, cb
        self.bytes = sum(synth.layer_bytes(l.out_features, l.in_features, NE, BS, 1, 0, 0)
                         for l in layers) + K * 2 + N * 4
        self.args = (x.data_ptr(), _lib.NB_BF16, K, packed.data_ptr(), cb.data_ptr(),
                     y.data_ptr(), _lib.NB_F32, N, 1, N, K, BITS, NE, BS)


def build_step(dev, n_layers):
    """Generates the 26x7 layers on the GPU and groups them per decode launch."""
    from nativebit_amd import synth
    launches = []
    t0 = time.time()
    for l in range(n_layers):
        mats = {name: synth.make_layer(N, K, NE, BS, seed=l * 7 + j, device=dev)
                for j, (name, N, K) in enumerate(synth.LAYER_SHAPES)}
        for gname, members in (("qkv", ("q", "k", "v")), ("o", ("o",)),
                               ("gateup", ("gate", "up")), ("down", ("down",))):
            lays = [mats[m] for m in members]
            K = lays[0].in_features
            N = sum(m.out_features for m in lays)
            # rows never share a block (K % BS == 0): the concatenated streams
            # and codebooks are byte-identical to one (N x K) packed layer.
            packed = torch.cat([m.packed for m in lays]) if len(lays) > 1 else lays[0].packed
            cb = torch.cat([m.codebook for m in lays]) if len(lays) > 1 else lays[0].codebook
            x = synth.make_activation(K, seed=10_000 + l * 7 + len(launches) % 4, device=dev,
                                      dtype=torch.bfloat16)[0].contiguous()
            y = torch.empty(N, dtype=torch.float32, device=dev)
            launches.append(Launch(gname, lays, x, y, packed.contiguous(), cb.contiguous(), N, K))
        del mats
    torch.cuda.synchronize()
    log(f"[bench] generated {n_layers} layers x 7 packed matmuls on {dev} in {time.time()-t0:.1f}s")
    return launches


def run_launches(lib, launches):
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for a in launches:
        rc = lib.nb_gemv(*a.args, s)
        if rc:
            from nativebit_amd import _lib
            _lib.check(rc)


def time_graph(lib, launches, steps, warmup):
    """Captures one pass over `launches` in a HIP graph; ms per replay."""
    run_launches(lib, launches)          # eager warm-up (first-call setup)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run_launches(lib, launches)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps, g


def check_outputs(launches, n=2):
    """Spot-checks the first launches' outputs against the fp64 oracle."""
    import numpy as np
    from oracle import oracle as O
    worst = 0.0
    for a in launches[:n]:
        idx = O.unpack(a.packed.cpu().numpy(), a.N * a.K, BITS)
        w = O.dequant(idx, a.cb.cpu().numpy(), BS, a.N * a.K).reshape(a.N, a.K)
        ref = O.matmul_f64(a.x.float().cpu().numpy(), w)[0]
        y = a.y.cpu().numpy()
        worst = max(worst, float(np.linalg.norm(y - ref) / np.linalg.norm(ref)))
    return worst


def cpu_baseline(launches, reps):
    """The reference CPU path (unpack + gather + F.linear, restated in
    oracle.torch_packed_linear_f32) on layer 0's four launches (7 matmuls)."""
    from oracle import oracle as O
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    torch.set_num_threads(threads)
    sample = launches[:4]
    host = [(a.x.float().cpu(), a.packed.cpu(), a.cb.cpu(), a.N, a.K) for a in sample]
    nbytes = sum(a.bytes for a in sample)

    def once():
        for x, p, cb, N, K in host:
            O.torch_packed_linear_f32(x, p, cb, N, K, BS, BITS)

    once()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        once()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            cpu_model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    return {
        "value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": (f"layer 0 of config 1 (q|k|v, o, gate|up, down = 7 matmuls, {nbytes} B): "
                   f"torch CPU unpack+gather+F.linear (reference triton_kernel.py:258-275), "
                   f"x bf16 upcast to fp32, median of {reps} after 1 warm-up, {t*1e3:.1f} ms; "
                   f"{threads} threads on {cpu_model or platform.processor()}"),
        "seconds_per_sample": round(t, 4),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build's "
              "packed GEMV path is single-GPU by design -- run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a gfx950 GPU", file=sys.stderr)
        sys.exit(1)
    from nativebit_amd import _lib
    lib = _lib.load()
    dev = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(dev)
    log(f"[bench] {torch.cuda.get_device_name(dev)} {props.gcnArchName} CUs={props.multi_processor_count}")

    launches = build_step(dev, args.layers)
    step_bytes = sum(a.bytes for a in launches)
    ms, _ = time_graph(lib, launches, args.steps, args.warmup)
    gbs = step_bytes / (ms * 1e-3) / 1e9
    err = check_outputs(launches)
    log(f"[bench] decode schedule: {len(launches)} launches/step, {step_bytes} B/step, "
        f"{ms*1e3:.1f} us/step, {gbs:.1f} GB/s ({100*gbs/HBM_PEAK_GBS:.1f}% of 8 TB/s), "
        f"spot-check rel err {err:.2e}")

    extra = {}
    if not args.no_breakdown:
        breakdown = {}
        for gname in ("qkv", "o", "gateup", "down"):
            sub = [a for a in launches if a.name == gname]
            sms, _ = time_graph(lib, sub, max(10, args.steps // 2), 3)
            sb = sum(a.bytes for a in sub)
            breakdown[gname] = {"N": sub[0].N, "K": sub[0].K, "launches": len(sub),
                                "us_per_launch": round(sms * 1e3 / len(sub), 3),
                                "GB_s": round(sb / (sms * 1e-3) / 1e9, 1)}
            log(f"[bench]   {gname:6s} {sub[0].N}x{sub[0].K}: {sms*1e3/len(sub):.2f} us/launch, "
                f"{breakdown[gname]['GB_s']:.1f} GB/s")
        extra["breakdown"] = breakdown
        # eager (no graph) for reference: includes host launch overhead
        run_launches(lib, launches)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(5):
            run_launches(lib, launches)
        torch.cuda.synchronize()
        extra["eager_us_per_step"] = round((time.perf_counter() - t0) / 5 * 1e6, 1)

    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": ("config1: 2.2B-shape decode-step GEMVs, 26 layers x (q,k,v,o 2560x2560; "
                         "gate,up 6912x2560; down 2560x6912), 3-bit NE 8 BS 128, batch 1, "
                         "x bf16 N(0,1), y fp32, weights fp32 codebook values"),
            "schedule": "per layer: qkv, o, gate|up, down (104 launches/step, HIP graph)",
            "layers": args.layers,
            "bytes_per_step": step_bytes,
            "tokens_per_s_gemv_only": round(1e3 / ms, 1),
            "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "gemv_fast_kernel<3,128,bf16x>",
            "method": "algorithmic bytes of all launches in the timed region / HIP-event time "
                      "of the graph replays on the launch stream",
        },
        "parity": {"spot_check_rel_err_vs_f64": err},
    }
    result.update(extra)
    if not args.no_cpu_baseline:
        log("[bench] timing CPU baseline ...")
        result["cpu_baseline"] = cpu_baseline(launches, args.cpu_reps)
        log(f"[bench] cpu baseline {result['cpu_baseline']['value']} GB/s "
            f"({result['cpu_baseline']['cores']} threads)")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
