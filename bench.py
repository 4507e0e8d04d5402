#!/usr/bin/env python3
"""Benchmark: batch-1 packed GEMV over every matmul of the 2.2B shape.

Workload: 26 layers x 7 packed matmuls (q, k, v, o:
2560x2560; gate, up: 6912x2560; down: 2560x6912), 3-bit, 8 entries, block
128, random-init weights quantized as the reference does (per-block quantile
codebooks, nearest-entry indices), activations bf16 N(0,1) (one independent
x per matmul, as config 1 defines), outputs fp32.  All 182 packed layers
(1.29 GB) stay resident in HBM -- more than the 256 MB Infinity Cache -- so
every step streams them from HBM.

A step is one token's 182 GEMVs.  Three launch schedules are timed over the
same buffers, each captured once in a HIP graph and replayed:

  batched   all 182 GEMVs in one persistent launch (nb_gemv_batched)  <- value
  per_layer one batched launch per layer (26 launches)
  decode    the launches a decode step makes: q|k|v, o, gate|up, down per
            layer (104 nb_gemv launches; q|k|v and gate|up share x)

`value` is the batched schedule: algorithmic bytes per step / HIP-event time
per replay.  The other two are reported beside it.

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
    p = argparse.ArgumentParser(description=__doc__,
                                formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=500)
    p.add_argument("--warmup", type=int, default=500)
    p.add_argument("--layers", type=int, default=26)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--schedules", default="batched,per_layer,decode",
                   help="comma list of schedules to time (batched is the reported value)")
    p.add_argument("--cpu-reps", type=int, default=3, help="minimum CPU baseline passes")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="CPU baseline passes continue until this much time has been spent")
    p.add_argument("--copy-calibration", action="store_true",
                   help="also time a plain 1 GiB device copy (the yardstick that scales "
                        "rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes)")
    return p.parse_args()


class Mat:
    """One packed matmul of the model with its own x and y."""

    def __init__(self, name, N, K, packed, cb, x, y):
        from nativebit_amd import synth
        self.name, self.N, self.K = name, N, K
        self.packed, self.cb, self.x, self.y = packed, cb, x, y
        self.bytes = synth.layer_bytes(N, K, NE, BS, 1, x_bytes=2, y_bytes=4)


def build_model(dev, n_layers):
    """182 packed layers generated on the GPU.  q|k|v and gate|up of a layer
    live in one buffer each (rows never share a block when K % 128 == 0, so
    the concatenation is byte-identical to one fused packed layer, as the
    reference fuses qkv, inference/generate_torch.py:68); the individual
    matrices are views into it."""
    from nativebit_amd import synth
    layers = []
    t0 = time.time()
    for l in range(n_layers):
        gen = {name: synth.make_layer(N, K, NE, BS, seed=l * 7 + j, device=dev)
               for j, (name, N, K) in enumerate(synth.LAYER_SHAPES)}
        mats = {}
        for group in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",)):
            packed = torch.cat([gen[m].packed for m in group]).contiguous()
            cb = torch.cat([gen[m].codebook for m in group]).contiguous()
            po = co = 0
            for m in group:
                g = gen[m]
                pn, cn = g.packed.numel(), g.codebook.shape[0]
                j = [s[0] for s in synth.LAYER_SHAPES].index(m)
                x = synth.make_activation(g.in_features, seed=100_000 + l * 7 + j, device=dev,
                                          dtype=torch.bfloat16)[0].contiguous()
                y = torch.empty(g.out_features, dtype=torch.float32, device=dev)
                mats[m] = Mat(m, g.out_features, g.in_features, packed[po:po + pn],
                              cb[co:co + cn], x, y)
                po += pn
                co += cn
            mats["_" + "".join(group)] = (packed, cb)
        layers.append(mats)
        del gen
    torch.cuda.synchronize()
    log(f"[bench] generated {n_layers} layers x 7 packed matmuls on {dev} in {time.time()-t0:.1f}s")
    return layers


def graph_time(run, steps, warmup):
    """Captures run() once in a HIP graph; returns ms per replay."""
    run()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def copy_calibration(dev, steps, warmup):
    """A plain device copy of 1 GiB (torch's copy kernel), timed like the
    GEMV.  Its known byte counts (1 GiB read, 1 GiB written) are the scale for
    the FETCH_SIZE / WRITE_SIZE counters read in the same profiled process."""
    n = 2**30 // 4
    src = torch.randn(n, device=dev)
    dst = torch.empty_like(src)
    ms = graph_time(lambda: dst.copy_(src), max(5, steps // 20), max(2, warmup // 20))
    out = {"bytes_read": 2**30, "bytes_written": 2**30, "us": round(ms * 1e3, 2),
           "GB_s": round(2 * 2**30 / ms / 1e6, 1)}
    del src, dst
    return out


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter
    summary (profiles/traffic_<kernel>_config1.txt, key `traffic_bytes`), or
    None when no such summary exists."""
    path = os.path.join(ROOT, "profiles", f"traffic_{kernel}_config1.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def decode_launches(layers):
    """(x, packed, cb, y, N, K) of the 104 decode-step launches."""
    out = []
    for mats in layers:
        qkv_p, qkv_c = mats["_qkv"]
        gu_p, gu_c = mats["_gateup"]
        dev = qkv_p.device
        if "_y_qkv" not in mats:
            mats["_y_qkv"] = torch.empty(7680, dtype=torch.float32, device=dev)
            mats["_y_gu"] = torch.empty(13824, dtype=torch.float32, device=dev)
        out.append((mats["q"].x, qkv_p, qkv_c, mats["_y_qkv"], 7680, 2560))
        o = mats["o"]
        out.append((o.x, o.packed, o.cb, o.y, o.N, o.K))
        out.append((mats["gate"].x, gu_p, gu_c, mats["_y_gu"], 13824, 2560))
        d = mats["down"]
        out.append((d.x, d.packed, d.cb, d.y, d.N, d.K))
    return out


def spot_check(mats):
    """fp64 brute force (bf16-rounded weights, bf16 x) for a few matmuls."""
    import numpy as np
    from oracle import oracle as O
    worst = 0.0
    for m in mats:
        idx = O.unpack(m.packed.cpu().numpy(), m.N * m.K, BITS)
        w = O.dequant(idx, m.cb.cpu().numpy(), BS, m.N * m.K).reshape(m.N, m.K)
        w = torch.from_numpy(w).to(torch.bfloat16).float().numpy()
        ref = O.matmul_f64(m.x.float().cpu().numpy(), w)[0]
        y = m.y.cpu().numpy()
        worst = max(worst, float(np.linalg.norm(y - ref) / np.linalg.norm(ref)))
    return worst


def cpu_baseline(mats, reps, seconds):
    """The reference CPU path (unpack + gather + F.linear, restated in
    oracle.torch_packed_linear_f32) on layer 0's 7 matmuls."""
    from oracle import oracle as O
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    torch.set_num_threads(threads)
    host = [(m.x.float().cpu(), m.packed.cpu(), m.cb.cpu(), m.N, m.K) for m in mats]
    nbytes = sum(m.bytes for m in mats)

    def once():
        for x, p, cb, N, K in host:
            O.torch_packed_linear_f32(x, p, cb, N, K, BS, BITS)

    once()
    times = []
    t_start = time.perf_counter()
    while len(times) < reps or time.perf_counter() - t_start < seconds:
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
        "sample": (f"layer 0 of config 1 (q, k, v, o, gate, up, down; {nbytes} B): torch CPU "
                   f"unpack+gather+F.linear (reference triton_kernel.py:258-275), x bf16 upcast "
                   f"to fp32, median of {len(times)} passes ({sum(times):.1f} s) after 1 warm-up "
                   f"= {t*1e3:.1f} ms per pass; {threads} "
                   f"threads on {cpu_model or platform.processor()}"),
        "seconds_per_sample": round(t, 4),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): the packed GEMV path "
              "is built and measured on a single MI355X -- run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a gfx950 GPU", file=sys.stderr)
        sys.exit(1)
    from nativebit_amd import _lib, ops, synth
    lib = _lib.load()
    dev = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(dev)
    log(f"[bench] {torch.cuda.get_device_name(dev)} {props.gcnArchName} "
        f"CUs={props.multi_processor_count}")

    layers = build_model(dev, args.layers)
    all_mats = [mats[name] for mats in layers for name, _, _ in synth.LAYER_SHAPES]
    step_bytes = sum(m.bytes for m in all_mats)
    wanted = args.schedules.split(",")
    results = {}

    batch = ops.GemvBatch([(m.x, m.packed, m.cb, m.y, m.N, m.K) for m in all_mats])
    ms = graph_time(batch.run, args.steps, args.warmup)
    err = spot_check(all_mats[:7])
    results["batched"] = {"launches": 1, "us_per_step": round(ms * 1e3, 2),
                          "GB_s": round(step_bytes / ms / 1e6, 1)}
    log(f"[bench] batched  : 1 launch/step, {step_bytes} B, {ms*1e3:.1f} us/step, "
        f"{step_bytes/ms/1e6:.1f} GB/s ({step_bytes/ms/1e6/HBM_PEAK_GBS*100:.1f}% of 8 TB/s), "
        f"spot-check rel err {err:.2e}")

    if "per_layer" in wanted:
        per = [ops.GemvBatch([(mats[n].x, mats[n].packed, mats[n].cb, mats[n].y,
                               mats[n].N, mats[n].K) for n in ("q", "k", "v", "o", "gate", "up",
                                                               "down")]) for mats in layers]

        def run_per():
            for b in per:
                b.run()
        pms = graph_time(run_per, max(10, args.steps // 2), args.warmup)
        results["per_layer"] = {"launches": len(per), "us_per_step": round(pms * 1e3, 2),
                                "GB_s": round(step_bytes / pms / 1e6, 1)}
        log(f"[bench] per_layer: {len(per)} launches/step, {pms*1e3:.1f} us/step, "
            f"{step_bytes/pms/1e6:.1f} GB/s")

    if "decode" in wanted:
        dl = decode_launches(layers)
        dec_bytes = sum(synth.layer_bytes(N, K, NE, BS, 1, 2, 4) for (_, _, _, _, N, K) in dl)
        args_c = [(x.data_ptr(), _lib.NB_BF16, K, p.data_ptr(), c.data_ptr(), y.data_ptr(),
                   _lib.NB_F32, N, 1, N, K, BITS, NE, BS) for (x, p, c, y, N, K) in dl]

        def run_dec():
            s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for a in args_c:
                rc = lib.nb_gemv(*a, s)
                if rc:
                    _lib.check(rc)
        dms = graph_time(run_dec, max(10, args.steps // 2), args.warmup)
        results["decode"] = {"launches": len(dl), "us_per_step": round(dms * 1e3, 2),
                             "GB_s": round(dec_bytes / dms / 1e6, 1), "bytes_per_step": dec_bytes}
        log(f"[bench] decode   : {len(dl)} launches/step, {dms*1e3:.1f} us/step, "
            f"{dec_bytes/dms/1e6:.1f} GB/s")

    gbs = step_bytes / ms / 1e6
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
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": ("config1: 2.2B-shape GEMVs of one token, 26 layers x (q,k,v,o 2560x2560; "
                         "gate,up 6912x2560; down 2560x6912), 3-bit NE 8 BS 128, batch 1, "
                         "x bf16 N(0,1) per matmul, y fp32, bf16 weights, fp32 accumulation"),
            "schedule": "batched: all 182 GEMVs in one persistent launch (HIP graph replay)",
            "layers": args.layers,
            "bytes_per_step": step_bytes,
            "gemv_steps_per_s": round(1e3 / ms, 1),
            "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic("gemv_stream_kernel"),
            "kernel": "gemv_stream_kernel",
            "method": ("algorithmic bytes per launch (0.625 B/weight + x + y) / HIP-event time "
                       "per graph replay of the single launch, on the launch stream"),
        },
        "schedules": results,
        "parity": {"spot_check_rel_err_vs_f64": err},
    }
    if args.copy_calibration:
        result["copy_calibration"] = copy_calibration(dev, args.steps, args.warmup)
        log(f"[bench] copy calibration: {result['copy_calibration']}")
    if not args.no_cpu_baseline:
        log("[bench] timing CPU baseline ...")
        result["cpu_baseline"] = cpu_baseline([layers[0][n] for n in
                                               ("q", "k", "v", "o", "gate", "up", "down")],
                                              args.cpu_reps, args.cpu_seconds)
        log(f"[bench] cpu baseline {result['cpu_baseline']['value']} GB/s "
            f"({result['cpu_baseline']['cores']} threads)")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
