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

  batched   all 182 GEMVs in one persistent launch (nb_gemv_batched_sel on
            the streams in the selector-ordered unit layout, made once by
            nb_stream_layout outside the timing, as at model load: the same
            bytes, bit-identical products)                             <- value
  per_layer one batched launch per layer (26 launches)
  decode    the launches a decode step makes: q|k|v, o, gate|up, down per
            layer (104 nb_gemv launches; q|k|v and gate|up share x)

`value` is the batched schedule: algorithmic bytes per step / HIP-event time
per replay.  The other two are reported beside it, and the batched launch
on the reference's own stream layout (nb_gemv_batched) as
batched_original_layout.  The other BASELINE
configurations are reported in the same JSON line under "configs":

  config0  config 0: one 6912x2560 layer, x fp32 (the reference's exact fp32
           arithmetic), one nb_gemv launch per matvec over rotated copies,
           beside the reference CPU torch path on the same layer

  decode   config 4b: random-init 2.2B packed model (vocab 32000), greedy,
           128 prompt + 256 generated tokens, tokens/s of the generation
           (nativebit_amd.decode: one HIP graph per token)
  prefill  config 4a: nb_gemm_prefill on one layer's matmuls at M = 512 and
           2048 tokens, TFLOP/s and fraction of the 2.5 PFLOP/s bf16 MFMA
           peak, beside torch's dense bf16 matmul of an unpacked weight
  skinny   config 2: M = 1, 2, 4, 8, 16 activation rows over all 182 matmuls,
           one batched launch per step (M = 1 on the selector-ordered unit
           layout, M = 2 on the row-quad layout, M > 2 on the tile
           layout, each beside the same launch on the original layout),
           and 182 per-matmul nb_gemv launches
  quantize nb_quantize_pack: nearest-entry quantization straight into the
           3-bit stream for one 6912x2560 layer (GB/s), beside the
           reference's distance-tensor formulation on the GPU
  sweep    config 3: nb_gemv at batch 1, NE in {4, 8, 16} x BS in {64, 128,
           256} on 6912x2560 and 2560x6912 (random indices and codebooks;
           copies rotated over > 512 MB so no cache holds them)

Usage: python bench.py [--steps K] [--warmup W] [--no-cpu-baseline]
                       [--no-extra] [--extra config0,decode,prefill,skinny,sweep,quantize]
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
    p.add_argument("--no-extra", action="store_true",
                   help="skip the decode / prefill / skinny / sweep configurations")
    p.add_argument("--extra", default="config0,decode,prefill,skinny,sweep,quantize,codec",
                   help="comma list of extra configurations to run")
    p.add_argument("--decode-tokens", type=int, default=256,
                   help="tokens generated after the 128-token prompt in the decode leg")
    p.add_argument("--random-weights", action="store_true",
                   help="uniformly random index bytes and codebooks instead of quantized "
                        "N(0, 0.02) weights (same kernels and bytes; for profiled runs, where "
                        "the quantile/argmin generator's many small launches are slow)")
    p.add_argument("--skinny-m", default="1,2,4,8,16",
                   help="activation rows of the skinny configuration (comma list)")
    p.add_argument("--no-per-matmul", action="store_true",
                   help="skip the skinny configuration's one-launch-per-matmul comparison "
                        "(182 launches a step; slow under counter collection)")
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


def _make(random_weights):
    from nativebit_amd import synth
    return synth.make_random_layer if random_weights else synth.make_layer


def build_model(dev, n_layers, random_weights=False):
    """182 packed layers generated on the GPU.  q|k|v and gate|up of a layer
    live in one buffer each (rows never share a block when K % 128 == 0, so
    the concatenation is byte-identical to one fused packed layer, as the
    reference fuses qkv, inference/generate_torch.py:68); the individual
    matrices are views into it."""
    from nativebit_amd import synth
    layers = []
    t0 = time.time()
    for l in range(n_layers):
        gen = {name: _make(random_weights)(N, K, NE, BS, seed=l * 7 + j, device=dev)
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


# GPU time spent running the timed work back to back, untimed, before its
# warm-up steps.  On MI355X a memory-bound load that starts on an idle GPU
# runs its first ~1 ms at full clocks, then the power controller
# over-corrects for ~20 ms (the same launch takes up to 1.45x as long), then
# settles; an idle gap of a millisecond starts the cycle over.  Timing a few
# replays right after the warm-up would measure that transient, not the
# kernel, so every timed region here starts after this much continuous work
# (the transient itself is reported beside the headline number).
SETTLE_S = 0.15


def _settle(fn, seconds=SETTLE_S, cap=20000):
    """Runs fn() back to back for about `seconds` of GPU time (the count
    from one timed call), without host synchronisation in between."""
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    fn()
    e.record()
    torch.cuda.synchronize()
    per_ms = max(s.elapsed_time(e), 1e-3)
    n = int(min(cap, max(1, seconds * 1e3 / per_ms)))
    for _ in range(n):
        fn()
    return n + 1


def graph_time(run, steps, warmup, settle_s=SETTLE_S, info=None):
    """Captures run() once in a HIP graph; returns ms per replay over
    `steps` timed replays, after `settle_s` seconds of untimed replays and
    `warmup` untimed replays (see SETTLE_S).

    One step per replay, not many steps captured back to back: the
    headline kernel streams HBM at the power limit, and without the few
    microseconds between replays the same launches run ~7 % slower (a
    20-launch chain measured 217.8 us per step against 210.4)."""
    run()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    n_settle = _settle(g.replay, settle_s) if settle_s > 0 else 0
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    if info is not None:
        info["settle_replays"] = n_settle
        info["graph"] = g
    return start.elapsed_time(end) / steps


def transient_profile(g, idle_s=0.05, n=40):
    """Per-replay times (us) of graph g replayed n times after the GPU has
    idled for idle_s: the power controller's transient that SETTLE_S
    keeps out of the timed regions."""
    torch.cuda.synchronize()
    time.sleep(idle_s)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    ev[0].record()
    for i in range(n):
        g.replay()
        ev[i + 1].record()
    torch.cuda.synchronize()
    return [round(ev[i].elapsed_time(ev[i + 1]) * 1e3, 1) for i in range(n)]


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


def host_cpu():
    """The host's CPU resources as this process sees them: the CPUs in its
    affinity mask, the cgroup CPU quota (cpu.max), the physical cores behind
    the affinity CPUs and the CPU model.  ``threads`` = the affinity count,
    capped by the quota when one is set (more threads than the quota only
    time-slice)."""
    aff = sorted(os.sched_getaffinity(0))
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()[:2]
            if q != "max":
                quota = max(1, int(int(q) // int(period)))
    except (OSError, ValueError):
        pass
    model, cores, cur = "", set(), {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "processor":
                    cur = {"cpu": int(v)}
                elif k in ("physical id", "core id"):
                    cur[k] = v
                elif k == "model name":
                    model = model or v
                if "core id" in cur and cur.get("cpu") in aff:
                    cores.add((cur.get("physical id"), cur["core id"]))
    except OSError:
        pass
    threads = min(len(aff), quota) if quota else len(aff)
    return {"threads": threads, "affinity_cpus": len(aff), "cgroup_quota_cpus": quota,
            "physical_cores": len(cores) or None, "model": model or platform.processor()}


def _host_desc(h):
    q = f", cgroup quota {h['cgroup_quota_cpus']} CPUs" if h["cgroup_quota_cpus"] else ""
    return (f"{h['threads']} threads ({h['affinity_cpus']} CPUs in the affinity mask{q}, "
            f"{h['physical_cores']} physical cores) of {h['model']}")


def cpu_baseline(mats, reps, seconds):
    """The reference CPU path (unpack + gather + F.linear, restated in
    oracle.torch_packed_linear_f32) on layer 0's 7 matmuls."""
    from oracle import oracle as O
    h = host_cpu()
    torch.set_num_threads(h["threads"])
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
    dec = cpu_decode_sample(t, seconds=min(6.0, seconds / 2))
    return {
        "value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": h["threads"], "kind": "port",
        "sample": (f"layer 0 of config 1 (q, k, v, o, gate, up, down; {nbytes} B): torch CPU "
                   f"unpack+gather+F.linear (reference triton_kernel.py:258-275), x bf16 upcast "
                   f"to fp32, median of {len(times)} passes ({sum(times):.1f} s) after 1 warm-up "
                   f"= {t*1e3:.1f} ms per pass; {_host_desc(h)}"),
        "seconds_per_sample": round(t, 4),
        "host": h,
        "decode_tokens_per_s": dec["tokens_per_s"],
        "decode_sample": dec["sample"],
    }


def cpu_decode_sample(t_layer_linears, seconds=6.0, pos=256):
    """Config 4b's greedy decode on the CPU, layer-bounded: one token's cost
    = 26 x (the packed linears of one layer, timed above by cpu_baseline,
    + that layer's two RMSNorms and its attention over `pos` cached
    positions) + the final norm, the tied fp32 head 30 tanh(l / 30) over
    32000 rows and the argmax -- the reference's CPU module path
    (generate_torch.py:29-162, 298-313) with its fallback packed linear
    (triton_kernel.py:258-275), timed piece by piece on this host."""
    C, H, D, V, L = 2560, 20, 128, 32000, 26
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 1, C, generator=g)
    w = torch.ones(C)
    q = torch.randn(1, H, 1, D, generator=g)
    kc = torch.randn(1, H, pos + 1, D, generator=g)
    vc = torch.randn(1, H, pos + 1, D, generator=g)
    emb = torch.randn(V, C, generator=g) * 0.02

    def norm(v):
        return v / torch.sqrt(v.pow(2).mean(-1, keepdim=True) + 1e-6) * w

    def layer_rest():
        norm(x)
        norm(x)
        att = (q * D ** -0.5) @ kc.transpose(-1, -2)
        (torch.softmax(att, dim=-1) @ vc).transpose(1, 2).reshape(1, 1, C)

    def head():
        logits = 30.0 * torch.tanh((norm(x) @ emb.t()) / 30.0)
        return int(logits[0, -1].argmax())

    def timed(fn, budget):
        fn()
        ts, t_start = [], time.perf_counter()
        while len(ts) < 5 or time.perf_counter() - t_start < budget:
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts), len(ts)

    t_rest, n_rest = timed(layer_rest, seconds / 3)
    t_head, n_head = timed(head, seconds / 3)
    t_tok = L * (t_layer_linears + t_rest) + t_head
    return {
        "tokens_per_s": round(1.0 / t_tok, 3),
        "sample": (f"{L} x (one layer's packed linears {t_layer_linears*1e3:.1f} ms + its norms and "
                   f"attention over {pos} positions {t_rest*1e3:.2f} ms, median of {n_rest}) + "
                   f"final norm, tied fp32 head over {V} rows and argmax {t_head*1e3:.1f} ms "
                   f"(median of {n_head}) = {t_tok*1e3:.0f} ms per token"),
    }


def event_time(fn, reps, warmup=3, settle_s=SETTLE_S):
    """ms per call of fn() on the current stream (HIP events), after
    settle_s seconds of untimed calls (see SETTLE_S) and `warmup` more."""
    if settle_s > 0:
        _settle(fn, settle_s, cap=2000)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps


def graph_calls_time(fn, calls=10, reps=10, settle_s=SETTLE_S):
    """ms per call of fn() with `calls` calls captured back to back in one
    HIP graph, replayed `reps` times (after settle_s seconds of untimed
    replays): GPU time per call including the launch gaps inside a graph,
    without the host's per-call Python and ctypes cost."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(calls):
            fn()
    if settle_s > 0:
        _settle(g.replay, settle_s, cap=2000)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        g.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / (calls * reps)


def bench_decode(dev, n_gen=256):
    """Config 4b: greedy decode tokens/s of a random-init 2.2B packed model
    (one HIP graph of launches replayed per token)."""
    from nativebit_amd.decode import DecodeEngine
    from nativebit_amd.model import ModelConfig, random_packed_model
    cfg = ModelConfig(vocab_size=32000)
    t0 = time.time()
    model = random_packed_model(cfg, seed=0, device=dev)
    eng = DecodeEngine(model, max_steps=128 + max(n_gen, 2))
    gen = torch.Generator().manual_seed(2024)
    prompt = torch.randint(0, cfg.vocab_size, (128,), generator=gen).tolist()
    n_gen = max(n_gen, 2)
    r = eng.benchmark(prompt, n_gen, n_runs=3)
    out = {"tokens_per_s": round(r["generate_tps"], 1), "ms_per_token": round(r["per_token_ms"], 4),
           "prompt_ms": round(r["prompt_ms"], 3), "prompt_tokens_per_s": round(r["prompt_tps"], 1),
           "prompt_tokens": 128, "generated_tokens": n_gen, "vocab": cfg.vocab_size,
           "runs": r["runs"], "model_build_s": round(time.time() - t0, 1),
           "engine": "DecodeEngine: the prompt as one batched pass (packed MFMA GEMMs over the "
                     "128 rows, row kernels for norms / RoPE / causal attention; its launches "
                     "captured in a HIP graph once per prompt length, in the first run, and "
                     "replayed), then one HIP graph of the step's launches replayed per token",
           "method": "median of 3 runs; each: the prompt pass timed on its own (prompt_ms, "
                     f"which also chooses the first generated token), then {n_gen - 1} graph "
                     "replays timed (tokens_per_s)"}
    del eng, model
    torch.cuda.empty_cache()
    return out


PREFILL_SHAPES = (("qkv", 7680, 2560), ("o", 2560, 2560), ("gate|up", 13824, 2560),
                  ("down", 2560, 6912))


def bench_prefill(dev, random_weights=False):
    """Config 4a: prefill-sized contraction with the packed weights.

    The value is nb_gemm_prefill_split (ops.gemm_prefill's default): the
    hand-written MFMA kernels that dequantize the 3-bit stream into LDS
    tiles, split over K ranges where one launch's tile grid would leave CUs
    idle; beside it the one-launch kernel (nb_gemm_prefill) and, for
    comparison only, the reference's order of work on the GPU (the weight
    expanded to bf16 by the format kernel, then torch's dense bf16 matmul,
    i.e. hipBLASLt) and torch's dense bf16 matmul of an already-unpacked
    weight."""
    from nativebit_amd import _lib, ops, synth
    layers = {n: _make(random_weights)(N, K, seed=50 + i, device=dev)
              for i, (n, N, K) in enumerate(PREFILL_SHAPES)}
    out = {}
    for M in (512, 2048):
        xs = {K: synth.make_activation(K, m=M, seed=M + K, device=dev, dtype=torch.bfloat16)
              for K in (2560, 6912)}
        per, tot_ms, tot_fl, ref_ms, blas_ms = {}, 0.0, 0, 0.0, 0.0
        f32_ms, f32_ref_ms = 0.0, 0.0
        wx = {}
        xf = {K: v.float() for K, v in xs.items()}
        for n, N, K in PREFILL_SHAPES:
            lay = layers[n]
            y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
            w = torch.empty(N, K, dtype=torch.bfloat16, device=dev).normal_()
            wx[n] = torch.empty(N * K, dtype=torch.bfloat16, device=dev)

            def expanded(lay=lay, N=N, K=K, wb=wx[n]):
                ops.dequant(lay.packed, lay.codebook, N * K, 3, 128, torch.bfloat16, out=wb)
                torch.matmul(xs[K], wb.view(N, K).T, out=y)

            yf = torch.empty(M, N, dtype=torch.float32, device=dev)
            wf = torch.empty(N * K, dtype=torch.float32, device=dev)

            def f32_ref(lay=lay, N=N, K=K, wb=wf):
                # fp32 x the reference's way: W gathered at fp32, dense fp32 matmul
                ops.dequant(lay.packed, lay.codebook, N * K, 3, 128, torch.float32, out=wb)
                torch.matmul(xf[K], wb.view(N, K).T, out=yf)

            fns = [lambda: ops.gemm_prefill(xs[K], lay.packed, lay.codebook, N, K, out=y),
                   lambda: ops.gemm_prefill(xs[K], lay.packed, lay.codebook, N, K, out=y,
                                            path="fused"),
                   expanded,
                   lambda: torch.matmul(xs[K], w.T),
                   lambda: ops.gemm_prefill_f32(xf[K], lay.packed, lay.codebook, N, K, out=yf),
                   f32_ref]
            # each form timed twice, in alternation, and the lower time kept
            # (the first graph timed after a shape change can run up to ~30 %
            # slow while the clocks settle)
            t = [min(a, b) for a, b in zip([graph_calls_time(f) for f in fns],
                                           [graph_calls_time(f) for f in fns])]
            ms, ms_one, ms_blas, ms_ref, ms_f32, ms_f32_ref = t
            fl = 2 * M * N * K
            ws = int(_lib.load().nb_gemm_prefill_split_ws_bytes(M, N, K))
            per[n] = {"us": round(ms * 1e3, 1), "TFLOP_s": round(fl / ms / 1e9, 1),
                      "k_split_partials_MiB": round(ws / 2**20, 2),
                      "one_launch_us": round(ms_one * 1e3, 1),
                      "expand_then_torch_bf16_us": round(ms_blas * 1e3, 1),
                      "torch_dense_bf16_us": round(ms_ref * 1e3, 1),
                      "f32_x_us": round(ms_f32 * 1e3, 1),
                      "f32_x_gather_then_torch_f32_us": round(ms_f32_ref * 1e3, 1)}
            tot_ms += ms
            blas_ms += ms_blas
            ref_ms += ms_ref
            tot_fl += fl
            f32_ms += ms_f32
            f32_ref_ms += ms_f32_ref
            del w, wx[n], wf
        out[f"M{M}"] = {"layer_us": round(tot_ms * 1e3, 1),
                        "TFLOP_s": round(tot_fl / tot_ms / 1e9, 1),
                        "pct_bf16_mfma_peak": round(tot_fl / tot_ms / 1e9 / 2500 * 100, 2),
                        "model_26_layers_ms": round(26 * tot_ms, 3),
                        "expand_then_torch_bf16_layer_us": round(blas_ms * 1e3, 1),
                        "torch_dense_bf16_layer_us": round(ref_ms * 1e3, 1),
                        "f32_x_layer_us": round(f32_ms * 1e3, 1),
                        "f32_x_TFLOP_s": round(tot_fl / f32_ms / 1e9, 1),
                        "f32_x_gather_then_torch_f32_layer_us": round(f32_ref_ms * 1e3, 1),
                        "per_matmul": per}
    out["note"] = ("us / TFLOP_s: nb_gemm_prefill_split, the hand-written MFMA kernels that "
                   "read the 3-bit stream and codebooks and dequantize into LDS (bf16 operands, "
                   "fp32 accumulation, bf16 y), with a K split (fp32 partials in a workspace, "
                   "one reduction launch) where the tile grid would leave CUs idle "
                   "(k_split_partials_MiB > 0); one_launch = nb_gemm_prefill (no split); "
                   "every column is GPU time per call, 10 calls per HIP graph replay, the "
                   "lower of two timings; "
                   "comparison columns only: expand_then_torch_bf16 = "
                   "nb_dequant (W expanded to bf16 by the format kernel) then torch.matmul "
                   "(hipBLASLt), the expansion inside the timed call, "
                   "torch_dense_bf16 = torch.matmul on an already-unpacked bf16 weight (the "
                   "reference's path also unpacks and gathers W on every call, "
                   "triton_kernel.py:258-275); f32_x = nb_gemm_prefill_f32 for fp32 activations "
                   "against the exact fp32 weights (three bf16 MFMA passes over the hi / lo parts "
                   "of x and W, fp32-level products), beside f32_x_gather_then_torch_f32 = the "
                   "reference's fp32 batched branch on the GPU (nb_dequant to fp32 W, then "
                   "torch.matmul in fp32)")
    return out


def bench_skinny(dev, layers, ms=(1, 2, 4, 8, 16), per_matmul=True):
    """Config 2: M activation rows over all 182 matmuls of a step.

    batched: one launch per step -- nb_gemv_batched_sel (the streaming
    kernel, on the selector-ordered unit layout made once by
    nb_stream_layout) at M = 1, nb_gemm_skinny_quad_batched on the row-quad layout at M = 2
    (the layers re-ordered once by nb_quad_layout, outside the timing, as
    at model load), nb_gemm_skinny_tile_batched on the tile layout at M > 2
    (nb_tile_layout, likewise once; at M = 3 / 4 it measured 3-4 % faster
    than the row-quad kernel, at M = 2 about 1 % slower) -- replayed as a
    HIP graph;
    rows_layout: nb_gemm_skinny_batched on the original layout, for
    comparison; per_matmul: 182 nb_gemv launches per step (one per matmul)
    in a graph."""
    from nativebit_amd import ops, synth
    mats = [mats[name] for mats in layers for name, _, _ in synth.LAYER_SHAPES]
    quads = [ops.quad_layout(m.packed, m.cb, m.N, m.K) for m in mats] if 2 in ms else []
    tiles = [ops.tile_layout(m.packed, m.cb, m.N, m.K) for m in mats] if max(ms) > 2 else []
    sels = [ops.stream_layout(m.packed, m.N, m.K) for m in mats] if 1 in ms else []
    torch.cuda.synchronize()
    out = {}
    for M in ms:
        xs = {K: synth.make_activation(K, m=M, seed=M, device=dev, dtype=torch.bfloat16)
              for K in (2560, 6912)}
        ys = [torch.empty(M, m.N, device=dev) for m in mats]
        nbytes = sum(synth.layer_bytes(m.N, m.K, NE, BS, M, 2, 4) for m in mats)
        fl = 2 * M * sum(m.N * m.K for m in mats)
        batch = ops.GemvBatch([((xs[m.K][0] if M == 1 else xs[m.K]), m.packed, m.cb,
                                (y[0] if M == 1 else y), m.N, m.K) for m, y in zip(mats, ys)],
                              m=M)
        ms_rows = graph_time(batch.run, 20, 5)
        ms_b, kernel = ms_rows, "gemv_stream_kernel" if M == 1 else "gemv_skinny_kernel"
        extra = {}
        if M == 1:
            ysl = [torch.empty(m.N, device=dev) for m in mats]
            lbatch = ops.GemvBatch([(xs[m.K][0], p, m.cb, y, m.N, m.K)
                                    for m, p, y in zip(mats, sels, ysl)], layout="sel")
            ms_b = graph_time(lbatch.run, 20, 5)
            kernel = "gemv_stream_kernel (selector-ordered unit layout)"
            # the same selectors in the same order: the same bits
            if not all(torch.equal(a, b[0]) for a, b in zip(ysl, ys)):
                raise RuntimeError("skinny M=1: selector-ordered and original layouts disagree")
            extra = {"rows_layout_us_per_step": round(ms_rows * 1e3, 1),
                     "rows_layout_GB_s": round(nbytes / ms_rows / 1e6, 1)}
            del ysl, lbatch
        elif M == 2:
            yq = [torch.empty(M, m.N, device=dev) for m in mats]
            qbatch = ops.GemvBatch([(xs[m.K], q[0], q[1], y, m.N, m.K)
                                    for m, q, y in zip(mats, quads, yq)], m=M, layout="quad")
            ms_b, kernel = graph_time(qbatch.run, 20, 5), "gemv_quad_kernel"
            # the two kernels' products agree (fp32 sums in different orders)
            worst = max(float((a - b).norm() / b.norm()) for a, b in zip(yq[:7], ys[:7]))
            if worst > 1e-5:
                raise RuntimeError(f"skinny M={M}: quad and row layouts disagree ({worst:.2e})")
            extra = {"rows_layout_us_per_step": round(ms_rows * 1e3, 1),
                     "rows_layout_GB_s": round(nbytes / ms_rows / 1e6, 1)}
            del yq, qbatch
        elif M > 2:
            yq = [torch.empty(M, m.N, device=dev) for m in mats]
            sbatch = ops.GemvBatch([(xs[m.K], t[0], t[1], y, m.N, m.K)
                                    for m, t, y in zip(mats, tiles, yq)], m=M, layout="tile")
            ms_b = graph_time(sbatch.run, 20, 5)
            kernel = "gemv_skinny_kernel (tile layout)"
            # the same MFMAs in the same order: the same bits
            if not all(torch.equal(a, b) for a, b in zip(yq, ys)):
                raise RuntimeError(f"skinny M={M}: tile and row layouts disagree")
            extra = {"rows_layout_us_per_step": round(ms_rows * 1e3, 1),
                     "rows_layout_GB_s": round(nbytes / ms_rows / 1e6, 1)}
            del yq, sbatch

        def run():
            for m, y in zip(mats, ys):
                ops.gemv(xs[m.K], m.packed, m.cb, m.N, m.K, out=y)
        ms_p = graph_time(run, 20, 5) if per_matmul else float("nan")
        out[f"M{M}"] = {"us_per_step": round(ms_b * 1e3, 1), "GB_s": round(nbytes / ms_b / 1e6, 1),
                        "pct_hbm_peak": round(nbytes / ms_b / 1e6 / HBM_PEAK_GBS * 100, 1),
                        "TFLOP_s": round(fl / ms_b / 1e9, 2), "kernel": kernel, **extra,
                        "per_matmul_us_per_step": round(ms_p * 1e3, 1) if per_matmul else None,
                        "per_matmul_GB_s": round(nbytes / ms_p / 1e6, 1) if per_matmul else None}
        log(f"[bench] skinny M={M}: batched {ms_b*1e3:.1f} us ({nbytes/ms_b/1e6:.0f} GB/s, "
            f"{kernel}), per-matmul launches {ms_p*1e3:.1f} us")
        del ys, xs, batch
    out["note"] = ("batched: every matmul of the step in one launch (graph replay); M = 1 on "
                   "the selector-ordered unit layout (nb_stream_layout, once, untimed; "
                   "bit-identical to the original layout's products), M = 2 "
                   "on the row-quad layout (nb_quad_layout, once, untimed), M > 2 on the "
                   "tile layout (nb_tile_layout, once, untimed; bit-identical to the "
                   "original layout's products), rows_layout the same products on the "
                   "original layout; per_matmul: 182 nb_gemv launches per step in one graph")
    del quads, tiles, sels
    return out


def bench_config0(dev, cpu=True):
    """Config 0: one packed 6912x2560 layer (NE 8, BS 128, quantized N(0, 0.02)
    weights), x fp32 N(0, 1), batch 1 -- nb_gemv with the reference's exact
    fp32 arithmetic (gemv_fast_kernel), one launch per matvec, each timed
    launch reading a different copy of the layer (> 512 MB in all); beside
    it the reference CPU torch path on the same layer."""
    from nativebit_amd import ops, synth
    N, K = 6912, 2560
    lay = synth.make_layer(N, K, NE, BS, seed=0, device=dev)
    per = synth.layer_bytes(N, K, NE, BS, 1, x_bytes=4, y_bytes=4)
    copies = max(2, -(-(512 << 20) // per))
    ps = [lay.packed.clone() for _ in range(copies)]
    cbs = [lay.codebook.clone() for _ in range(copies)]
    x = synth.make_activation(K, seed=1000, device=dev)[0].contiguous()
    y = torch.empty(1, N, device=dev)

    def run():
        for p, c in zip(ps, cbs):
            ops.gemv(x, p, c, N, K, out=y)
    ms = graph_time(run, 10, 3) / copies
    out = {"us": round(ms * 1e3, 2), "GB_s": round(per / ms / 1e6, 1),
           "pct_hbm_peak": round(per / ms / 1e6 / HBM_PEAK_GBS * 100, 2), "bytes": per,
           "copies": copies, "kernel": "gemv_fast_kernel (fp32 x, exact fp32 codebook values)"}
    if cpu:
        from oracle import oracle as O
        threads = host_cpu()["threads"]
        torch.set_num_threads(threads)
        xh, ph, ch = x.cpu(), lay.packed.cpu(), lay.codebook.cpu()
        O.torch_packed_linear_f32(xh, ph, ch, N, K, BS, BITS)
        times = []
        t_start = time.perf_counter()
        while len(times) < 5 or time.perf_counter() - t_start < 3.0:
            t0 = time.perf_counter()
            O.torch_packed_linear_f32(xh, ph, ch, N, K, BS, BITS)
            times.append(time.perf_counter() - t0)
        t = statistics.median(times)
        out["cpu_reference_path"] = {"us": round(t * 1e6, 1), "GB_s": round(per / t / 1e9, 3),
                                     "threads": threads, "passes": len(times),
                                     "what": "torch CPU unpack + gather + F.linear "
                                             "(triton_kernel.py:258-275)"}
    del ps, cbs
    return out


def bench_quantize(dev):
    """Quantize-at-pack on the GPU (inference/pack.py:21-57): nearest-entry
    indices of a 6912x2560 fp32 weight against its per-block quantile
    codebooks, packed to the 3-bit stream by one kernel (nb_quantize_pack),
    beside the reference's formulation on the same device (a dense
    blocks x block_size x entries distance tensor, argmin, then nb_pack)."""
    from nativebit_amd import ops, synth
    N, K = 6912, 2560
    g = torch.Generator(device=dev).manual_seed(11)
    w = torch.randn(N * K, generator=g, device=dev) * 0.02
    cb = synth.block_codebooks(w, N * K, NE, BS)
    nbytes = w.numel() * 4 + cb.numel() * 4 + ops.packed_nbytes(N * K, BITS)
    ms = event_time(lambda: ops.quantize_pack(w, cb, BS), 20)
    ms_ref = event_time(lambda: ops.pack(synth.nearest_indices(w, N * K, cb, BS), BITS), 5)
    return {"us": round(ms * 1e3, 1), "GB_s": round(nbytes / ms / 1e6, 1),
            "pct_hbm_peak": round(nbytes / ms / 1e6 / HBM_PEAK_GBS * 100, 1), "bytes": nbytes,
            "torch_distance_argmin_then_pack_us": round(ms_ref * 1e3, 1),
            "bit_exact_vs_torch_path": bool(torch.equal(
                ops.quantize_pack(w, cb, BS), ops.pack(synth.nearest_indices(w, N * K, cb, BS), BITS))),
            "codebooks": bench_codebooks(w, N * K)}


def bench_codebooks(w, total):
    """Per-block quantile codebooks on the GPU (nb_block_codebooks: one
    64-lane workgroup sorts each block in LDS) beside torch.quantile over the
    same blocks on the same device, both timed with events."""
    from nativebit_amd import ops, synth
    ms = event_time(lambda: ops.block_codebooks(w, NE, BS), 10)
    ms_ref = event_time(lambda: synth.block_codebooks(w, total, NE, BS), 3)
    return {"us": round(ms * 1e3, 1), "GB_s_read": round(total * 4 / ms / 1e6, 1),
            "torch_quantile_us": round(ms_ref * 1e3, 1),
            "bit_exact_vs_torch_quantile": bool(torch.equal(
                ops.block_codebooks(w, NE, BS), synth.block_codebooks(w, total, NE, BS)))}


def bench_codec(dev):
    """The format kernels on one 6912x2560 layer at 2, 3 and 4 bits: nb_unpack
    (stream -> uint8 indices), nb_pack (indices -> stream; the reference's
    pack_nbits is a per-bit Python loop, nativebit/pack.py:97-138) and
    nb_dequant to fp32 / bf16 (the reference's gather, pack.py:145-169).
    Bytes = what each kernel must read and write; every timed launch of a
    graph reads a different copy (copies x bytes > 512 MB)."""
    from nativebit_amd import ops
    N, K = 6912, 2560
    total = N * K
    out = {}
    gen = torch.Generator(device=dev).manual_seed(13)
    for bits in (2, 3, 4):
        ne = 1 << bits
        pb = ops.packed_nbytes(total, bits)
        nb = total // BS
        copies = max(2, -(-(512 << 20) // (total + pb)))
        idx = [torch.randint(0, ne, (total,), dtype=torch.uint8, device=dev, generator=gen)
               for _ in range(copies)]
        ps = [ops.pack(i, bits) for i in idx]
        cbs = [torch.randn(nb, ne, device=dev, generator=gen) for _ in range(copies)]
        res = {}
        for name, fn, nbytes in (
                ("unpack", lambda i: ops.unpack(ps[i], total, bits), pb + total),
                ("pack", lambda i: ops.pack(idx[i], bits), total + pb),
                ("dequant_f32", lambda i: ops.dequant(ps[i], cbs[i], total, bits, BS),
                 pb + nb * ne * 4 + total * 4),
                ("dequant_bf16", lambda i: ops.dequant(ps[i], cbs[i], total, bits, BS,
                                                       torch.bfloat16),
                 pb + nb * ne * 4 + total * 2)):
            def run():
                for i in range(copies):
                    fn(i)
            ms = graph_time(run, 10, 3) / copies
            res[name] = {"us": round(ms * 1e3, 2), "GB_s": round(nbytes / ms / 1e6, 1),
                         "pct_hbm_peak": round(nbytes / ms / 1e6 / HBM_PEAK_GBS * 100, 1),
                         "bytes": nbytes}
        out[f"bits{bits}"] = res
        del idx, ps, cbs
    out["note"] = ("6912x2560 weights, block 128, one launch per copy inside a HIP graph; "
                   "unpack and pack verified against the oracle in tests/test_gpu_parity.py")
    return out


def bench_sweep(dev):
    """Config 3: bit width x block size at batch 1 (nb_gemv)."""
    from nativebit_amd import ops, synth
    out = {}
    gen = torch.Generator(device=dev).manual_seed(7)
    for (N, K) in ((6912, 2560), (2560, 6912)):
        x = synth.make_activation(K, seed=K, device=dev, dtype=torch.bfloat16)[0].contiguous()
        for ne in (4, 8, 16):
            bits = {4: 2, 8: 3, 16: 4}[ne]
            for bs in (64, 128, 256):
                per = synth.layer_bytes(N, K, ne, bs, 1, 2, 4)
                copies = max(2, -(-(512 << 20) // per))
                nb = N * K // bs
                from nativebit_amd import pack as host_pack
                pbytes = host_pack.packed_nbytes(nb * bs, bits)
                ps = [torch.randint(0, 256, (pbytes,), dtype=torch.uint8, device=dev, generator=gen)
                      for _ in range(copies)]
                cbs = [torch.randn(nb, ne, device=dev, generator=gen) * 0.02 for _ in range(copies)]
                y = torch.empty(1, N, device=dev)

                def run():
                    for p, c in zip(ps, cbs):
                        ops.gemv(x, p, c, N, K, bits=bits, block_size=bs, out=y)
                ms = graph_time(run, 10, 3) / copies
                out[f"{N}x{K}_NE{ne}_BS{bs}"] = {"us": round(ms * 1e3, 2),
                                                 "GB_s": round(per / ms / 1e6, 1),
                                                 "bytes": per, "copies": copies}
                del ps, cbs
    out["note"] = ("batch-1 nb_gemv, bf16 x, fp32 y; each timed launch reads a different copy "
                   "(copies x bytes > 512 MB); random indices and codebooks")
    return out


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

    layers = build_model(dev, args.layers, args.random_weights)
    all_mats = [mats[name] for mats in layers for name, _, _ in synth.LAYER_SHAPES]
    step_bytes = sum(m.bytes for m in all_mats)
    wanted = args.schedules.split(",")
    results = {}

    # The streams in the selector-ordered unit layout, made once outside the
    # timing as at model load (the same bytes; the products bit-identical).
    sel = [ops.stream_layout(m.packed, m.N, m.K) for m in all_mats]
    batch = ops.GemvBatch([(m.x, p, m.cb, m.y, m.N, m.K) for m, p in zip(all_mats, sel)],
                          layout="sel")
    y_ref = [torch.empty_like(m.y) for m in all_mats]
    batch_ref = ops.GemvBatch([(m.x, m.packed, m.cb, y, m.N, m.K)
                               for m, y in zip(all_mats, y_ref)])
    batch.run()
    batch_ref.run()
    torch.cuda.synchronize()
    if not all(torch.equal(m.y, y) for m, y in zip(all_mats, y_ref)):
        raise RuntimeError("batched: the selector-ordered and original layouts disagree")
    ginfo = {}
    ms = graph_time(batch.run, args.steps, args.warmup, info=ginfo)
    transient = transient_profile(ginfo.pop("graph"))
    err = spot_check(all_mats[:7])
    ms_ref = graph_time(batch_ref.run, args.steps, args.warmup)
    results["batched"] = {"launches": 1, "us_per_step": round(ms * 1e3, 2),
                          "GB_s": round(step_bytes / ms / 1e6, 1),
                          "settle_replays": ginfo["settle_replays"],
                          "layout": "selector-ordered units (nb_stream_layout, once, untimed)"}
    results["batched_original_layout"] = {
        "launches": 1, "us_per_step": round(ms_ref * 1e3, 2),
        "GB_s": round(step_bytes / ms_ref / 1e6, 1),
        "note": "the same launch on the reference's stream layout (nb_gemv_batched); "
                "bit-identical outputs (checked)"}
    log(f"[bench] batched  : 1 launch/step, {step_bytes} B, {ms*1e3:.1f} us/step, "
        f"{step_bytes/ms/1e6:.1f} GB/s ({step_bytes/ms/1e6/HBM_PEAK_GBS*100:.1f}% of 8 TB/s), "
        f"spot-check rel err {err:.2e}; original layout {ms_ref*1e3:.1f} us/step")

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
            "schedule": ("batched: all 182 GEMVs in one persistent launch (HIP graph replay), "
                         "index streams in the selector-ordered unit layout made once at load "
                         "(nb_stream_layout; same bytes, bit-identical products)"),
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
            "kernel": "gemv_stream_kernel (selector-ordered unit layout)",
            "method": ("algorithmic bytes per launch (0.625 B/weight + x + y) / HIP-event time "
                       "per graph replay of the single launch, on the launch stream"),
        },
        "schedules": results,
        "timing": {
            "settle": (f"{ginfo['settle_replays']} untimed replays (~{SETTLE_S} s of GPU time) "
                       f"before the {args.warmup} warm-up and {args.steps} timed replays"),
            "after_idle_us_per_replay": transient,
            "after_idle_note": ("the same graph replayed right after 50 ms of GPU idle: the "
                                "first ~1 ms runs at full clocks, then the power controller "
                                "throttles for ~20 ms before it settles; the timed region "
                                "above starts after that"),
        },
        "parity": {"spot_check_rel_err_vs_f64": err},
    }
    if not args.no_extra:
        extra = {}
        wanted_extra = [e for e in args.extra.split(",") if e]
        for name, fn in (("config0", lambda: bench_config0(dev, not args.no_cpu_baseline)),
                         ("decode", lambda: bench_decode(dev, args.decode_tokens)),
                         ("prefill", lambda: bench_prefill(dev, args.random_weights)),
                         ("skinny", lambda: bench_skinny(
                             dev, layers, tuple(int(v) for v in args.skinny_m.split(",")),
                             not args.no_per_matmul)),
                         ("sweep", lambda: bench_sweep(dev)),
                         ("quantize", lambda: bench_quantize(dev)),
                         ("codec", lambda: bench_codec(dev))):
            if name not in wanted_extra:
                continue
            t0 = time.time()
            log(f"[bench] {name} ...")
            extra[name] = fn()
            log(f"[bench] {name} done in {time.time() - t0:.1f}s: "
                f"{json.dumps(extra[name])[:300]}")
        result["configs"] = extra
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
