#!/usr/bin/env python3
"""Prefill-attention throughput of libqattn.so on one MI355X (BASELINE.json metric).

One step = the hot path over the two workloads the metric is quoted on, each for all 28 layers
of independent seeded Q/K/V resident in HBM:
  * 16 x 500 tokens, full causal      (BASELINE config 2)
  * 1 x 5000 tokens, 176-prefix + 432-local sparse causal (the metric's sparse row)
Every launch is one layer's attention through the C ABI (qattn_run_encode), exactly what the
Node engine issues.  Timing: HIP events on the launch stream around exactly K steps, with a
device synchronize on both sides.  A second pass brackets every launch with its own events to
get the kernel's average duration for the roofline figure.

cpu_baseline: the reference's tiled algorithm restated on the CPU (oracle/, f16-faithful, the
"port"), timed on a bounded sample of the same workload on this host's cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload both|full|sparse|cfg3|cfg4]
"""
import argparse
import importlib.util
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "qwen3-embedding-webgpu-prepacked_amd")
LAYERS = 28
PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16/bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

WORKLOADS = {
    # name: (config id for seeds, lengths, mask kind, description)
    "full": (2, [500] * 16, 0, "16x500 full causal"),
    "sparse": (5, [5000], 1, "1x5000 sparse (176 prefix + 432 window)"),
    "cfg3": (3, [1500], 1, "1x1500 sparse (176 prefix + 432 window)"),
    "cfg4": (4, [5000] * 4, 1, "4x5000 sparse (176 prefix + 432 window) + last rows"),
}
SETS = {"both": ["full", "sparse"], "full": ["full"], "sparse": ["sparse"], "cfg3": ["cfg3"],
        "cfg4": ["cfg4"]}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def load_binding():
    spec = importlib.util.spec_from_file_location("qattn", os.path.join(PKG, "qattn.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["qattn"] = mod
    spec.loader.exec_module(mod)
    return mod


class Workload:
    """28 layers of one packing, resident in HBM, with one planned run per layer."""

    def __init__(self, ctx, q, name):
        self.name = name
        cfg, lengths, mask, desc = WORKLOADS[name]
        self.desc_text = desc
        self.lengths = lengths
        self.cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
        T = int(self.cu[-1])
        self.tokens = T
        nseq = len(lengths)
        self.bufs, self.runs = [], []
        for layer in range(LAYERS):
            bq, bk, bv = ctx.alloc(T * 4096), ctx.alloc(T * 2048), ctx.alloc(T * 2048)
            bo = ctx.alloc(T * 4096)
            bl = ctx.alloc(nseq * 4096) if name == "cfg4" else None
            ctx.gen_qkv(cfg, layer, self.cu, bq.ptr, bk.ptr, bv.ptr)
            d = q.make_desc(bq.ptr, bk.ptr, bv.ptr, bo.ptr, self.cu, mask=mask,
                            o_last=bl.ptr if bl else None)
            self.runs.append(ctx.run(d))
            self.bufs += [b for b in (bq, bk, bv, bo, bl) if b]
        ctx.synchronize()
        self.info = self.runs[0].info()

    def encode_all(self):
        for r in self.runs:
            r.encode()

    def free(self):
        for r in self.runs:
            r.destroy()
        for b in self.bufs:
            b.free()


def cpu_baseline(selected):
    """Time the oracle's f16-faithful restatement of the reference's tiled kernel on a bounded
    sample of each workload's layer, scale to 28 layers, return tokens/s over the same step."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle
    threads = oracle.get_threads()
    total_s = 0.0
    samples = []
    for name in selected:
        cfg, lengths, mask, _ = WORKLOADS[name]
        if len(lengths) > 1:
            # whole sequences: 4 of the batch (all equal length), scaled by nseq / 4
            k = min(4, len(lengths))
            sub = lengths[:k]
            cu = np.concatenate([[0], np.cumsum(sub)]).astype(np.int32)
            qh, kh, vh = oracle.gen_qkv(cfg, 0, cu)
            t0 = time.perf_counter()
            oracle.attention_tiled16(qh, kh, vh, cu, kind=mask)
            dt = time.perf_counter() - t0
            layer_s = dt * len(lengths) / k
            samples.append(f"{name}: {k} of {len(lengths)} sequences of layer 0")
        else:
            # every 4th 16-query tile of the single sequence, scaled by the tile count ratio
            L = lengths[0]
            cu = np.array([0, L], dtype=np.int32)
            qh, kh, vh = oracle.gen_qkv(cfg, 0, cu)
            ntiles = (L + 15) // 16
            step = 4
            done = len(range(0, ntiles, step))
            t0 = time.perf_counter()
            oracle.attention_tiled16_tiles(qh, kh, vh, cu, 0, 0, ntiles, step, kind=mask)
            dt = time.perf_counter() - t0
            layer_s = dt * ntiles / done
            samples.append(f"{name}: every {step}th 16-query tile ({done} of {ntiles}) of layer 0")
        log(f"cpu baseline {name}: sample {dt:.2f} s -> {layer_s:.2f} s per layer")
        total_s += layer_s * LAYERS
    tokens = sum(sum(WORKLOADS[n][1]) for n in selected) * LAYERS
    return {
        "value": tokens / total_s,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": "; ".join(samples) + f"; x{LAYERS} layers; f16-faithful restatement of the "
                  "reference's 16x16 tiled WGSL kernel (oracle/oracle.c, OpenMP)",
    }


def copy_calibration(mib):
    """Five copies of `mib` MiB between two device buffers: each dispatch reads and writes exactly
    mib MiB, so a profiler's per-dispatch FETCH_SIZE / WRITE_SIZE (KiB) divided by 1024*mib is the
    counter's scale for a plain streaming kernel."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy calibration: 5 x {mib} MiB device copies done")


def pool_timing(reps):
    """The consumer kernel alone (not the headline metric): qattn_pool_last_l2 over the last rows
    of a 16 x 500 packing, at width 2048 (attention output rows) and 1024 (the reference pool's
    hidden width, ops.ts:371), `reps` back-to-back launches each between HIP events on the
    context stream.  One JSON line per width; algorithmic bytes = 16 rows x width x (2 + 4)."""
    q = load_binding()
    ctx = q.Context(0)
    cu = np.concatenate([[0], np.cumsum([500] * 16)]).astype(np.int32)
    T = int(cu[-1])
    for width in (2048, 1024):
        x, out = ctx.alloc(T * width * 2), ctx.alloc(16 * width * 4)
        ctx.fill_normal(x.ptr, T, width, width, 7)
        for _ in range(10):
            ctx.pool_last_l2(x.ptr, width, width, cu, out.ptr)
        e0, e1 = ctx.event(), ctx.event()
        ctx.synchronize()
        e0.record()
        for _ in range(reps):
            ctx.pool_last_l2(x.ptr, width, width, cu, out.ptr)
        e1.record()
        ctx.synchronize()
        us = e0.elapsed_ms(e1) * 1000.0 / reps
        nbytes = 16 * width * 6
        print(json.dumps({"kernel": "pool_last_l2_kernel", "sequences": 16, "width": width, "launches": reps,
                          "us_per_launch": round(us, 3), "bytes": nbytes, "GB/s": round(nbytes / us / 1e3, 2)}),
              flush=True)
        for b in (x, out):
            b.free()
        e0.destroy()
        e1.destroy()
    ctx.close()


def q4_timing(reps):
    """The projection kernel alone (not the headline metric): qattn_q4_matmul at the shapes one
    layer of the 16 x 500 packing multiplies (M = 8000 tokens): the fused QKV projection
    (K 1024 -> N 4096), the attention output projection (2048 -> 1024), the gate/up projection
    (1024 -> 6144) and the down projection (3072 -> 1024).  Random Q4_0 records, `reps` launches
    per shape between HIP events; algorithmic FLOP = 2 M N K.  One JSON line per shape."""
    q = load_binding()
    ctx = q.Context(0)
    rng = np.random.default_rng(0)
    M = 8000
    for name, K, N in (("qkv", 1024, 4096), ("attn_out", 2048, 1024), ("gate_up", 1024, 6144), ("down", 3072, 1024)):
        nbytes = q.lib().qattn_q4_compact_bytes(K, N)
        wts = rng.integers(0, 256, size=nbytes, dtype=np.uint8)
        rec = wts.reshape(-1, 20)
        rec[:, 0:2] = np.full((rec.shape[0], 1), 0.01, np.float16).view(np.uint8)  # scale 0.01
        bw = ctx.upload(wts)
        bx, by = ctx.alloc(M * K * 2), ctx.alloc(M * N * 2)
        ctx.fill_normal(bx.ptr, M, K, K, 11)
        for _ in range(3):
            ctx.q4_matmul(bx.ptr, M, K, bw.ptr, nbytes, N, by.ptr)
        e0, e1 = ctx.event(), ctx.event()
        ctx.synchronize()
        e0.record()
        for _ in range(reps):
            ctx.q4_matmul(bx.ptr, M, K, bw.ptr, nbytes, N, by.ptr)
        e1.record()
        ctx.synchronize()
        us = e0.elapsed_ms(e1) * 1000.0 / reps
        flop = 2.0 * M * N * K
        print(json.dumps({"kernel": "q4_matmul_kernel", "shape": name, "M": M, "K": K, "N": N, "launches": reps,
                          "us_per_launch": round(us, 2), "TFLOP/s": round(flop / us / 1e6, 1),
                          "frac_of_fp16_peak": round(flop / us / 1e6 / PEAK_FP16_TFLOPS, 3)}), flush=True)
        for b in (bw, bx, by):
            b.free()
        e0.destroy()
        e1.destroy()
    ctx.close()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=sorted(SETS), default="both")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 plain device copies of MIB MiB (torch copy_) and exit: the "
                         "known-size reference for rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    ap.add_argument("--pool", type=int, default=0, metavar="N",
                    help="only time N launches of the last-token pool kernel per width and exit")
    ap.add_argument("--q4", type=int, default=0, metavar="N",
                    help="only time N launches of the Q4_0 dequant-GEMM per projection shape and exit")
    args = ap.parse_args()
    if args.q4:
        q4_timing(args.q4)
        return
    if args.pool:
        pool_timing(args.pool)
        return
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each GPU box has one "
              "MI355X). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    q = load_binding()
    ctx = q.Context(0)
    dev, cus = ctx.device_name()
    log(f"device {dev} ({cus} CUs)")
    selected = SETS[args.workload]
    wls = [Workload(ctx, q, n) for n in selected]
    for w in wls:
        i = w.info
        log(f"{w.name}: {w.desc_text}: tokens {i.tokens}, pairs {i.pairs}, work items {i.work_items}, "
            f"flops/launch {i.flops:.4e}, bytes/launch {i.bytes:.4e}, tile waste {i.tile_pairs / i.pairs:.3f}")

    def step():
        for w in wls:
            w.encode_all()

    for _ in range(args.warmup):
        step()
    ctx.synchronize()

    # ---- timed region: exactly K steps ----
    e0, e1 = ctx.event(), ctx.event()
    ctx.synchronize()
    t_host = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    ctx.synchronize()
    host_ms = (time.perf_counter() - t_host) * 1e3
    region_ms = e0.elapsed_ms(e1)
    ms_per_step = region_ms / args.steps
    log(f"timed {args.steps} steps: {region_ms:.3f} ms on device events ({host_ms:.3f} ms host)")

    # ---- per-launch kernel durations (separate pass, same launches) ----
    reps = max(3, min(args.steps, 10))
    per = {w.name: [] for w in wls}
    evs = [(ctx.event(), ctx.event()) for _ in range(LAYERS)]
    for _ in range(reps):
        for w in wls:
            for r, (a, b) in zip(w.runs, evs):
                a.record()
                r.encode()
                b.record()
            ctx.synchronize()
            per[w.name] += [a.elapsed_ms(b) for a, b in evs]
    for a, b in evs:
        a.destroy()
        b.destroy()

    tokens_per_step = sum(w.tokens for w in wls) * LAYERS
    value = tokens_per_step / (ms_per_step / 1e3)
    total_flops = sum(w.info.flops for w in wls) * LAYERS
    total_bytes = sum(w.info.bytes for w in wls) * LAYERS
    kern_ms_step = sum(np.mean(per[w.name]) * LAYERS for w in wls)
    breakdown = {}
    for w in wls:
        avg = float(np.mean(per[w.name]))
        breakdown[w.name] = {
            "workload": w.desc_text,
            "kernel_avg_us": round(avg * 1e3, 3),
            "tokens_per_s": round(w.tokens / (avg / 1e3), 1),
            "tflops": round(w.info.flops / (avg / 1e3) / 1e12, 2),
            "mfma_frac": round(w.info.flops / (avg / 1e3) / 1e12 / PEAK_FP16_TFLOPS, 4),
            "gbs": round(w.info.bytes / (avg / 1e3) / 1e9, 1),
            "hbm_frac": round(w.info.bytes / (avg / 1e3) / 1e9 / PEAK_HBM_GBS, 4),
        }
        log(f"{w.name}: kernel avg {avg * 1e3:.2f} us, {breakdown[w.name]}")
    achieved = total_flops / (kern_ms_step / 1e3) / 1e12

    traffic = None
    tpath = os.path.join(REPO, "profiles", "traffic.json")
    if os.path.exists(tpath):
        try:
            traffic = json.load(open(tpath)).get(args.workload)
        except (ValueError, OSError):
            traffic = None

    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline(selected)
        except Exception as e:  # the baseline is reported, never the measured path
            log(f"cpu baseline failed: {e}")

    out = {
        "metric": "prefill-attn tokens/s/GPU at 16x500 full & 1x5000 sparse; % fp16 MFMA peak",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded N(0,1) Q/K/V, QK RMSNorm + RoPE theta 1e6, generated on device)",
        "config": {
            "workload": " + ".join(w.desc_text for w in wls) + f", {LAYERS} layers each, "
                        "16 q heads / 8 kv heads, head_dim 128",
            "layers": LAYERS,
            "tokens_per_step": tokens_per_step,
            "launches_per_step": LAYERS * len(wls),
            "breakdown": breakdown,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_FP16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP16_TFLOPS, 4),
            "traffic": traffic,
            "traffic_note": "HBM bytes per launch (mean over the step's launches), rocprofv3 "
                            "FETCH_SIZE x2.0 + WRITE_SIZE x1.0 (copy-calibrated), profiles/traffic.json",
            "kernel": "attn_fwd_kernel (+ attn_merge_kernel on split-K plans)",
            "algorithmic_flops_per_step": total_flops,
            "algorithmic_bytes_per_step": total_bytes,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    for w in wls:
        w.free()
    ctx.close()


if __name__ == "__main__":
    main()
