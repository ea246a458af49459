#!/usr/bin/env python3
"""Prefill-attention throughput of libqattn.so on one MI355X (BASELINE.json metric).

One step = the hot path over the two workloads the metric is quoted on, each for all 28 layers
of independent seeded Q/K/V resident in HBM:
  * 16 x 500 tokens, full causal      (BASELINE config 2)
  * 1 x 5000 tokens, 176-prefix + 432-local sparse causal (the metric's sparse row)
Every launch is one layer's attention through the C ABI (qattn_run_encode), exactly what the
Node engine issues.  Timing: HIP events on the launch stream around exactly K steps, with a
device synchronize on both sides; roofline.achieved is the step's algorithmic FLOPs over the same
step time.  A second pass times each workload alone on the same basis -- its 28 layer launches,
several rounds back to back between one pair of events, no synchronisation inside -- and divides
by the launch count: the workload's average launch duration (gaps between consecutive launches
included), for the headline workloads and, reported beside them in config.breakdown, for the
batch-invariant 1 x 5000 plan the engine uses and the other BASELINE configs (0: 1 x 50, 1: 16
ragged 10..150, 3: 1 x 1500 sparse, 4: 4 x 5000 sparse with last-token rows).

cpu_baseline: the reference's tiled kernel (src/webgpu/ops.ts:168-241) restated in JavaScript
(oracle/tiled16.js, f16 rounding points as the WGSL) and run under Node on this host's cores,
on a bounded sample of the same two workloads, once on one thread and once on worker threads;
its output is first checked bit for bit against the C restatement on config 0.  The C port's
own OpenMP timing is reported beside it as a cross-check.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload both|full|sparse|cfg3|cfg4]
"""
import argparse
import hashlib
import importlib.util
import json
import os
import re
import shutil
import subprocess
import sys
import tempfile
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "qwen3-embedding-webgpu-prepacked_amd")
LAYERS = 28
PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16/bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
CPU_THREADS_MAX = 16        # a GPU box's CPU share


def mix64(z):
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9 & 0xFFFFFFFFFFFFFFFF
    z = (z ^ (z >> 27)) * 0x94D049BB133111EB & 0xFFFFFFFFFFFFFFFF
    return z ^ (z >> 31)


def config_seed(config, layer, tensor):
    return 0x51574E3300000000 | (config & 0xFF) << 16 | (layer & 0xFF) << 8 | (tensor & 0xFF)


def config1_lengths():
    """16 lengths uniform in 10..150 from the SplitMix64 stream of tensor 3
    (the generator qattn_gen_qkv seeds Q/K/V from: seed + (i + 1) * golden ratio, finalised)."""
    s = config_seed(1, 0, 3)
    return [10 + (mix64((s + (i + 1) * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF) >> 33) % 141
            for i in range(16)]


FLAG_BATCH_INVARIANT = 1
WORKLOADS = {
    # name: (config id for seeds, lengths, mask kind, o_last, description, run flags)
    "full": (2, [500] * 16, 0, False, "16x500 full causal", 0),
    "sparse": (5, [5000], 1, False, "1x5000 sparse (176 prefix + 432 window)", 0),
    # The same launch with the plan the Node engine and the model plan use by default
    # (QATTN_FLAG_BATCH_INVARIANT: no split-K, no merge kernel).
    "sparse_bi": (5, [5000], 1, False, "1x5000 sparse, batch-invariant plan (the engine's default)",
                  FLAG_BATCH_INVARIANT),
    "cfg0": (0, [50], 1, False, "cfg0 1x50 causal", 0),
    "cfg1": (1, None, 1, False, "cfg1 16 ragged 10..150 causal", 0),
    "cfg3": (3, [1500], 1, False, "cfg3 1x1500 sparse (176 prefix + 432 window)", 0),
    "cfg4": (4, [5000] * 4, 1, True, "cfg4 4x5000 sparse (176 prefix + 432 window) + last rows", 0),
}
SETS = {"both": ["full", "sparse"], "full": ["full"], "sparse": ["sparse"], "cfg3": ["cfg3"],
        "cfg4": ["cfg4"]}
EXTRA = ["sparse_bi", "cfg0", "cfg1", "cfg3", "cfg4"]  # in the breakdown of the default run
PEAK_HBM_MEASURED_GBS = 6100.0  # streaming copy on these boxes (the attainable-roofline ceiling)


def lengths_of(name):
    lengths = WORKLOADS[name][1]
    return config1_lengths() if lengths is None else lengths


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
        cfg, _, mask, o_last, desc, flags = WORKLOADS[name]
        self.desc_text = desc
        self.lengths = lengths_of(name)
        self.cu = np.concatenate([[0], np.cumsum(self.lengths)]).astype(np.int32)
        T = int(self.cu[-1])
        self.tokens = T
        nseq = len(self.lengths)
        self.bufs, self.runs = [], []
        for layer in range(LAYERS):
            bq, bk, bv = ctx.alloc(T * 4096), ctx.alloc(T * 2048), ctx.alloc(T * 2048)
            bo = ctx.alloc(T * 4096)
            bl = ctx.alloc(nseq * 4096) if o_last else None
            ctx.gen_qkv(cfg, layer, self.cu, bq.ptr, bk.ptr, bv.ptr)
            d = q.make_desc(bq.ptr, bk.ptr, bv.ptr, bo.ptr, self.cu, mask=mask,
                            o_last=bl.ptr if bl else None, flags=flags)
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


# ---- CPU baseline (the checker's restatements; never the measured GPU path) --------------------

def visited_key_tiles(L, kind, prefix=176, window=432):
    """16-key tiles the reference kernel visits per 16-query tile gx (its loop and skip,
    ops.ts:205-209): the work measure the sample is scaled by."""
    out = []
    ps, ws = min(L, prefix), min(L, window)
    for gx in range((L + 15) // 16):
        limit = min(L, (gx + 1) * 16)
        start = gx * 16 + 1 - ws if gx * 16 + 1 > ws else 0
        n = 0
        for kb in range(0, limit, 16):
            if kind == 1 and kb >= ps and kb + 15 < start:
                continue
            n += 1
        out.append(n)
    return out


def node_samples(name, per_stratum):
    """Sample of (sequence, query tile, head) groups of one workload's layer 0, and the factor that
    scales its visited-tile count to the whole layer's.  16 x 500: every 2nd query tile of
    sequence 0 (all sequences are alike), `per_stratum` heads each; 1 x 5000: every 16th query
    tile, `per_stratum` heads each (heads cost the same).  A run on N threads takes N heads per
    query tile, so its wall time stays near the one-thread run's."""
    cfg, _, kind = WORKLOADS[name][:3]
    lengths = lengths_of(name)
    L = lengths[0]
    vt = visited_key_tiles(L, kind)
    step = 2 if name == "full" else 16
    sample, sampled = [], 0
    for gx in range(0, len(vt), step):
        for j in range(per_stratum):
            sample.append([0, gx, (gx // step * per_stratum + j) % 16])
            sampled += vt[gx]
    total = sum(vt) * 16 * len(lengths)
    return sample, total / sampled, kind


def cpu_baseline(selected):
    """The JS restatement under Node: parity-checked on config 0, then timed on one thread and on
    N worker threads over bounded samples; per-layer times scaled by visited-tile counts and to
    28 layers; tokens/s over the same step as the GPU value."""
    node = shutil.which("node")
    if node is None:
        raise RuntimeError("node is not installed on this host")
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle
    js = os.path.join(REPO, "oracle", "tiled16.js")
    nthreads = min(CPU_THREADS_MAX, len(os.sched_getaffinity(0)))
    version = subprocess.run([node, "--version"], capture_output=True, text=True).stdout.strip()
    with tempfile.TemporaryDirectory() as tmp:
        def stage(cfg, cu, kind, sample=None):
            q, k, v = oracle.gen_qkv(cfg, 0, cu)
            q.tofile(os.path.join(tmp, "q.bin"))
            k.tofile(os.path.join(tmp, "k.bin"))
            v.tofile(os.path.join(tmp, "v.bin"))
            meta = {"cu": [int(x) for x in cu], "kind": kind, "prefix": 176, "window": 432}
            if sample is not None:
                meta["sample"] = sample
            with open(os.path.join(tmp, "meta.json"), "w") as f:
                json.dump(meta, f)
            return q, k, v

        # parity first: config 0 through the JS restatement equals the C restatement bit for bit
        cu0 = np.array([0, 50], np.int32)
        q, k, v = stage(0, cu0, 1)
        subprocess.run([node, js, "run", tmp], check=True, timeout=120)
        got = np.fromfile(os.path.join(tmp, "o.bin"), np.uint16).reshape(50, 2048)
        want = oracle.attention_tiled16(q, k, v, cu0, kind=1).reshape(50, 2048)
        if not np.array_equal(got, want):
            raise RuntimeError(f"JS restatement differs from the C one on config 0 "
                               f"({int((got != want).sum())} values)")
        log(f"cpu baseline: node {version}: JS restatement equals the C one on config 0 (bit for bit)")

        layer_s = {1: 0.0, nthreads: 0.0}
        notes = []
        for name in selected:
            lengths = lengths_of(name)
            cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
            if len(lengths) > 1:
                cu = cu[:2]  # sequence 0 carries the sample (the sequences are alike)
            for threads in (1, nthreads):
                sample, scale, kind = node_samples(name, threads)
                stage(WORKLOADS[name][0], cu, kind, sample)
                r = subprocess.run([node, js, "time", tmp, str(threads)], capture_output=True,
                                   text=True, timeout=600, check=True)
                rep = json.loads(r.stdout.strip().splitlines()[-1])
                layer_s[threads] += rep["seconds"] * scale
                log(f"cpu baseline {name}: {len(sample)} groups on {threads} thread(s): "
                    f"{rep['seconds']:.2f} s -> {rep['seconds'] * scale:.1f} s per layer")
            notes.append(f"{name}: 1 in {2 if name == 'full' else 16} 16-query tiles of sequence 0 "
                         f"x 1 head per thread (scaled by visited 16-key tiles)")
        # The C port (OpenMP) as a cross-check of the JS figures.
        c_threads = oracle.get_threads()
        c_layer_s = 0.0
        for name in selected:
            lengths = lengths_of(name)
            L = lengths[0]
            cu = np.array([0, L], np.int32)
            q, k, v = oracle.gen_qkv(WORKLOADS[name][0], 0, cu)
            vt = visited_key_tiles(L, WORKLOADS[name][2])
            step = 4
            t0 = time.perf_counter()
            oracle.attention_tiled16_tiles(q, k, v, cu, 0, 0, len(vt), step, kind=WORKLOADS[name][2])
            dt = time.perf_counter() - t0
            c_layer_s += dt * sum(vt) * len(lengths) / sum(vt[::step])
    tokens = sum(sum(lengths_of(n)) for n in selected) * LAYERS
    return {
        "value": tokens / (layer_s[nthreads] * LAYERS),
        "unit": "tokens/s",
        "cores": nthreads,
        "kind": "port",
        "sample": "; ".join(notes) + f"; x{LAYERS} layers; the reference's 16x16 tiled WGSL kernel "
                  "(ops.ts:168-241) restated in JavaScript (oracle/tiled16.js, f16 rounding points "
                  "as the WGSL), bit-identical to the C restatement on config 0",
        "runtime": f"node {version}, worker_threads",
        "single_thread_value": tokens / (layer_s[1] * LAYERS),
        "host_cpus": os.cpu_count(),
        "c_port_cross_check": {"value": tokens / (c_layer_s * LAYERS), "cores": c_threads,
                               "kind": "port", "runtime": "oracle/oracle.c, OpenMP"},
    }


# ---- auxiliary timings --------------------------------------------------------------------------

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


def rope_timing(reps):
    """The producer alone (not the headline metric): qattn_qk_norm_rope_qkv over one layer of the
    16 x 500 packing -- qkvRaw [8000, 4096] -> compact Q [8000, 2048] and K [8000, 1024], RMSNorm
    with gains + RoPE -- `reps` back-to-back launches between HIP events on the context stream.
    Algorithmic bytes = 8000 tokens x 3072 values x (2 read + 2 written)."""
    q = load_binding()
    ctx = q.Context(0)
    cu = np.concatenate([[0], np.cumsum([500] * 16)]).astype(np.int32)
    T = int(cu[-1])
    x, bq, bk = ctx.alloc(T * 4096 * 2), ctx.alloc(T * 2048 * 2), ctx.alloc(T * 1024 * 2)
    w = ctx.upload(np.ones(256, np.float32))
    ctx.fill_normal(x.ptr, T, 4096, 4096, 5)
    for _ in range(10):
        ctx.qk_norm_rope_qkv(x.ptr, bq.ptr, bk.ptr, cu, q_weight_ptr=w.ptr, k_weight_ptr=w.ptr + 512)
    e0, e1 = ctx.event(), ctx.event()
    ctx.synchronize()
    e0.record()
    for _ in range(reps):
        ctx.qk_norm_rope_qkv(x.ptr, bq.ptr, bk.ptr, cu, q_weight_ptr=w.ptr, k_weight_ptr=w.ptr + 512)
    e1.record()
    ctx.synchronize()
    us = e0.elapsed_ms(e1) * 1000.0 / reps
    nbytes = T * 3072 * 4
    print(json.dumps({"kernel": "qk_norm_rope_kernel", "workload": "16x500 qkvRaw -> Q, K", "tokens": T,
                      "launches": reps, "us_per_launch": round(us, 3), "bytes": nbytes,
                      "GB/s": round(nbytes / us / 1e3, 1),
                      "hbm_frac": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 3)}), flush=True)
    for b in (x, bq, bk, w):
        b.free()
    e0.destroy()
    e1.destroy()
    ctx.close()


Q4_SHAPES = (("qkv", 1024, 4096), ("attn_out", 2048, 1024), ("gate_up", 1024, 6144), ("down", 3072, 1024))


def q4_timing(reps, ms=(8000,)):
    """The projection kernel alone (not the headline metric): qattn_q4_matmul at the shapes one
    layer multiplies for M tokens (8000 = one 16 x 500 packing): the fused QKV projection
    (K 1024 -> N 4096), the attention output projection (2048 -> 1024), the gate/up projection
    (1024 -> 6144) and the down projection (3072 -> 1024).  Random Q4_0 records, `reps` launches
    per shape between HIP events; algorithmic FLOP = 2 M N K.  One JSON line per shape."""
    q = load_binding()
    ctx = q.Context(0)
    rng = np.random.default_rng(0)
    for M, (name, K, N) in ((M, s) for M in ms for s in Q4_SHAPES):
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


def dense_gemm_timing(reps, ms=(8000,)):
    """A reference ceiling for the projection shapes, not part of the path: torch.matmul on dense
    fp16 operands (hipBLASLt's GEMM, no dequantisation) at the shapes q4_timing runs, `reps`
    launches between events after 3 warm-ups.  Runs without libqattn.so in the process: torch
    brings its own HIP runtime, which finds no device once the library's runtime holds it."""
    import torch
    torch.manual_seed(0)
    for M, (name, K, N) in ((M, s) for M in ms for s in Q4_SHAPES):
        x = torch.randn(M, K, device="cuda", dtype=torch.float16)
        wt = (torch.randn(N, K, device="cuda", dtype=torch.float16) * 0.02).t()
        for _ in range(3):
            torch.matmul(x, wt)
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record()
        for _ in range(reps):
            torch.matmul(x, wt)
        t1.record()
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) * 1000.0 / reps
        flop = 2.0 * M * N * K
        print(json.dumps({"kernel": "torch.matmul fp16 (hipBLASLt)", "shape": name, "M": M, "K": K, "N": N,
                          "launches": reps, "us_per_launch": round(us, 2), "TFLOP/s": round(flop / us / 1e6, 1),
                          "frac_of_fp16_peak": round(flop / us / 1e6 / PEAK_FP16_TFLOPS, 3)}), flush=True)
        del x, wt


def synthetic_model(ctx, q, n_layers, vocab, seed=0, scale=0.005, flags=0):
    """Random weights of the model's shapes, written straight into the device layouts the forward
    reads (no file, no packing step): a Q6_K token table of `vocab` rows (random codes, int8
    scales 1..15 with random sign, d ~ 0.006), norm gains 1 + 0.1 N(0,1), and per layer the four
    q4_0-tile32-compact projections as random 20-byte records (f16 scale ~ `scale`, two zero
    bytes, nibbles 1..15 so the weights q - 8 are zero-mean).  Returns (model, buffers)."""
    rng = np.random.default_rng(seed)
    bufs = []

    def up(a):
        b = ctx.upload(np.ascontiguousarray(a))
        bufs.append(b)
        return b

    def compact(K, N):
        nbytes = q.lib().qattn_q4_compact_bytes(K, N)
        rec = np.empty((nbytes // 20, 20), np.uint8)
        rec[:, 0:2] = (scale * rng.uniform(0.5, 1.5, (len(rec), 1))).astype(np.float16).view(np.uint8)
        rec[:, 2:4] = 0
        rec[:, 4:] = (rng.integers(1, 16, (len(rec), 16)) | rng.integers(1, 16, (len(rec), 16)) << 4).astype(np.uint8)
        return (up(rec).ptr, nbytes)

    gain = lambda n: up((1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)).ptr
    blocks = rng.integers(0, 256, (vocab, 4, 210), dtype=np.uint8)
    blocks[..., 192:208] = (rng.integers(1, 16, (vocab, 4, 16)) * rng.choice([-1, 1], (vocab, 4, 16))).astype(np.int8).view(np.uint8)
    blocks[..., 208:210] = (0.006 * rng.uniform(0.5, 1.5, (vocab, 4, 1))).astype(np.float16).view(np.uint8)
    table = up(blocks)
    layers = [{"attn_norm": gain(1024), "attn_qkv": compact(1024, 4096), "attn_q_norm": gain(128),
               "attn_k_norm": gain(128), "attn_output": compact(2048, 1024), "ffn_norm": gain(1024),
               "ffn_gate_up": compact(1024, 6144), "ffn_down": compact(3072, 1024)} for _ in range(n_layers)]
    model = ctx.model((table.ptr, blocks.nbytes), gain(1024), layers, flags=flags)
    return model, bufs


MODEL_VOCAB = 151669  # Qwen3 tokenizer vocabulary (the reference's token_embd rows)


def retained_pairs_sparse(L, prefix=176, window=432):
    """Retained (q, k) pairs of one sequence under the model's prefix + local mask (ops.ts:206):
    every key up to q while q < prefix + window, then exactly prefix + window keys per query."""
    n = min(L, prefix + window)
    return n * (n + 1) // 2 + max(0, L - prefix - window) * (prefix + window)


def model_timing(reps, names=("full", "sparse", "cfg4", "cfg1", "cfg3")):
    """The whole 28-layer forward (f4; not the headline metric): qattn_model_plan_run -- embedding
    lookup, 28 x (norms, four Q4_0 projections, QK-norm + RoPE, attention, SwiGLU), pool -- on
    synthetic weights at the BASELINE packings, random token ids over the full vocabulary.
    `reps` forwards between HIP events per config after 2 warm-up runs, then one profiled run for
    the per-stage split (the reference's profile() stages, model.ts:157-168).  FLOP counts the
    projections (2 x 15.73 M per token per layer) and the attention pairs."""
    q = load_binding()
    ctx = q.Context(0)
    model, bufs = synthetic_model(ctx, q, LAYERS, MODEL_VOCAB)
    rng = np.random.default_rng(1)
    gemm_flop_per_token = 2.0 * (1024 * 4096 + 2048 * 1024 + 1024 * 6144 + 3072 * 1024) * LAYERS
    for name in names:
        lengths = lengths_of(name)
        cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
        T = int(cu[-1])
        mask_pairs = sum(retained_pairs_sparse(L) for L in lengths)
        ids = rng.integers(0, MODEL_VOCAB, T).astype(np.int32)
        plan = model.plan(T, len(lengths))
        out = ctx.alloc(len(lengths) * 1024 * 4)
        for _ in range(2):
            plan.run(ids, cu, out.ptr)
        e0, e1 = ctx.event(), ctx.event()
        ctx.synchronize()
        e0.record()
        for _ in range(reps):
            plan.run(ids, cu, out.ptr)
        e1.record()
        ctx.synchronize()
        ms = e0.elapsed_ms(e1) / reps
        stages = plan.profile(ids, cu, out.ptr)
        emb = out.read(np.float32, (len(lengths), 1024))
        flop = gemm_flop_per_token * T + 8192.0 * mask_pairs * LAYERS
        print(json.dumps({"path": "qattn_model_plan_run (28 layers)", "workload": name, "sequences": len(lengths),
                          "tokens": T, "runs": reps, "ms_per_forward": round(ms, 3),
                          "tokens_per_s": round(T / (ms / 1e3), 1),
                          "requests_per_s": round(len(lengths) / (ms / 1e3), 1),
                          "TFLOP/s": round(flop / (ms / 1e3) / 1e12, 1),
                          "frac_of_fp16_peak": round(flop / (ms / 1e3) / 1e12 / PEAK_FP16_TFLOPS, 3),
                          "stage_ms": {k: round(v, 3) for k, v in stages.items()},
                          "embeddings_finite": bool(np.isfinite(emb).all()),
                          "embedding_norms": [round(float(x), 4) for x in np.linalg.norm(emb, axis=1)[:4]]}),
              flush=True)
        out.free()
        plan.destroy()
        e0.destroy()
        e1.destroy()
    model.destroy()
    for b in bufs:
        b.free()
    ctx.close()


def timeline_report(names):
    """Per-workgroup phase timeline of the attention launch (qattn_debug_run_timeline: the
    kernel's timeline variant stamps s_memrealtime, 100 MHz, at fixed points).  Each workload's
    28 layers run 3 times back to back, then layers 0..26 once more and layer 27 under the
    timeline, so its inputs are HBM-resident like every timed launch's.  One JSON line per
    workload: slot start / prologue / end spread, and per entry phase durations (median, mean,
    p90 in us) over the slots' first 15 entries."""
    q = load_binding()
    ctx = q.Context(0)
    for name in names:
        w = Workload(ctx, q, name)
        for _ in range(3):
            w.encode_all()
        for r in w.runs[:-1]:
            r.encode()
        st = w.runs[-1].timeline().astype(np.int64)
        d = w.runs[-1].desc
        entries, _ = q.plan_describe(d)
        slots = q.plan_slots(d)
        nslots = len(slots) - 1
        assert st.shape[0] == nslots, (st.shape, nslots)
        used = [b for b in range(nslots) if slots[b + 1] > slots[b]]
        t0 = min(st[b, 0] for b in used)
        us = lambda a, b: ((a - b) % (1 << 32)) * 0.01
        ph = {k: [] for k in ("tile_body_per_tile", "entry_top_to_first_barrier", "last_tile_next_loads_issue",
                              "last_tile_softmax_and_last_pv", "handover_wait", "stage_rows_and_next_s0",
                              "row_stores")}
        starts, prologue, ends, dur = [], [], [], []
        for b in used:
            starts.append(us(st[b, 0], t0))
            prologue.append(us(st[b, 1], st[b, 0]))
            ends.append(us(st[b, 127], t0))
            dur.append(us(st[b, 127], st[b, 0]))
            for e in range(min(15, slots[b + 1] - slots[b])):
                t = st[b, 2 + 8 * e: 10 + 8 * e]
                n = int(entries[slots[b] + e][5] - entries[slots[b] + e][4])
                if n >= 2:
                    ph["tile_body_per_tile"].append(us(t[2], t[1]) / (n - 1))
                ph["entry_top_to_first_barrier"].append(us(t[1], t[0]))
                ph["last_tile_next_loads_issue"].append(us(t[3], t[2]))
                ph["last_tile_softmax_and_last_pv"].append(us(t[4], t[3]))
                ph["handover_wait"].append(us(t[5], t[4]))
                ph["stage_rows_and_next_s0"].append(us(t[6], t[5]))
                ph["row_stores"].append(us(t[7], t[6]))
        stat = lambda a: {"median": round(float(np.median(a)), 3), "mean": round(float(np.mean(a)), 3),
                          "p90": round(float(np.percentile(a, 90)), 3)} if len(a) else None
        print(json.dumps({"timeline": "attn_fwd_kernel", "workload": name, "slots": len(used),
                          "entries": int(slots[-1]), "split_items": int(w.info.split_items),
                          "slot_start_us": stat(starts), "prologue_us": stat(prologue), "slot_end_us": stat(ends),
                          "slot_end_max_us": round(max(ends), 3), "slot_duration_us": stat(dur),
                          "per_entry_us": {k: stat(v) for k, v in ph.items()}}), flush=True)
        w.free()
    ctx.close()


MATRIX_LENGTHS = (15, 50, 150, 500, 1500, 5000)


def model_matrix(reps):
    """The reference's measurement matrix (README.md:14-21, protocol src/main.ts:302-321) on the
    28-layer forward: one request and 16 concurrent requests of 15, 50, 150, 500, 1,500 and 5,000
    tokens, each 16-request round one packed batch (5,000 tokens: four batches of four, as the
    reference runs it), with the batch-invariant plan the engine uses and the model's 176 + 432
    mask (full causal up to 608 tokens).  Synthetic weights of the real shapes, random token ids;
    `reps` forwards between HIP events after 2 warm-ups, then one profiled run for the stage split.
    Device time only: no tokenizer, no host round trip per request."""
    q = load_binding()
    ctx = q.Context(0)
    model, bufs = synthetic_model(ctx, q, LAYERS, MODEL_VOCAB, flags=FLAG_BATCH_INVARIANT)
    rng = np.random.default_rng(2)
    gemm_flop_per_token = 2.0 * (1024 * 4096 + 2048 * 1024 + 1024 * 6144 + 3072 * 1024) * LAYERS
    plan = model.plan(16 * 1500, 16)  # the largest batch: 16 x 1,500 tokens
    out = ctx.alloc(16 * 1024 * 4)
    e0, e1 = ctx.event(), ctx.event()
    for L in MATRIX_LENGTHS:
        for conc in (1, 16):
            per_batch = 4 if (L == 5000 and conc == 16) else conc
            batches = conc // per_batch
            lengths = [L] * per_batch
            cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
            T = int(cu[-1])
            ids = rng.integers(0, MODEL_VOCAB, T).astype(np.int32)
            for _ in range(2):
                plan.run(ids, cu, out.ptr)
            ctx.synchronize()
            e0.record()
            for _ in range(reps * batches):
                plan.run(ids, cu, out.ptr)
            e1.record()
            ctx.synchronize()
            ms_round = e0.elapsed_ms(e1) / reps  # one round of `conc` requests
            stages = plan.profile(ids, cu, out.ptr)
            flop = batches * (gemm_flop_per_token * T + 8192.0 * sum(retained_pairs_sparse(x) for x in lengths) * LAYERS)
            print(json.dumps({"path": "qattn_model_plan_run (28 layers)", "tokens": L, "concurrency": conc,
                              "batches_per_round": batches, "runs": reps, "ms_per_round": round(ms_round, 3),
                              "requests_per_s": round(conc / (ms_round / 1e3), 1),
                              "tokens_per_s": round(conc * L / (ms_round / 1e3), 1),
                              "TFLOP/s": round(flop / (ms_round / 1e3) / 1e12, 1),
                              "frac_of_fp16_peak": round(flop / (ms_round / 1e3) / 1e12 / PEAK_FP16_TFLOPS, 3),
                              "stage_ms_one_batch": {k: round(v, 3) for k, v in stages.items()}}), flush=True)
    e0.destroy()
    e1.destroy()
    out.free()
    plan.destroy()
    model.destroy()
    for b in bufs:
        b.free()
    ctx.close()


def kernel_sources_sha():
    """Hash of the code the attention launch is built from (kernels and planner, with comments
    and whitespace removed): HBM traffic measured on other code (profiles/traffic.json) is not
    reported as this build's."""
    h = hashlib.sha256()
    for f in ("attn_fwd.hip", "attn_common.h", "planner.h", "planner.cpp"):
        with open(os.path.join(PKG, "csrc", f), encoding="utf-8") as fh:
            text = re.sub(r"/\*.*?\*/", " ", fh.read(), flags=re.S)
        text = re.sub(r"//[^\n]*", " ", text)
        h.update(" ".join(text.split()).encode())
    return h.hexdigest()[:16]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=sorted(SETS), default="both")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the other BASELINE configs in the breakdown")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 plain device copies of MIB MiB (torch copy_) and exit: the "
                         "known-size reference for rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    ap.add_argument("--pool", type=int, default=0, metavar="N",
                    help="only time N launches of the last-token pool kernel per width and exit")
    ap.add_argument("--q4", type=int, default=0, metavar="N",
                    help="only time N launches of the Q4_0 dequant-GEMM per projection shape and exit")
    ap.add_argument("--q4-m", default="8000", metavar="M[,M...]",
                    help="token counts for --q4 (default 8000, one 16 x 500 packing)")
    ap.add_argument("--dense-gemm", type=int, default=0, metavar="N",
                    help="only time N launches of torch.matmul (hipBLASLt) on dense fp16 operands of each "
                         "--q4-m projection shape (a reference ceiling, without libqattn.so) and exit")
    ap.add_argument("--rope", type=int, default=0, metavar="N",
                    help="only time N launches of the fused QK-norm + RoPE producer and exit")
    ap.add_argument("--model", type=int, default=0, metavar="N",
                    help="only time N runs of the whole 28-layer forward (synthetic weights) per config and exit")
    ap.add_argument("--timeline", action="store_true",
                    help="only print the attention kernel's per-workgroup phase timeline (qattn_debug_run_timeline) "
                         "for the headline workloads and exit")
    ap.add_argument("--model-matrix", type=int, default=0, metavar="N",
                    help="only run the reference's single / 16-request matrix at 15..5000 tokens through "
                         "the 28-layer forward, N rounds each, and exit")
    args = ap.parse_args()
    if args.timeline:
        timeline_report(["full", "sparse", "sparse_bi"] if args.workload == "both" else [args.workload])
        return
    if args.model_matrix:
        model_matrix(args.model_matrix)
        return
    if args.model:
        if args.workload == "both":
            model_timing(args.model)
        else:
            model_timing(args.model, (args.workload,))
        return
    if args.rope:
        rope_timing(args.rope)
        return
    if args.q4:
        q4_timing(args.q4, tuple(int(m) for m in args.q4_m.split(",")))
        return
    if args.dense_gemm:
        dense_gemm_timing(args.dense_gemm, tuple(int(m) for m in args.q4_m.split(",")))
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
    extra = [] if (args.no_extra or args.workload != "both") else [Workload(ctx, q, n) for n in EXTRA]
    for w in wls + extra:
        i = w.info
        log(f"{w.name}: {w.desc_text}: tokens {i.tokens}, pairs {i.pairs}, work items {i.work_items}, "
            f"flops/launch {i.flops:.4e}, bytes/launch {i.bytes:.4e}, tile waste {i.tile_pairs / i.pairs:.3f}, "
            f"split items {i.split_items}")

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

    # ---- per-workload launch durations on the same basis as `value`: each workload's 28 layer
    # launches, `reps` rounds back to back between one pair of events on the launch stream, with
    # no synchronisation inside (so no idle gap and no clock ramp between launches), divided by
    # the launch count.  The headline workloads' figures times 28 should add up to ms_per_step.
    reps = max(3, min(args.steps, 10))
    per = {}
    ea, eb = ctx.event(), ctx.event()
    for w in wls + extra:
        for _ in range(2):
            w.encode_all()
        ctx.synchronize()
        ea.record()
        for _ in range(reps):
            w.encode_all()
        eb.record()
        ctx.synchronize()
        per[w.name] = ea.elapsed_ms(eb) / (reps * len(w.runs))
    ea.destroy()
    eb.destroy()

    tokens_per_step = sum(w.tokens for w in wls) * LAYERS
    value = tokens_per_step / (ms_per_step / 1e3)
    total_flops = sum(w.info.flops for w in wls) * LAYERS
    total_bytes = sum(w.info.bytes for w in wls) * LAYERS
    kern_ms_step = sum(per[w.name] * LAYERS for w in wls)
    breakdown = {}
    for w in wls + extra:
        avg = per[w.name]
        ai = w.info.flops / w.info.bytes
        attainable = min(PEAK_FP16_TFLOPS * 1e12, ai * PEAK_HBM_MEASURED_GBS * 1e9)
        breakdown[w.name] = {
            "workload": w.desc_text,
            "headline": w in wls,
            "kernel_avg_us": round(avg * 1e3, 3),
            "tokens_per_s": round(w.tokens / (avg / 1e3), 1),
            "tflops": round(w.info.flops / (avg / 1e3) / 1e12, 2),
            "mfma_frac": round(w.info.flops / (avg / 1e3) / 1e12 / PEAK_FP16_TFLOPS, 4),
            "gbs": round(w.info.bytes / (avg / 1e3) / 1e9, 1),
            "hbm_frac": round(w.info.bytes / (avg / 1e3) / 1e9 / PEAK_HBM_GBS, 4),
            "attainable_frac": round(w.info.flops / (avg / 1e3) / attainable, 4),
            "split_items": w.info.split_items,
        }
        log(f"{w.name}: kernel avg {avg * 1e3:.2f} us, {breakdown[w.name]}")
    # The roofline figure on value's own basis: the step's algorithmic FLOPs over the step time.
    achieved = total_flops / (ms_per_step / 1e3) / 1e12
    log(f"basis check: headline launches {kern_ms_step:.4f} ms per step back to back vs the step's "
        f"{ms_per_step:.4f} ms")

    traffic, traffic_note = None, "no profiles/traffic.json"
    tpath = os.path.join(REPO, "profiles", "traffic.json")
    if os.path.exists(tpath):
        try:
            tj = json.load(open(tpath))
            if tj.get("sources_sha") == kernel_sources_sha():
                traffic = tj.get(args.workload)
                traffic_note = ("HBM bytes per launch (mean over the step's launches), rocprofv3 "
                                "FETCH_SIZE x2.0 + WRITE_SIZE x1.0 (copy-calibrated), profiles/traffic.json, "
                                "measured on these kernel sources")
            else:
                traffic_note = ("profiles/traffic.json was measured on other kernel sources "
                                f"({tj.get('sources_sha')} vs {kernel_sources_sha()}): not reported")
        except (ValueError, OSError):
            traffic = None
    for w in extra:
        w.free()

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
            "basis": "the step: algorithmic FLOPs of the step's 56 launches / ms_per_step (as value)",
            "launches_ms_per_step": round(kern_ms_step, 4),
            "traffic": traffic,
            "traffic_note": traffic_note,
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
