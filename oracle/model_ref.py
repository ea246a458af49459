"""CPU restatement of the Qwen3-Embedding-0.6B forward around the attention path.

TEST INFRASTRUCTURE ONLY.  Imported by tests/ and bench.py's cpu_baseline leg, as the checker.
The product never imports it.

Reference behaviour restated (paths relative to the reference checkout):
  src/gguf/quantization.ts:46-70   Q6_K block decoder (q6k_rows)
  src/webgpu/ops.ts:381-412        Q6_K embedding shader, element by element (q6k_rows_shader_form)
  src/webgpu/ops.ts:21-57          residual add + RMSNorm (rmsnorm)
  src/webgpu/ops.ts:74-89          SwiGLU (swiglu)
  src/webgpu/model.ts:49-139       the execution plan: stage order and buffers (forward)
and, through oracle.py, the Q4_0 compact dequant-GEMM, the QK-norm + RoPE producer, the
attention and the last-token pool.

Every stage rounds its output to fp16 where the reference stores fp16 (x, normalized, qkvRaw, q,
k, attention, delta, gateUp, ffn); arithmetic inside a stage is f64, so the device result differs
from this one only by fp32 rounding and summation order inside a stage.
"""
import numpy as np

import oracle as orc

HIDDEN, INTERMEDIATE, Q_WIDTH, KV_WIDTH = 1024, 3072, 2048, 1024
QKV_WIDTH = Q_WIDTH + 2 * KV_WIDTH
Q6K_BLOCK_BYTES = 210


# ---- Q6_K -------------------------------------------------------------------------------------

def q6k_rows(table, ids, width=HIDDEN):
    """Rows `ids` of a Q6_K table (uint8 bytes, width/256 blocks of 210 per row) as the float
    values d * scale * (q - 32) of quantization.ts:46-70 (f64, before any fp16 rounding).

    Block layout: ql[128] | qh[64] | int8 scales[16] | f16 d.  Output index 128 h + 32 j + l
    (h < 2, j < 4, l < 32) takes the low nibble of ql[64h + l] (j = 0), of ql[64h + l + 32] (j = 1),
    their high nibbles (j = 2, 3), high bits (qh[32h + l] >> 2j) & 3, scale[8h + l//16 + 2j]."""
    table = np.frombuffer(bytes(table), np.uint8) if not isinstance(table, np.ndarray) else table
    nb = width // 256
    blocks = table.reshape(-1, nb, Q6K_BLOCK_BYTES)[np.asarray(ids, np.int64)]   # [n, nb, 210]
    ql = blocks[..., 0:128].astype(np.int32)
    qh = blocks[..., 128:192].astype(np.int32)
    scales = blocks[..., 192:208].view(np.int8).astype(np.float64)
    d = blocks[..., 208:210].copy().view(np.float16)[..., 0].astype(np.float64)     # [n, nb]
    out = np.empty(blocks.shape[:2] + (256,), np.float64)
    lane = np.arange(32)
    for h in range(2):
        high = qh[..., 32 * h + lane]
        low_a = ql[..., 64 * h + lane]
        low_b = ql[..., 64 * h + lane + 32]
        codes = [(low_a & 15) | ((high & 3) << 4),
                 (low_b & 15) | (((high >> 2) & 3) << 4),
                 (low_a >> 4) | (((high >> 4) & 3) << 4),
                 (low_b >> 4) | (((high >> 6) & 3) << 4)]
        for j, q in enumerate(codes):
            sc = scales[..., 8 * h + lane // 16 + 2 * j]
            out[..., 128 * h + 32 * j + lane] = d[..., None] * sc * (q - 32)
    return out.reshape(len(blocks), width)


def q6k_rows_shader_form(table, ids, width=HIDDEN):
    """The same rows through the embedding shader's own index arithmetic (ops.ts:390-401),
    one element at a time: an independent restatement the vectorised decoder is checked against."""
    table = np.frombuffer(bytes(table), np.uint8) if not isinstance(table, np.ndarray) else table
    nb = width // 256
    out = np.empty((len(ids), width), np.float64)
    for r, tok in enumerate(ids):
        for column in range(width):
            block = (int(tok) * nb + column // 256) * Q6K_BLOCK_BYTES
            within = column & 255
            half, position = within // 128, within & 127
            quadrant, lane = position // 32, position & 31
            low = int(table[block + half * 64 + lane + (quadrant & 1) * 32])
            low = low >> 4 if quadrant >= 2 else low & 15
            high = (int(table[block + 128 + half * 32 + lane]) >> (quadrant * 2)) & 3
            q = (low | (high << 4)) - 32
            s = int(table[block + 192 + half * 8 + lane // 16 + quadrant * 2])
            s = s - 256 if s >= 128 else s
            d = float(np.frombuffer(bytes(table[block + 208:block + 210]), np.float16)[0])
            out[r, column] = d * s * q
    return out


def embed(table, ids, width=HIDDEN):
    """The embedding shader's fp16 rows: f16(f32(f32(d) * scale) * q) (ops.ts:401, f32 math)."""
    v = q6k_rows(table, ids, width)
    return v.astype(np.float32).astype(np.float16)


# ---- row-wise stages ---------------------------------------------------------------------------

def rmsnorm(x, residual, weight, eps=1e-6):
    """ops.ts:33-56 on fp16 rows: returns (x', normalized), both fp16.  With a residual,
    v = x + r, x' = f16(v) and the sum of squares takes the unrounded v; normalized =
    f16(x' * inv * w) with inv = 1 / sqrt(mean(v^2) + eps)."""
    xf = np.asarray(x, np.float16).astype(np.float64)
    v = xf + np.asarray(residual, np.float16).astype(np.float64) if residual is not None else xf
    xn = v.astype(np.float16)
    inv = 1.0 / np.sqrt(np.mean(v * v, axis=1, keepdims=True) + eps)
    out = xn.astype(np.float64) * inv * np.asarray(weight, np.float32).astype(np.float64)[None, :]
    return xn, out.astype(np.float16)


def swiglu(gate_up, width=INTERMEDIATE):
    """ops.ts:81-88: f16(silu(g) * u) with g, u the two halves of each row."""
    gu = np.asarray(gate_up, np.float16).astype(np.float64)
    g, u = gu[:, :width], gu[:, width:2 * width]
    return (g / (1.0 + np.exp(-g)) * u).astype(np.float16)


def linear(x, weight):
    """A compact Q4_0 projection: weight = (packed bytes, K, N); fp16 rows out."""
    packed, k, n = weight
    return orc.q4_matmul(x, packed, k, n).astype(np.float16)


# ---- the forward ---------------------------------------------------------------------------------

def forward(weights, ids, cu_seqlens, eps=1e-6, theta=1e6, kind=orc.MASK_PREFIX_LOCAL, prefix=176,
            window=432, trace=None):
    """Embeddings (f64 [nseq, 1024]) of a packed varlen batch, in the reference's stage order
    (model.ts:117-131).  `weights`: {"token_embd": bytes, "output_norm": f32 [1024],
    "layers": [ {attn_norm, attn_q_norm, attn_k_norm, ffn_norm: f32 arrays;
                 attn_qkv, attn_output, ffn_gate_up, ffn_down: (packed, K, N)} ]}.
    `trace`, if a dict, receives the residual stream after each layer ("x{l}")."""
    cu = np.asarray(cu_seqlens, np.int32)
    layers = weights["layers"]
    x = embed(weights["token_embd"], ids)
    x, normalized = rmsnorm(x, None, layers[0]["attn_norm"], eps)
    for li, lw in enumerate(layers):
        qkv = linear(normalized, lw["attn_qkv"])                               # qkvRaw [T, 4096]
        raw = qkv.view(np.uint16).copy()
        q = np.ascontiguousarray(raw[:, :Q_WIDTH])
        k = np.ascontiguousarray(raw[:, Q_WIDTH:Q_WIDTH + KV_WIDTH])
        orc.qk_norm_rope(q, cu, heads=16, weight=lw["attn_q_norm"], eps=eps, theta=theta)
        orc.qk_norm_rope(k, cu, heads=8, weight=lw["attn_k_norm"], eps=eps, theta=theta)
        v = np.ascontiguousarray(raw[:, Q_WIDTH + KV_WIDTH:])
        attn = orc.attention_exact(q, k, v, cu, kind=kind, prefix=prefix, window=window)
        attn = attn.reshape(len(attn), Q_WIDTH).astype(np.float16)
        delta = linear(attn, lw["attn_output"])
        x, normalized = rmsnorm(x, delta, lw["ffn_norm"], eps)
        ffn = swiglu(linear(normalized, lw["ffn_gate_up"]))
        delta = linear(ffn, lw["ffn_down"])
        nxt = layers[li + 1]["attn_norm"] if li + 1 < len(layers) else weights["output_norm"]
        x, normalized = rmsnorm(x, delta, nxt, eps)
        if trace is not None:
            trace[f"x{li}"] = x.copy()
    return orc.pool_last_l2(normalized, cu, HIDDEN)


# ---- synthetic weights --------------------------------------------------------------------------

def q40_rows(rng, n, k, scale):
    """n GGML Q4_0 rows of k values: f16 scale (scale * U[0.5, 1.5)) and nibbles uniform in
    1..15, so the weights q - 8 are zero-mean (uniform 0..15 has mean -0.5, which makes random
    layers amplify the rows' common component until fp16 overflows)."""
    kb = k // 32
    rows = np.zeros((n, kb, 18), np.uint8)
    d = (scale * rng.uniform(0.5, 1.5, (n, kb))).astype(np.float16)
    rows[..., 0:2] = d.view(np.uint8).reshape(n, kb, 2)
    lo = rng.integers(1, 16, (n, kb, 16))
    hi = rng.integers(1, 16, (n, kb, 16))
    rows[..., 2:] = (lo | (hi << 4)).astype(np.uint8)
    return rows.reshape(-1)


def q6k_table(rng, vocab, width=HIDDEN, d=0.006):
    """A random Q6_K table: random codes, int8 scales in [1, 15] with random sign, f16 d."""
    nb = width // 256
    blocks = rng.integers(0, 256, (vocab, nb, Q6K_BLOCK_BYTES), dtype=np.uint8)
    sc = rng.integers(1, 16, (vocab, nb, 16)) * rng.choice([-1, 1], (vocab, nb, 16))
    blocks[..., 192:208] = sc.astype(np.int8).view(np.uint8)
    dd = (d * rng.uniform(0.5, 1.5, (vocab, nb))).astype(np.float16)
    blocks[..., 208:210] = dd.view(np.uint8).reshape(vocab, nb, 2)
    return blocks.reshape(-1)


def synthetic_weights(seed, n_layers, vocab=512, scale=0.005):
    """Random weights of the model's shapes (host arrays), for parity tests and the benchmark:
    a `vocab`-row Q6_K table, gains 1 + 0.1 N(0,1), Q4_0 projections with per-block scales around
    `scale` (the packed QKV and gate/up tensors are the reference's fused parts, model.ts:241-244)."""
    rng = np.random.default_rng(seed)
    gain = lambda n: (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)

    def compact(parts):
        packed, k, n = orc.pack_q40_tile32(parts)
        return (packed, k, n)

    layers = []
    for _ in range(n_layers):
        layers.append({
            "attn_norm": gain(HIDDEN),
            "attn_qkv": compact([(HIDDEN, Q_WIDTH, q40_rows(rng, Q_WIDTH, HIDDEN, scale)),
                                 (HIDDEN, KV_WIDTH, q40_rows(rng, KV_WIDTH, HIDDEN, scale)),
                                 (HIDDEN, KV_WIDTH, q40_rows(rng, KV_WIDTH, HIDDEN, scale))]),
            "attn_q_norm": gain(128),
            "attn_k_norm": gain(128),
            "attn_output": compact([(Q_WIDTH, HIDDEN, q40_rows(rng, HIDDEN, Q_WIDTH, scale))]),
            "ffn_norm": gain(HIDDEN),
            "ffn_gate_up": compact([(HIDDEN, INTERMEDIATE, q40_rows(rng, INTERMEDIATE, HIDDEN, scale)),
                                    (HIDDEN, INTERMEDIATE, q40_rows(rng, INTERMEDIATE, HIDDEN, scale))]),
            "ffn_down": compact([(INTERMEDIATE, HIDDEN, q40_rows(rng, HIDDEN, INTERMEDIATE, scale))]),
        })
    return {"token_embd": q6k_table(rng, vocab), "output_norm": gain(HIDDEN), "layers": layers,
            "vocab": vocab}
