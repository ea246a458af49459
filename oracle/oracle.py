"""ctypes/numpy front end of the CPU oracle (oracle.c).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker.  The product never imports it.

Reference behaviour restated (paths relative to the reference checkout):
  src/webgpu/ops.ts:168-241   tiled flash attention (f16-faithful restatement: tiled16)
  src/webgpu/ops.ts:205-220   causal + 176-prefix/432-window mask
  src/webgpu/ops.ts:104-150   QK RMSNorm + RoPE producer, model.ts:76-83 RoPE table
  src/webgpu/ops.ts:347-379   last-token pool + L2 normalisation (pool_last_l2)
  src/prepacked/format.ts:64-96, src/webgpu/quant-matmul.ts:99-108, 267-307
                              Q4_0 tile32-compact packing and the dequant-GEMM (pack_q40_tile32,
                              q40_compact_weights, q4_matmul)
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# QATTN_ORACLE_LIB selects another build (the sanitizer build of tests/sanitize.sh).
LIB_PATH = os.environ.get("QATTN_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")

MASK_CAUSAL = 0
MASK_PREFIX_LOCAL = 1
HQ, HKV, HD = 16, 8, 128

_lib = None


def build():
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


class _Args(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("q_stride", ctypes.c_int64), ("k_stride", ctypes.c_int64),
        ("v_stride", ctypes.c_int64), ("v_offset", ctypes.c_int64),
        ("cu_seqlens", ctypes.c_void_p), ("nseq", ctypes.c_int32),
        ("kind", ctypes.c_int32), ("prefix", ctypes.c_int32), ("window", ctypes.c_int32),
    ]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        u16, f32, u64, i64, i32 = (ctypes.c_uint16, ctypes.c_float, ctypes.c_uint64,
                                   ctypes.c_int64, ctypes.c_int32)
        vp = ctypes.c_void_p
        sig = {
            "orc_f32_to_f16": (u16, [f32]),
            "orc_f16_to_f32": (f32, [u16]),
            "orc_ref_float_to_half": (u16, [f32]),
            "orc_ref_half_to_float": (ctypes.c_double, [u16]),
            "orc_rand_u64": (u64, [u64, u64]),
            "orc_normal": (ctypes.c_double, [u64, u64]),
            "orc_seed": (u64, [ctypes.c_uint32] * 3),
            "orc_gen_normal_f16": (None, [u64, i64, vp]),
            "orc_rope_table": (None, [i32, ctypes.c_double, vp, vp]),
            "orc_qk_norm_rope": (None, [vp, i64, i64, i32, vp, i32, vp, ctypes.c_double,
                                        ctypes.c_double]),
            "orc_gen_lengths": (None, [u64, i32, i32, i32, vp]),
            "orc_retained": (ctypes.c_int, [i64, i64, i64, i32, i64, i64]),
            "orc_mask_bits": (None, [i32, i32, i32, i32, vp]),
            "orc_mask_pairs": (i64, [i32, i32, i32, i32]),
            "orc_ref_tile_skipped": (ctypes.c_int, [i64, i64, i64]),
            "orc_attention_exact": (None, [ctypes.POINTER(_Args), vp, i64, vp]),
            "orc_attention_tiled16": (None, [ctypes.POINTER(_Args), vp, i64]),
            "orc_attention_tiled16_tiles": (None, [ctypes.POINTER(_Args), i32, i64, i64, i64,
                                                    vp, i64]),
            "orc_set_threads": (None, [i32]),
            "orc_get_threads": (i32, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


# ---- fp16 ----------------------------------------------------------------------------------

def f32_to_f16(x):
    return lib().orc_f32_to_f16(float(x))


def f16_to_f32(h):
    return lib().orc_f16_to_f32(int(h))


def ref_float_to_half(x):
    return lib().orc_ref_float_to_half(float(x))


def ref_half_to_float(h):
    return lib().orc_ref_half_to_float(int(h))


# ---- generator -----------------------------------------------------------------------------

def seed(config, layer, tensor):
    return lib().orc_seed(config, layer, tensor)


def normal_f16(seed_value, n):
    out = np.empty(n, dtype=np.uint16)
    lib().orc_gen_normal_f16(seed_value, n, _ptr(out))
    return out


def rope_table(npos, theta=1e6):
    c = np.empty((npos, 64), dtype=np.float32)
    s = np.empty((npos, 64), dtype=np.float32)
    lib().orc_rope_table(npos, theta, _ptr(c), _ptr(s))
    return c, s


def qk_norm_rope(x, cu_seqlens, heads, col0=0, weight=None, eps=1e-6, theta=1e6):
    """In place on a uint16 [T, stride] array."""
    assert x.dtype == np.uint16 and x.flags.c_contiguous
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    w = None if weight is None else np.ascontiguousarray(weight, dtype=np.float32)
    lib().orc_qk_norm_rope(_ptr(x), x.shape[1], col0, heads, _ptr(cu), len(cu) - 1,
                           None if w is None else _ptr(w), eps, theta)
    return x


def pool_last_l2(x, cu_seqlens, width=None):
    """Last-token pool + L2 norm (LastTokenPoolKernel, src/webgpu/ops.ts:347-379), exact in f64.

    x: fp16 rows [T, >= width]; sequence i pools row cu_seqlens[i+1]-1 (the reference's row
    b*S + lengths[b]-1 of its padded layout, ops.ts:357): out = x / sqrt(sum x^2) over the first
    `width` columns (ops.ts:358-363), as f64.  No epsilon, as in the reference: an all-zero row
    gives NaN (0 * inverseSqrt(0)).  An empty sequence (which the reference never forms) gives
    zeros, the library's documented choice."""
    x = np.asarray(x)
    width = x.shape[1] if width is None else width
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    out = np.zeros((len(cu) - 1, width), dtype=np.float64)
    for i in range(len(cu) - 1):
        if cu[i + 1] == cu[i]:
            continue
        row = x[cu[i + 1] - 1, :width].astype(np.float64)
        with np.errstate(divide="ignore", invalid="ignore"):
            out[i] = row * (1.0 / np.sqrt(np.sum(row * row)))
    return out


def pack_q40_tile32(parts):
    """packQ40Tile32 (src/prepacked/format.ts:64-96): GGML Q4_0 rows (18-byte blocks: f16 scale,
    16 quant bytes; element j of a block in the low nibble of byte j, element j+16 in its high
    nibble) of one or more parts (k, n, bytes), stacked by rows, into 20-byte records (scale,
    2 zero bytes, the 16 quant bytes) ordered ((n // 32) * (k // 32) + k_block) * 32 + n % 32.
    Rows past n in the last 32-row tile stay zero.  Returns (bytes as uint8, k, n)."""
    k = parts[0][0]
    if k % 32:
        raise ValueError(f"K={k} is not divisible by 32")
    rows = []
    for pk, pn, pbytes in parts:
        if pk != k:
            raise ValueError("mismatched K dimensions")
        pbytes = np.frombuffer(bytes(pbytes), np.uint8)
        if pbytes.size != pn * (k // 32) * 18:
            raise ValueError("part size")
        rows.append(pbytes.reshape(pn, k // 32, 18))
    src = np.concatenate(rows, axis=0)
    n, kb = src.shape[0], k // 32
    tiles = -(-n // 32)
    out = np.zeros((tiles, kb, 32, 20), np.uint8)
    for r in range(n):
        out[r // 32, :, r % 32, 0:2] = src[r, :, 0:2]
        out[r // 32, :, r % 32, 4:20] = src[r, :, 2:18]
    return out.reshape(-1), k, n


def q40_compact_weights(packed, k, n):
    """The fp16 weights W[n, k] a tile32-compact tensor holds, as the reference's compact shaders
    dequantise them (quant-matmul.ts:99-108, 276-282): f16(scale) * (q - 8), rounded to f16 (the
    f32 product is exact, so this equals the shader's f16 multiply)."""
    kb = k // 32
    rec = np.asarray(packed, np.uint8).reshape(-1, kb, 32, 20)
    scale = rec[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float32)    # [tiles, kb, 32]
    q = rec[..., 4:20]
    lo = (q & 15).astype(np.float32) - 8.0
    hi = (q >> 4).astype(np.float32) - 8.0
    vals = np.concatenate([lo, hi], axis=-1) * scale[..., None]                   # [tiles, kb, 32, 32]
    w = vals.transpose(0, 2, 1, 3).reshape(-1, k)                                 # rows tile*32 + r
    return w[:n].astype(np.float16)


def q4_matmul(x, packed, k, n):
    """Y = X W^T exactly (f64) for fp16 X [m, k] and the tile32-compact weights W [n, k]: the
    compact batch matmul's result (quant-matmul.ts:267-307) without its f16 accumulation."""
    w = q40_compact_weights(packed, k, n).astype(np.float64)
    return np.asarray(x, np.float16).astype(np.float64) @ w.T


def gen_lengths(seed_value, n, lo=10, hi=150):
    out = np.empty(n, dtype=np.int32)
    lib().orc_gen_lengths(seed_value, n, lo, hi, _ptr(out))
    return out


def gen_qkv(config, layer, cu_seqlens):
    """Deterministic Q, K, V (uint16 fp16 bits) for packed varlen tokens.

    Q [T,16,128] and K [T,8,128]: N(0,1) -> f16, per-head RMSNorm (unit gain, eps 1e-6), RoPE
    theta 1e6 at per-sequence positions -> f16.  V [T,8,128]: N(0,1) -> f16.
    """
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    T = int(cu[-1])
    q = normal_f16(seed(config, layer, 0), T * HQ * HD).reshape(T, HQ * HD)
    k = normal_f16(seed(config, layer, 1), T * HKV * HD).reshape(T, HKV * HD)
    v = normal_f16(seed(config, layer, 2), T * HKV * HD).reshape(T, HKV * HD)
    qk_norm_rope(q, cu, HQ)
    qk_norm_rope(k, cu, HKV)
    return q, k, v


# ---- mask ----------------------------------------------------------------------------------

def retained(q, k, S, kind=MASK_PREFIX_LOCAL, P=176, W=432):
    return bool(lib().orc_retained(q, k, S, kind, P, W))


def mask_bits(L, kind=MASK_PREFIX_LOCAL, P=176, W=432):
    words = (L + 31) // 32
    out = np.zeros((L, words), dtype=np.uint32)
    if L:
        lib().orc_mask_bits(L, kind, P, W, _ptr(out))
    return out


def mask_pairs(L, kind=MASK_PREFIX_LOCAL, P=176, W=432):
    return int(lib().orc_mask_pairs(L, kind, P, W))


def ref_tile_skipped(S, q_tile_start, key_base):
    return bool(lib().orc_ref_tile_skipped(S, q_tile_start, key_base))


# ---- attention -----------------------------------------------------------------------------

def _args(q, k, v, cu_seqlens, kind, prefix, window, v_offset=0):
    for a in (q, k, v):
        assert a.dtype == np.uint16 and a.flags.c_contiguous and a.ndim == 2
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    a = _Args(_ptr(q).value, _ptr(k).value, _ptr(v).value, q.shape[1], k.shape[1], v.shape[1],
              v_offset, _ptr(cu).value, len(cu) - 1, kind, prefix, window)
    return a, cu


def attention_exact(q, k, v, cu_seqlens, kind=MASK_PREFIX_LOCAL, prefix=176, window=432,
                    rows=None, v_offset=0):
    """f64 O for the given token rows (default all): array [nrows, 16, 128]."""
    a, cu = _args(q, k, v, cu_seqlens, kind, prefix, window, v_offset)
    T = int(cu[-1])
    if rows is None:
        out = np.empty((T, HQ, HD), dtype=np.float64)
        lib().orc_attention_exact(ctypes.byref(a), None, T, _ptr(out))
    else:
        r = np.ascontiguousarray(rows, dtype=np.int64)
        out = np.empty((len(r), HQ, HD), dtype=np.float64)
        if len(r):
            lib().orc_attention_exact(ctypes.byref(a), _ptr(r), len(r), _ptr(out))
    return out


def attention_tiled16(q, k, v, cu_seqlens, kind=MASK_PREFIX_LOCAL, prefix=176, window=432,
                      v_offset=0):
    """f16-faithful restatement of the reference's 16x16 tiled kernel: uint16 [T, 2048]."""
    a, cu = _args(q, k, v, cu_seqlens, kind, prefix, window, v_offset)
    T = int(cu[-1])
    out = np.zeros((T, HQ * HD), dtype=np.uint16)
    lib().orc_attention_tiled16(ctypes.byref(a), _ptr(out), HQ * HD)
    return out


def attention_tiled16_tiles(q, k, v, cu_seqlens, seq, tile_begin, tile_end, tile_step,
                            kind=MASK_PREFIX_LOCAL, prefix=176, window=432, out=None):
    """Restatement over a strided subset of one sequence's 16-query tiles (CPU timing sample)."""
    a, cu = _args(q, k, v, cu_seqlens, kind, prefix, window)
    T = int(cu[-1])
    if out is None:
        out = np.zeros((T, HQ * HD), dtype=np.uint16)
    lib().orc_attention_tiled16_tiles(ctypes.byref(a), seq, tile_begin, tile_end, tile_step,
                                      _ptr(out), HQ * HD)
    return out


def set_threads(n):
    lib().orc_set_threads(int(n))


def get_threads():
    return int(lib().orc_get_threads())


def f16_bits_to_f32(a):
    return np.asarray(a, dtype=np.uint16).view(np.float16).astype(np.float32)
