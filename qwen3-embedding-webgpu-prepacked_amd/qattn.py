"""ctypes binding of libqattn.so (C ABI: include/qattn.h) for Python hosts: the test suite and
bench.py.  The product's own host is the Node engine in js/; this module mirrors the same
operator interface (the reference's CausalAttentionKernel.createRun / encode,
src/webgpu/ops.ts:327-345) so Python callers drive exactly the code Node drives.

There is no fallback: if libqattn.so is missing or no gfx950 device is present, the calls raise.
"""
import ctypes
import os
import subprocess

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
# QATTN_LIB selects another build of the same library (the sanitizer build of tests/sanitize.sh).
LIB_PATH = os.environ.get("QATTN_LIB") or os.path.join(PKG_DIR, "libqattn.so")
HEADER_PATH = os.path.join(REPO_DIR, "include", "qattn.h")

OK, EINVAL, EHIP, ENOMEM, ENODEV = 0, -1, -2, -3, -4
MASK_CAUSAL, MASK_PREFIX_LOCAL = 0, 1
FLAG_BATCH_INVARIANT = 1  # qattn_run_flags
HQ, HKV, HD = 16, 8, 128


class QattnError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f"qattn error {code}: {message}")
        self.code = code


class RunDesc(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("q_row_stride", ctypes.c_int64), ("k_row_stride", ctypes.c_int64),
        ("v_row_stride", ctypes.c_int64), ("o_row_stride", ctypes.c_int64),
        ("v_offset", ctypes.c_int64),
        ("cu_seqlens", ctypes.c_void_p), ("nseq", ctypes.c_int32),
        ("mask", ctypes.c_int32), ("prefix", ctypes.c_int32), ("window", ctypes.c_int32),
        ("o_last", ctypes.c_void_p), ("flags", ctypes.c_int32),
    ]


class RunInfo(ctypes.Structure):
    _fields_ = [
        ("tokens", ctypes.c_int64), ("pairs", ctypes.c_int64), ("flops", ctypes.c_int64),
        ("bytes", ctypes.c_int64), ("work_items", ctypes.c_int32),
        ("block_queries", ctypes.c_int32), ("tile_pairs", ctypes.c_int64),
        ("slots", ctypes.c_int32), ("split_items", ctypes.c_int32),
    ]

    def as_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}


HIDDEN, INTERMEDIATE, MAX_LAYERS, Q6K_BLOCK_BYTES = 1024, 3072, 28, 210
# enum qattn_model_stage, in the reference's profile() order (model.ts:157-168)
STAGES = ("embedding_norm", "qkv", "rope_attention", "attention_output", "post_attention_norm",
          "ffn_up_gate", "swiglu", "ffn_down", "post_ffn_norm", "pool")


class LayerWeights(ctypes.Structure):
    """qattn_layer_weights: device pointers of one layer's tensors (model.ts:86-106)."""
    _fields_ = [
        ("attn_norm", ctypes.c_void_p),
        ("attn_qkv", ctypes.c_void_p), ("attn_qkv_bytes", ctypes.c_int64),
        ("attn_q_norm", ctypes.c_void_p), ("attn_k_norm", ctypes.c_void_p),
        ("attn_output", ctypes.c_void_p), ("attn_output_bytes", ctypes.c_int64),
        ("ffn_norm", ctypes.c_void_p),
        ("ffn_gate_up", ctypes.c_void_p), ("ffn_gate_up_bytes", ctypes.c_int64),
        ("ffn_down", ctypes.c_void_p), ("ffn_down_bytes", ctypes.c_int64),
    ]


class ModelDesc(ctypes.Structure):
    """qattn_model_desc."""
    _fields_ = [
        ("token_embd", ctypes.c_void_p), ("token_embd_bytes", ctypes.c_int64),
        ("output_norm", ctypes.c_void_p),
        ("n_layers", ctypes.c_int32),
        ("layers", ctypes.POINTER(LayerWeights)),
        ("eps", ctypes.c_double), ("rope_theta", ctypes.c_double),
        ("mask", ctypes.c_int32), ("prefix", ctypes.c_int32), ("window", ctypes.c_int32),
        ("flags", ctypes.c_int32),
    ]


def build():
    """Compile libqattn.so for gfx950 with the package Makefile."""
    subprocess.run(["make", "-s", "-C", PKG_DIR, "lib"], check=True)


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise QattnError(ENODEV, f"{LIB_PATH} is not built (run __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, i64, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t
    pvp = ctypes.POINTER(ctypes.c_void_p)
    sigs = {
        "qattn_abi_version": (ctypes.c_int, []),
        "qattn_create": (ctypes.c_int, [ctypes.c_int, pvp]),
        "qattn_destroy": (None, [vp]),
        "qattn_last_error": (ctypes.c_char_p, [vp]),
        "qattn_stream": (vp, [vp]),
        "qattn_synchronize": (ctypes.c_int, [vp]),
        "qattn_device_name": (ctypes.c_int, [vp, ctypes.c_char_p, sz, ctypes.POINTER(ctypes.c_int)]),
        "qattn_buffer_alloc": (ctypes.c_int, [vp, sz, pvp]),
        "qattn_buffer_free": (ctypes.c_int, [vp, vp]),
        "qattn_buffer_write": (ctypes.c_int, [vp, vp, sz, vp, sz]),
        "qattn_buffer_read": (ctypes.c_int, [vp, vp, sz, vp, sz]),
        "qattn_buffer_read_after": (ctypes.c_int, [vp, vp, vp, sz, vp, sz]),
        "qattn_buffer_fill_u16": (ctypes.c_int, [vp, vp, ctypes.c_uint16, sz]),
        "qattn_run_create": (ctypes.c_int, [vp, ctypes.POINTER(RunDesc), pvp]),
        "qattn_run_encode": (ctypes.c_int, [vp, vp]),
        "qattn_run_rebind": (ctypes.c_int, [vp, vp, vp, vp, vp, vp]),
        "qattn_run_update": (ctypes.c_int, [vp, vp, i32]),
        "qattn_run_destroy": (None, [vp]),
        "qattn_run_get_info": (ctypes.c_int, [vp, ctypes.POINTER(RunInfo)]),
        "qattn_plan_describe": (ctypes.c_int, [ctypes.POINTER(RunDesc), vp, i32,
                                               ctypes.POINTER(i32), ctypes.POINTER(RunInfo)]),
        "qattn_plan_slots": (ctypes.c_int, [ctypes.POINTER(RunDesc), i32, vp, i32, ctypes.POINTER(i32)]),
        "qattn_debug_xcd_map": (ctypes.c_int, [vp, i32, vp]),
        "qattn_prefill": (ctypes.c_int, [vp, ctypes.POINTER(RunDesc), vp]),
        "qattn_prefill_static": (ctypes.c_int, [vp, ctypes.POINTER(RunDesc), vp]),
        "qattn_debug_mask": (ctypes.c_int, [vp, i32, i32, i32, i32, vp]),
        "qattn_plan_mask": (ctypes.c_int, [i32, i32, i32, i32, vp]),
        "qattn_debug_run_mask": (ctypes.c_int, [vp, vp, i64, ctypes.POINTER(i32)]),
        "qattn_debug_fail_allocs": (None, [i32]),
        "qattn_debug_run_timeline": (ctypes.c_int, [vp, vp, i64, ctypes.POINTER(i32)]),
        "qattn_qk_norm_rope": (ctypes.c_int, [vp, vp, i64, i64, i32, vp, i32, vp,
                                              ctypes.c_double, ctypes.c_double, vp]),
        "qattn_qk_norm_rope_qkv": (ctypes.c_int, [vp, vp, i64, vp, i64, vp, i64, vp, i32, vp, vp,
                                                  ctypes.c_double, ctypes.c_double, vp]),
        "qattn_pool_last_l2": (ctypes.c_int, [vp, vp, i64, i32, vp, i32, vp, i64, vp]),
        "qattn_q4_compact_bytes": (i64, [i32, i32]),
        "qattn_q4_matmul": (ctypes.c_int, [vp, vp, i64, i32, i32, vp, i64, i32, vp, i64, vp]),
        "qattn_q4_matmul_swiglu": (ctypes.c_int, [vp, vp, i64, i32, i32, vp, i64, i32, vp, i64, vp]),
        "qattn_fill_normal": (ctypes.c_int, [vp, vp, i64, i64, i64, ctypes.c_uint64, vp]),
        "qattn_fill_token_rows": (ctypes.c_int, [vp, vp, vp, i64, i64, i64, ctypes.c_uint64, vp]),
        "qattn_gen_qkv": (ctypes.c_int, [vp, ctypes.c_uint32, ctypes.c_uint32, vp, i32,
                                         vp, i64, vp, i64, vp, i64, vp]),
        "qattn_event_create": (ctypes.c_int, [vp, pvp]),
        "qattn_event_record": (ctypes.c_int, [vp, vp]),
        "qattn_event_elapsed_ms": (ctypes.c_int, [vp, vp, ctypes.POINTER(ctypes.c_float)]),
        "qattn_event_synchronize": (ctypes.c_int, [vp]),
        "qattn_event_destroy": (ctypes.c_int, [vp]),
        "qattn_embed_q6k": (ctypes.c_int, [vp, vp, i64, vp, i64, i32, vp, i64, vp]),
        "qattn_rmsnorm": (ctypes.c_int, [vp, vp, i64, vp, i64, vp, vp, i64, i64, i32, ctypes.c_double, vp]),
        "qattn_swiglu": (ctypes.c_int, [vp, vp, i64, vp, i64, i64, i32, vp]),
        "qattn_model_create": (ctypes.c_int, [vp, ctypes.POINTER(ModelDesc), pvp]),
        "qattn_model_destroy": (None, [vp]),
        "qattn_model_plan_create": (ctypes.c_int, [vp, i32, i32, pvp]),
        "qattn_model_plan_destroy": (None, [vp]),
        "qattn_model_plan_run": (ctypes.c_int, [vp, vp, vp, i32, vp, i64, vp]),
        "qattn_model_plan_profile": (ctypes.c_int, [vp, vp, vp, i32, vp, i64, vp, vp]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _check(rc, ctx=None):
    if rc != OK:
        msg = lib().qattn_last_error(ctx)
        raise QattnError(rc, msg.decode() if msg else "")


def _np_ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def make_desc(q, k, v, o, cu_seqlens, mask=MASK_PREFIX_LOCAL, prefix=176, window=432,
              q_row_stride=HQ * HD, k_row_stride=HKV * HD, v_row_stride=HKV * HD,
              o_row_stride=HQ * HD, v_offset=0, o_last=None, flags=0):
    """Build a qattn_run_desc.  q/k/v/o/o_last are device addresses (int).  The returned desc
    keeps a reference to its cu_seqlens array."""
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    d = RunDesc(q, k, v, o, q_row_stride, k_row_stride, v_row_stride, o_row_stride, v_offset,
                cu.ctypes.data, len(cu) - 1, mask, prefix, window, o_last, flags)
    d._cu = cu
    return d


def plan_slots(desc, max_slots=0):
    """Host-only planner: slot offsets int32[nslots+1] into plan_describe's item list."""
    n = ctypes.c_int32(0)
    _check(lib().qattn_plan_slots(ctypes.byref(desc), max_slots, None, 0, ctypes.byref(n)))
    out = np.zeros(n.value + 1, dtype=np.int32)
    _check(lib().qattn_plan_slots(ctypes.byref(desc), max_slots, _np_ptr(out), n.value + 1, ctypes.byref(n)))
    return out


def plan_describe(desc):
    """Host-only planner: (work entries int32[n,8] grouped by slot, RunInfo)."""
    n = ctypes.c_int32(0)
    info = RunInfo()
    _check(lib().qattn_plan_describe(ctypes.byref(desc), None, 0, ctypes.byref(n), ctypes.byref(info)))
    items = np.zeros((n.value, 8), dtype=np.int32)
    if n.value:
        _check(lib().qattn_plan_describe(ctypes.byref(desc), _np_ptr(items), n.value,
                                         ctypes.byref(n), None))
    return items, info


def plan_mask(L, mask=MASK_PREFIX_LOCAL, prefix=176, window=432):
    """Host run of the kernel's key iteration: uint32 [L, ceil(L/32)] bitmask."""
    out = np.zeros((L, (L + 31) // 32), dtype=np.uint32)
    _check(lib().qattn_plan_mask(L, mask, prefix, window, _np_ptr(out) if L else None))
    return out


class Buffer:
    """Device allocation owned by a Context."""

    def __init__(self, ctx, nbytes):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        _check(lib().qattn_buffer_alloc(ctx.handle, self.nbytes, ctypes.byref(p)), ctx.handle)
        self.ptr = p.value

    def write(self, array, offset=0):
        a = np.ascontiguousarray(array)
        assert offset + a.nbytes <= self.nbytes
        _check(lib().qattn_buffer_write(self.ctx.handle, self.ptr, offset, _np_ptr(a), a.nbytes),
               self.ctx.handle)

    def read(self, dtype, shape, offset=0):
        out = np.empty(shape, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        _check(lib().qattn_buffer_read(self.ctx.handle, self.ptr, offset, _np_ptr(out), out.nbytes),
               self.ctx.handle)
        return out

    def read_after(self, event, dtype, shape, offset=0):
        """The buffer's contents once the work recorded before `event` has finished, without
        waiting for work enqueued after it (qattn_buffer_read_after)."""
        out = np.empty(shape, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        _check(lib().qattn_buffer_read_after(self.ctx.handle, event.handle, self.ptr, offset, _np_ptr(out),
                                             out.nbytes), self.ctx.handle)
        return out

    def fill_u16(self, value, count=None):
        count = self.nbytes // 2 if count is None else count
        _check(lib().qattn_buffer_fill_u16(self.ctx.handle, self.ptr, value, count), self.ctx.handle)

    def free(self):
        if self.ptr:
            _check(lib().qattn_buffer_free(self.ctx.handle, self.ptr), self.ctx.handle)
            self.ptr = None


class Run:
    """A planned attention launch (reference: AttentionRun from createRun, ops.ts:318-343)."""

    def __init__(self, ctx, desc):
        self.ctx = ctx
        self.desc = desc
        h = ctypes.c_void_p()
        _check(lib().qattn_run_create(ctx.handle, ctypes.byref(desc), ctypes.byref(h)), ctx.handle)
        self.handle = h.value

    def encode(self, stream=None):
        _check(lib().qattn_run_encode(self.handle, stream), self.ctx.handle)

    def rebind(self, q, k, v, o, o_last=None):
        _check(lib().qattn_run_rebind(self.handle, q, k, v, o, o_last), self.ctx.handle)

    def update(self, cu_seqlens):
        """Re-plan for new sequence lengths (qattn_run_update); same tensors and options."""
        cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
        _check(lib().qattn_run_update(self.handle, _np_ptr(cu), len(cu) - 1), self.ctx.handle)

    def info(self):
        i = RunInfo()
        _check(lib().qattn_run_get_info(self.handle, ctypes.byref(i)), self.ctx.handle)
        return i

    def mask_bits(self):
        """Keys the kernel kept (qattn_debug_run_mask): uint32 [16 heads, tokens, words]."""
        words = ctypes.c_int32()
        _check(lib().qattn_debug_run_mask(self.handle, None, 0, ctypes.byref(words)), self.ctx.handle)
        T = self.info().tokens
        out = np.zeros((HQ, T, words.value), dtype=np.uint32)
        _check(lib().qattn_debug_run_mask(self.handle, _np_ptr(out) if out.size else None, out.size,
                                          ctypes.byref(words)), self.ctx.handle)
        return out

    def timeline(self):
        """Phase timestamps of one launch (qattn_debug_run_timeline): uint32 [slots, 128], 100 MHz."""
        slots = ctypes.c_int32()
        _check(lib().qattn_debug_run_timeline(self.handle, None, 0, ctypes.byref(slots)), self.ctx.handle)
        out = np.zeros((slots.value, 128), dtype=np.uint32)
        _check(lib().qattn_debug_run_timeline(self.handle, _np_ptr(out) if out.size else None, out.size,
                                              ctypes.byref(slots)), self.ctx.handle)
        return out

    def destroy(self):
        if self.handle:
            lib().qattn_run_destroy(self.handle)
            self.handle = None


class Event:
    def __init__(self, ctx):
        self.ctx = ctx
        e = ctypes.c_void_p()
        _check(lib().qattn_event_create(ctx.handle, ctypes.byref(e)), ctx.handle)
        self.handle = e.value

    def record(self, stream=None):
        _check(lib().qattn_event_record(self.handle, stream if stream else self.ctx.stream))

    def elapsed_ms(self, later):
        ms = ctypes.c_float()
        _check(lib().qattn_event_elapsed_ms(self.handle, later.handle, ctypes.byref(ms)))
        return ms.value

    def synchronize(self):
        _check(lib().qattn_event_synchronize(self.handle))

    def destroy(self):
        if self.handle:
            lib().qattn_event_destroy(self.handle)
            self.handle = None


class Context:
    """Device context (reference: requestWebGPUDevice, src/webgpu/device.ts:6-24)."""

    def __init__(self, device=0):
        h = ctypes.c_void_p()
        _check(lib().qattn_create(device, ctypes.byref(h)))
        self.handle = h.value
        self.stream = lib().qattn_stream(self.handle)

    def close(self):
        if self.handle:
            lib().qattn_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def device_name(self):
        buf = ctypes.create_string_buffer(256)
        cu = ctypes.c_int()
        _check(lib().qattn_device_name(self.handle, buf, 256, ctypes.byref(cu)), self.handle)
        return buf.value.decode(), cu.value

    def synchronize(self):
        _check(lib().qattn_synchronize(self.handle), self.handle)

    def alloc(self, nbytes):
        return Buffer(self, nbytes)

    def upload(self, array):
        a = np.ascontiguousarray(array)
        b = Buffer(self, max(a.nbytes, 16))
        b.write(a)
        return b

    def run(self, desc):
        return Run(self, desc)

    def prefill(self, desc, stream=None):
        _check(lib().qattn_prefill(self.handle, ctypes.byref(desc), stream), self.handle)

    def prefill_static(self, desc, stream=None):
        """qattn_prefill_static: the same launch with no device allocation (batch-invariant plan)."""
        _check(lib().qattn_prefill_static(self.handle, ctypes.byref(desc), stream), self.handle)

    def debug_mask(self, L, mask=MASK_PREFIX_LOCAL, prefix=176, window=432):
        words = (L + 31) // 32
        out = np.zeros((L, words), dtype=np.uint32)
        _check(lib().qattn_debug_mask(self.handle, L, mask, prefix, window,
                                      _np_ptr(out) if L else None), self.handle)
        return out

    def xcd_map(self, n=512):
        """XCD of each of n workgroups of an attention-shaped launch (diagnostic)."""
        out = np.zeros(n, dtype=np.int32)
        _check(lib().qattn_debug_xcd_map(self.handle, n, _np_ptr(out)), self.handle)
        return out

    def qk_norm_rope(self, x_ptr, row_stride, col0, heads, cu_seqlens, weight_ptr=None,
                     eps=1e-6, theta=1e6, stream=None):
        cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
        _check(lib().qattn_qk_norm_rope(self.handle, x_ptr, row_stride, col0, heads, _np_ptr(cu),
                                        len(cu) - 1, weight_ptr, eps, theta, stream), self.handle)

    def qk_norm_rope_qkv(self, qkv_ptr, q_ptr, k_ptr, cu_seqlens, qkv_row_stride=4096,
                         q_row_stride=HQ * HD, k_row_stride=HKV * HD, q_weight_ptr=None,
                         k_weight_ptr=None, eps=1e-6, theta=1e6, stream=None):
        cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
        _check(lib().qattn_qk_norm_rope_qkv(self.handle, qkv_ptr, qkv_row_stride, q_ptr, q_row_stride,
                                            k_ptr, k_row_stride, _np_ptr(cu), len(cu) - 1, q_weight_ptr,
                                            k_weight_ptr, eps, theta, stream), self.handle)

    def pool_last_l2(self, x_ptr, row_stride, width, cu_seqlens, out_ptr, out_row_stride=None,
                     stream=None):
        """Last row of each sequence, L2-normalised, fp16 -> f32 (LastTokenPoolKernel,
        ops.ts:347-379)."""
        cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
        _check(lib().qattn_pool_last_l2(self.handle, x_ptr, row_stride, width, _np_ptr(cu), len(cu) - 1,
                                        out_ptr, width if out_row_stride is None else out_row_stride,
                                        stream), self.handle)

    def q4_matmul(self, x_ptr, M, K, w_ptr, w_bytes, N, y_ptr, ldx=None, ldy=None, stream=None):
        """y = x W^T for tile32-compact Q4_0 weights W [N, K] (quant-matmul.ts:267-307)."""
        _check(lib().qattn_q4_matmul(self.handle, x_ptr, K if ldx is None else ldx, M, K, w_ptr, w_bytes, N,
                                     y_ptr, N if ldy is None else ldy, stream), self.handle)

    def q4_matmul_swiglu(self, x_ptr, M, K, w_ptr, w_bytes, n_inter, y_ptr, ldx=None, ldy=None, stream=None):
        """y = swiglu(x W^T) for a [gate (n_inter rows) | up (n_inter rows)] tile32-compact Q4_0
        weight, in one launch: the compact matmul of quant-matmul.ts:267-307 followed by
        SwiGLUKernel (ops.ts:74-102), bit-identical to q4_matmul then swiglu."""
        _check(lib().qattn_q4_matmul_swiglu(self.handle, x_ptr, K if ldx is None else ldx, M, K, w_ptr, w_bytes,
                                            n_inter, y_ptr, n_inter if ldy is None else ldy, stream), self.handle)

    def fill_normal(self, ptr, rows, row_elems, row_stride, seed, stream=None):
        _check(lib().qattn_fill_normal(self.handle, ptr, rows, row_elems, row_stride, seed, stream),
               self.handle)

    def fill_token_rows(self, ptr, ids_ptr, rows, row_elems, row_stride, seed, stream=None):
        _check(lib().qattn_fill_token_rows(self.handle, ptr, ids_ptr, rows, row_elems, row_stride,
                                           seed, stream), self.handle)

    def gen_qkv(self, config, layer, cu_seqlens, q_ptr, k_ptr, v_ptr, q_row_stride=HQ * HD,
                k_row_stride=HKV * HD, v_row_stride=HKV * HD, stream=None):
        cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
        _check(lib().qattn_gen_qkv(self.handle, config, layer, _np_ptr(cu), len(cu) - 1,
                                   q_ptr, q_row_stride, k_ptr, k_row_stride, v_ptr, v_row_stride,
                                   stream), self.handle)

    def event(self):
        return Event(self)

    def embed_q6k(self, ids_ptr, tokens, table_ptr, table_bytes, out_ptr, width=HIDDEN, out_row_stride=None,
                  stream=None):
        """Q6_K token-embedding rows (EmbeddingLookupKernel, ops.ts:381-423)."""
        _check(lib().qattn_embed_q6k(self.handle, ids_ptr, tokens, table_ptr, table_bytes, width, out_ptr,
                                     width if out_row_stride is None else out_row_stride, stream), self.handle)

    def rmsnorm(self, x_ptr, weight_ptr, out_ptr, rows, width=HIDDEN, residual_ptr=None, eps=1e-6,
                x_row_stride=None, residual_row_stride=None, out_row_stride=None, stream=None):
        """Residual add (in place on x) + RMSNorm (RmsNormKernel, ops.ts:21-72)."""
        _check(lib().qattn_rmsnorm(self.handle, x_ptr, width if x_row_stride is None else x_row_stride,
                                   residual_ptr, width if residual_row_stride is None else residual_row_stride,
                                   weight_ptr, out_ptr, width if out_row_stride is None else out_row_stride,
                                   rows, width, eps, stream), self.handle)

    def swiglu(self, gate_up_ptr, out_ptr, rows, width=INTERMEDIATE, gate_up_row_stride=None,
               out_row_stride=None, stream=None):
        """silu(gate) * up (SwiGLUKernel, ops.ts:74-102)."""
        _check(lib().qattn_swiglu(self.handle, gate_up_ptr,
                                  2 * width if gate_up_row_stride is None else gate_up_row_stride, out_ptr,
                                  width if out_row_stride is None else out_row_stride, rows, width, stream),
               self.handle)

    def model(self, token_embd, output_norm, layers, eps=1e-6, rope_theta=1e6, mask=MASK_PREFIX_LOCAL,
              prefix=176, window=432, flags=0):
        """qattn_model_create over device tensors: token_embd = (ptr, bytes), output_norm = ptr,
        layers = list of dicts with the LayerWeights field names (compact tensors as (ptr, bytes))."""
        return Model(self, token_embd, output_norm, layers, eps, rope_theta, mask, prefix, window, flags)


class Model:
    """The weights of the forward (Qwen3WebGPUModel, model.ts:185-255); plan() makes an
    execution plan (Qwen3ExecutionPlan, model.ts:49-183)."""

    def __init__(self, ctx, token_embd, output_norm, layers, eps, rope_theta, mask, prefix, window, flags):
        self.ctx = ctx
        arr = (LayerWeights * len(layers))()
        for i, lw in enumerate(layers):
            for name in ("attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm"):
                setattr(arr[i], name, lw[name])
            for name in ("attn_qkv", "attn_output", "ffn_gate_up", "ffn_down"):
                ptr, nbytes = lw[name]
                setattr(arr[i], name, ptr)
                setattr(arr[i], name + "_bytes", nbytes)
        d = ModelDesc(token_embd[0], token_embd[1], output_norm, len(layers),
                      ctypes.cast(arr, ctypes.POINTER(LayerWeights)), eps, rope_theta, mask, prefix, window, flags)
        h = ctypes.c_void_p()
        _check(lib().qattn_model_create(ctx.handle, ctypes.byref(d), ctypes.byref(h)), ctx.handle)
        self.handle = h

    def plan(self, max_tokens, max_seqs=16):
        return ModelPlan(self, max_tokens, max_seqs)

    def destroy(self):
        if self.handle:
            lib().qattn_model_destroy(self.handle)
            self.handle = None


class ModelPlan:
    def __init__(self, model, max_tokens, max_seqs):
        self.model = model
        h = ctypes.c_void_p()
        _check(lib().qattn_model_plan_create(model.handle, max_tokens, max_seqs, ctypes.byref(h)),
               model.ctx.handle)
        self.handle = h

    def run(self, ids, cu_seqlens, out_ptr, out_row_stride=HIDDEN, stream=None):
        """Enqueue one packed batch; out_ptr: device f32 [nseq, out_row_stride]."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
        _check(lib().qattn_model_plan_run(self.handle, _np_ptr(ids) if ids.size else None, _np_ptr(cu),
                                          len(cu) - 1, out_ptr, out_row_stride, stream), self.model.ctx.handle)

    def profile(self, ids, cu_seqlens, out_ptr, out_row_stride=HIDDEN, stream=None):
        """One batch with per-stage timing: {stage name: ms over all layers}."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
        ms = np.zeros(len(STAGES), dtype=np.float32)
        _check(lib().qattn_model_plan_profile(self.handle, _np_ptr(ids) if ids.size else None, _np_ptr(cu),
                                              len(cu) - 1, out_ptr, out_row_stride, stream, _np_ptr(ms)),
               self.model.ctx.handle)
        return dict(zip(STAGES, (float(x) for x in ms)))

    def destroy(self):
        if self.handle:
            lib().qattn_model_plan_destroy(self.handle)
            self.handle = None


def header_symbols(path=HEADER_PATH):
    """Function names declared in include/qattn.h."""
    import re
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qattn_[a-z0-9_]+)\s*\(", text)))
