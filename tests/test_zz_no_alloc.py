"""qattn_prefill_static -- the entry point that allocates no device memory -- on the GPU.

Called through the C ABI twice in a row, the second time with a smaller input, each output must
equal qattn_prefill's with QATTN_FLAG_BATCH_INVARIANT bit for bit (same plan, same kernel), and
meet the parity bar against the default (split-K) plan and the f64 oracle.  Oversized launches
are rejected before any device work.
"""
import ctypes

import numpy as np
import pytest

from test_gpu_parity import ATOL, MIN_COS, compare, cu_of, f16

pytestmark = pytest.mark.gpu
FLAG_BATCH_INVARIANT = 1


def _run_both(ctx, qattn, oracle, lengths, mask, label):
    cu = cu_of(lengths)
    T = int(cu[-1])
    print(f"prefill_static {label}: lengths {lengths[:4]}{'...' if len(lengths) > 4 else ''} mask {mask}", flush=True)
    q, k, v = oracle.gen_qkv(1, 3, cu)
    bq, bk, bv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    outs = {}
    for name in ("static", "invariant", "default"):
        bo = ctx.alloc(T * 4096)
        bo.fill_u16(0x7E00)  # NaN: every row must be written
        flags = 0 if name == "default" else FLAG_BATCH_INVARIANT
        desc = qattn.make_desc(bq.ptr, bk.ptr, bv.ptr, bo.ptr, cu, mask, 176, 432, flags=flags)
        if name == "static":
            ctx.prefill_static(desc)
        else:
            ctx.prefill(desc)
        outs[name] = bo.read(np.uint16, (T, 2048))
        bo.free()
    assert np.array_equal(outs["static"], outs["invariant"]), label
    got, ref = f16(outs["static"]), f16(outs["default"])
    assert np.abs(got - ref).max() <= ATOL, label
    if T <= 2000:
        compare(outs["static"], oracle.attention_exact(q, k, v, cu, kind=mask), f"static {label} vs exact")
    for b in (bq, bk, bv):
        b.free()


def test_prefill_static_two_calls_second_smaller(ctx, qattn, oracle):
    _run_both(ctx, qattn, oracle, [5000, 33, 1500, 1, 700], 1, "first call")
    _run_both(ctx, qattn, oracle, [500, 64, 65, 17], 0, "second, smaller call")


def test_prefill_static_rejects_oversized_plan_before_device_work(ctx, qattn):
    # 5000 one-token sequences -> 5000 x 8 = 40000 work entries (32 bytes each), more than the
    # 1 MiB static work list holds (checked on the host first).  The tensors are real device
    # buffers sized for the batch: no attention launch can be handed a wild address.
    lengths = [1] * 5000
    cu = cu_of(lengths)
    T = int(cu[-1])
    bufs = [ctx.alloc(T * 4096), ctx.alloc(T * 2048), ctx.alloc(T * 2048), ctx.alloc(T * 4096)]
    desc = qattn.make_desc(*(b.ptr for b in bufs), cu, 1, 176, 432, flags=FLAG_BATCH_INVARIANT)
    entries, info = qattn.plan_describe(desc)
    assert len(entries) == 40000 and len(entries) * 32 > (1 << 20)
    with pytest.raises(qattn.QattnError) as e:
        ctx.prefill_static(desc)
    assert e.value.code == qattn.EINVAL and b"static" in qattn.lib().qattn_last_error(ctx.handle)
    for b in bufs:
        b.free()
