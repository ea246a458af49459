"""qattn_debug_run_timeline -- the attention kernel's phase-timestamp variant -- on the GPU.

The variant must write the same output rows as qattn_run_encode, bit for bit (split plans with
their merge kernel too), and its stamps must describe the plan: every used slot's stamps run
forward in the documented order (start, first loads landed, per entry top / first tile / last
tile / next loads issued / last PV / hand-over wait / rows staged / rows stored, end), the
entries a slot does not have stay 0, and slots without work stay all 0.
"""
import numpy as np
import pytest

from test_gpu_parity import cu_of

pytestmark = pytest.mark.gpu
STAMPS = 128


def _ticks(row, t0):
    return (row.astype(np.int64) - int(t0)) % (1 << 32)


@pytest.mark.parametrize("lengths,mask,flags", [
    ([500] * 16, 0, 0),                   # the 16x500 headline packing, unsplit
    ([5000], 1, 0),                       # 1x5000 sparse: split items + merge kernel
    ([700, 1, 33, 1500, 64, 65], 1, 1),   # ragged, batch-invariant
])
def test_timeline_variant_matches_encode_and_orders_its_stamps(ctx, qattn, lengths, mask, flags):
    cu = cu_of(lengths)
    T = int(cu[-1])
    print(f"timeline {lengths[:3]}{'...' if len(lengths) > 3 else ''} mask {mask} flags {flags}", flush=True)
    bq, bk, bv, bo = ctx.alloc(T * 4096), ctx.alloc(T * 2048), ctx.alloc(T * 2048), ctx.alloc(T * 4096)
    ctx.gen_qkv(1, 0, cu, bq.ptr, bk.ptr, bv.ptr)
    desc = qattn.make_desc(bq.ptr, bk.ptr, bv.ptr, bo.ptr, cu, mask, 176, 432, flags=flags)
    run = ctx.run(desc)
    info = run.info()
    bo.fill_u16(0x7E00)
    run.encode()
    ctx.synchronize()
    want = bo.read(np.uint16, (T, 2048))
    bo.fill_u16(0x7E00)
    st = run.timeline()
    got = bo.read(np.uint16, (T, 2048))
    assert np.array_equal(got, want)
    slots = qattn.plan_slots(desc)
    entries, _ = qattn.plan_describe(desc)
    assert st.shape == (len(slots) - 1, STAMPS) and st.shape[0] == info.slots
    for b in range(st.shape[0]):
        n = int(slots[b + 1] - slots[b])
        row = st[b]
        if n == 0:
            assert not row.any(), b
            continue
        assert row[0] != 0 and row[1] != 0 and row[STAMPS - 1] != 0, b
        seen = [1]
        for e in range(min(n, 15)):
            seen += list(range(2 + 8 * e, 10 + 8 * e))
        seen.append(STAMPS - 1)
        t = _ticks(row[seen], row[0])
        assert np.all(np.diff(t) >= 0), (b, t)
        assert t[-1] < 100_000_000, (b, t[-1])  # under a second
        unused = np.ones(STAMPS, bool)
        unused[[0] + seen] = False
        if n <= 15:
            assert not row[unused].any(), b
        tiles = entries[slots[b]:slots[b + 1], 5] - entries[slots[b]:slots[b + 1], 4]
        assert (tiles >= 1).all()
    run.destroy()
    for buf in (bq, bk, bv, bo):
        buf.free()
