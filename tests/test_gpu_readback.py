"""qattn_buffer_read_after / qattn_event_synchronize: the readback of one submit, ordered by its
event only (the reference copies its embeddings to a readback buffer inside the same submit and
maps it, model.ts:133-135)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_read_after_returns_the_buffer_as_of_its_event(ctx):
    """A buffer written before the event reads back whole while later work still runs on the
    context stream; the event's own wait also returns, and a plain read agrees afterwards."""
    a = ctx.alloc(4096 * 2)
    big = ctx.alloc(8192 * 4096 * 2)
    ctx.fill_normal(a.ptr, 1, 4096, 4096, 5)
    ev = ctx.event()
    ev.record()
    for seed in range(16):  # work enqueued after the event, on other memory
        ctx.fill_normal(big.ptr, 8192, 4096, 4096, 100 + seed)
    got = a.read_after(ev, np.uint16, (4096,))
    ev.synchronize()
    ctx.synchronize()
    want = a.read(np.uint16, (4096,))
    assert np.array_equal(got, want)
    assert np.isfinite(got.view(np.float16)).all() and np.abs(got.view(np.float16)).max() > 0
    ev.destroy()
    a.free()
    big.free()


def test_read_after_a_partial_length(ctx):
    """Any length up to the buffer: the first `bytes` of it."""
    a = ctx.alloc(1024 * 2)
    ctx.fill_normal(a.ptr, 1, 1024, 1024, 9)
    ev = ctx.event()
    ev.record()
    head = a.read_after(ev, np.uint16, (100,))
    ctx.synchronize()
    assert np.array_equal(head, a.read(np.uint16, (1024,))[:100])
    ev.destroy()
    a.free()
