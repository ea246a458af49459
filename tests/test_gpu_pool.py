"""GPU parity of the last-token pool + L2 norm (qattn_pool_last_l2, replacing the reference's
LastTokenPoolKernel, src/webgpu/ops.ts:347-379) against the f64 oracle, through the C ABI.

Tolerance: the kernel sums the squares in f32, n = 8 * ceil(width / 512) fused multiply-adds per
lane and then a 6-level wave tree, so the sum's relative error is at most (n + 6) u (u = 2^-24);
the square root halves it, and the root, the reciprocal and the final product add one u each:
|got - exact| <= rtol(width) * |exact| + 1e-12 with rtol = 2 * ((n + 6) / 2 + 3) u (a factor 2
of margin): 1.7e-6 at width 1024, 2.6e-6 at 2048, 8.3e-6 at 8192.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu



def rtol(width):
    n = 8 * -(-width // 512)
    return 2 * ((n + 6) / 2 + 3) * 2.0 ** -24

F32_NAN_FILL = 0x7FC0  # two of these halves read as one f32 NaN


def cu_of(lengths):
    return np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)


def run_pool(ctx, x, cu, width, row_stride=None, out_row_stride=None):
    row_stride = x.shape[1] if row_stride is None else row_stride
    out_row_stride = width if out_row_stride is None else out_row_stride
    assert x.shape[1] == row_stride
    bx = ctx.upload(x.view(np.uint16))
    nseq = len(cu) - 1
    bo = ctx.alloc(max(nseq * out_row_stride * 4, 16))
    bo.fill_u16(F32_NAN_FILL)
    ctx.pool_last_l2(bx.ptr, row_stride, width, cu, bo.ptr, out_row_stride)
    ctx.synchronize()
    out = bo.read(np.float32, (nseq, out_row_stride))
    bx.free()
    bo.free()
    return out


def check(oracle, out, x, cu, width, label):
    want = oracle.pool_last_l2(x, cu, width)
    got = out[:, :width].astype(np.float64)
    err = np.abs(got - want)
    bound = rtol(width) * np.abs(want) + 1e-12
    print(f"[{label}] max|err| {err.max():.3e}  max rel {np.max(err / np.maximum(np.abs(want), 1e-30)):.2e}",
          flush=True)
    assert np.isfinite(got).all(), label
    assert (err <= bound).all(), label


@pytest.mark.parametrize("width,row_stride,out_row_stride", [(1024, 1024, 1024), (2048, 2048, 2048),
                                                             (1024, 4096, 1028), (8, 8, 8), (520, 528, 520),
                                                             (4096, 4096, 4096), (4104, 4104, 4104),
                                                             (8192, 8200, 8192)])
def test_pool_matches_oracle(ctx, oracle, width, row_stride, out_row_stride):
    rng = np.random.default_rng(width + row_stride)
    lengths = [1, 7, 0, 150, 33, 2, 64]
    cu = cu_of(lengths)
    x = (rng.standard_normal((int(cu[-1]), row_stride)) * 3).astype(np.float16)
    out = run_pool(ctx, x, cu, width, row_stride, out_row_stride)
    check(oracle, out, x, cu, width, f"pool W={width} stride={row_stride}")
    assert not out[2, :width].any()  # the empty sequence: zeros
    np.testing.assert_allclose(np.linalg.norm(out[[0, 1, 3, 4, 5, 6], :width].astype(np.float64), axis=1), 1.0,
                               rtol=0, atol=2 * rtol(width))


def test_pool_more_sequences_than_one_launch(ctx, oracle):
    # 300 sequences: two launches of at most 256 rows each.
    rng = np.random.default_rng(11)
    lengths = rng.integers(1, 6, size=300)
    cu = cu_of(lengths)
    x = rng.standard_normal((int(cu[-1]), 1024)).astype(np.float16)
    out = run_pool(ctx, x, cu, 1024)
    check(oracle, out, x, cu, 1024, "pool nseq=300")


def test_pool_zero_row_is_nan_as_the_reference(ctx):
    x = np.zeros((3, 1024), np.float16)
    x[0, 5] = 1.0
    out = run_pool(ctx, x, cu_of([1, 2]), 1024)
    assert out[0, 5] == 1.0 and not np.delete(out[0], 5).any()
    assert np.isnan(out[1]).all()


def test_pool_of_attention_last_rows(ctx, qattn, oracle):
    # The embedding path: attention with o_last, then the pool over the last rows.  Pooling O at
    # stride 2048 and pooling the o_last rows give the same f32 vectors, bit for bit, and match
    # the oracle's pool of those rows.
    lengths = oracle.gen_lengths(0x51574E33, 16)
    cu = cu_of(lengths)
    T = int(cu[-1])
    bq, bk, bv = ctx.alloc(T * 4096), ctx.alloc(T * 2048), ctx.alloc(T * 2048)
    bo, bl = ctx.alloc(T * 4096), ctx.alloc(16 * 4096)
    pa, pb = ctx.alloc(16 * 2048 * 4), ctx.alloc(16 * 2048 * 4)
    ctx.gen_qkv(1, 0, cu, bq.ptr, bk.ptr, bv.ptr)
    ctx.prefill(qattn.make_desc(bq.ptr, bk.ptr, bv.ptr, bo.ptr, cu, o_last=bl.ptr))
    ctx.pool_last_l2(bo.ptr, 2048, 2048, cu, pa.ptr)
    ctx.pool_last_l2(bl.ptr, 2048, 2048, np.arange(17, dtype=np.int32), pb.ptr)
    ctx.synchronize()
    a = pa.read(np.float32, (16, 2048))
    b = pb.read(np.float32, (16, 2048))
    assert np.array_equal(a, b)
    o = bo.read(np.uint16, (T, 2048)).view(np.float16)
    check(oracle, a, o, cu, 2048, "pool of attention O")
    for buf in (bq, bk, bv, bo, bl, pa, pb):
        buf.free()


def test_pool_invalid_arguments(ctx, qattn):
    buf = ctx.alloc(4096 * 4)
    cu = np.array([0, 1], np.int32)
    bad = [dict(width=12), dict(row_stride=1020), dict(out_row_stride=1022), dict(x_off=2), dict(out_off=4),
           dict(cu=np.array([0, 3, 1], np.int32))]
    for b in bad:
        with pytest.raises(qattn.QattnError) as e:
            ctx.pool_last_l2(buf.ptr + b.get("x_off", 0), b.get("row_stride", 1024), b.get("width", 1024),
                             b.get("cu", cu), buf.ptr + b.get("out_off", 0), b.get("out_row_stride", 1024))
        assert e.value.code == qattn.EINVAL, b
    buf.free()
