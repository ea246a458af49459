"""GPU parity of the Q4_0 tile32-compact dequant-GEMM (qattn_q4_matmul, replacing the reference's
compact batch matmul, src/webgpu/quant-matmul.ts:267-307) against the f64 oracle, through the C ABI,
and of its fused gate/up + SwiGLU form (qattn_q4_matmul_swiglu).

Tolerance, per element: the fp32 sum of K exact products (f16 x f16 products are exact in fp32)
errs by at most (K + 2) u32 * sum_k |x_k w_k| (u32 = 2^-24), and the final fp16 rounding by half an
ulp: |y - exact| <= 2^-11 |exact| + (K + 2) 2^-24 (|x| |w|^T) + 2^-25 (fp16 subnormal spacing).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def random_compact(rng, n, k, scale_lo=0.002, scale_hi=0.05):
    """A tile32-compact tensor of random Q4_0 records; rows past n in the last tile stay zero."""
    tiles, kb = -(-n // 32), k // 32
    rec = np.zeros((tiles, kb, 32, 20), np.uint8)
    scales = rng.uniform(scale_lo, scale_hi, size=(tiles, kb, 32)).astype(np.float16)
    scales *= np.where(rng.random(scales.shape) < 0.5, -1, 1).astype(np.float16)
    rec[..., 0:2] = scales.view(np.uint8).reshape(tiles, kb, 32, 2)
    rec[..., 4:20] = rng.integers(0, 256, size=(tiles, kb, 32, 16), dtype=np.uint8)
    flat = rec.reshape(-1, 20)
    rows = (np.arange(tiles)[:, None, None] * 32 + np.arange(32)[None, None, :]).repeat(kb, axis=1).reshape(-1)
    flat[rows >= n] = 0
    return flat.reshape(-1)


def run_q4(ctx, x, packed, k, n, ldx=None, ldy=None):
    m = x.shape[0]
    ldx = k if ldx is None else ldx
    ldy = -(-n // 8) * 8 if ldy is None else ldy
    xs = np.zeros((max(m, 1), ldx), np.float16)
    xs[:m, :k] = x
    bx, bw = ctx.upload(xs.view(np.uint16)), ctx.upload(packed)
    by = ctx.alloc(max(m, 1) * ldy * 2)
    by.fill_u16(0x7E00)  # NaN: every valid element must be written
    ctx.q4_matmul(bx.ptr, m, k, bw.ptr, packed.size, n, by.ptr, ldx=ldx, ldy=ldy)
    ctx.synchronize()
    y = by.read(np.uint16, (max(m, 1), ldy)).view(np.float16)
    for b in (bx, bw, by):
        b.free()
    return y[:m]


def check(oracle, y, x, packed, k, n, label):
    exact = oracle.q4_matmul(x, packed, k, n)
    w = oracle.q40_compact_weights(packed, k, n).astype(np.float64)
    mag = np.abs(x.astype(np.float64)) @ np.abs(w).T
    bound = 2.0 ** -11 * np.abs(exact) + (k + 2) * 2.0 ** -24 * mag + 2.0 ** -25
    got = y[:, :n].astype(np.float64)
    err = np.abs(got - exact)
    print(f"[{label}] max|err| {err.max():.3e}  max err/bound {np.max(err / bound):.3f}", flush=True)
    assert np.isfinite(got).all(), label
    assert (err <= bound).all(), label


@pytest.mark.parametrize("m,k,n", [(1, 32, 1), (130, 96, 70), (64, 128, 128), (257, 2048, 1024),
                                   (33, 3072, 1024), (1280, 1024, 4096)])
def test_q4_matmul_matches_oracle(ctx, oracle, m, k, n):
    rng = np.random.default_rng(m * 7 + k + n)
    packed = random_compact(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float16)
    y = run_q4(ctx, x, packed, k, n)
    check(oracle, y, x, packed, k, n, f"q4 {m}x{k}x{n}")


def test_q4_matmul_strides_and_untouched_padding(ctx, oracle):
    rng = np.random.default_rng(1)
    m, k, n = 70, 160, 40
    packed = random_compact(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float16)
    y = run_q4(ctx, x, packed, k, n, ldx=k + 24, ldy=n + 8)
    check(oracle, y, x, packed, k, n, "q4 strided")
    assert np.isnan(y[:, n:].astype(np.float32)).all()  # columns past N are not written


def test_q4_matmul_reference_format_vector(ctx, oracle):
    # The reference's packing test (tests/prepacked-format.test.ts:13-22) as weights: row 0 holds
    # q - 8 (scale 1), row 1 holds 2 (7 - q) (scale 2); x = e_j picks column j.
    def block(scale_bits, quants):
        b = bytearray(18)
        b[0:2] = bytes(scale_bits)
        for i in range(16):
            b[2 + i] = quants[i] | (quants[i + 16] << 4)
        return bytes(b)
    first = block([0x00, 0x3C], [i & 15 for i in range(32)])
    second = block([0x00, 0x40], [15 - (i & 15) for i in range(32)])
    packed, k, n = oracle.pack_q40_tile32([(32, 1, first), (32, 1, second)])
    x = np.eye(32, dtype=np.float16)
    y = run_q4(ctx, x, packed, k, n).astype(np.float64)
    assert np.array_equal(y[:, 0], [(j & 15) - 8 for j in range(32)])
    assert np.array_equal(y[:, 1], [2 * (7 - (j & 15)) for j in range(32)])


def run_q4_swiglu(ctx, x, packed, k, n_inter, ldy=None):
    m = x.shape[0]
    ldy = n_inter if ldy is None else ldy
    bx, bw = ctx.upload(np.ascontiguousarray(x).view(np.uint16)), ctx.upload(packed)
    by = ctx.alloc(max(m, 1) * ldy * 2)
    by.fill_u16(0x7E00)
    ctx.q4_matmul_swiglu(bx.ptr, m, k, bw.ptr, packed.size, n_inter, by.ptr, ldy=ldy)
    ctx.synchronize()
    y = by.read(np.uint16, (max(m, 1), ldy)).view(np.float16)
    for b in (bx, bw, by):
        b.free()
    return y[:m]


@pytest.mark.parametrize("m,k,n_inter", [(1, 32, 64), (130, 96, 128), (257, 1024, 3072), (1100, 256, 3072)])
def test_q4_matmul_swiglu_equals_the_two_launches(ctx, oracle, m, k, n_inter):
    """The fused gate/up projection + SwiGLU (one launch) against the launches it replaces: the
    projection into [m, 2 n_inter] (checked against the oracle's product here too), then
    qattn_swiglu -- equal bit for bit -- and within one fp16 step of the f64 SwiGLU restatement
    (oracle/model_ref.py, ops.ts:81-88) of that projection."""
    import model_ref as mr
    rng = np.random.default_rng(m + k + n_inter)
    packed = random_compact(rng, 2 * n_inter, k)
    x = rng.standard_normal((m, k)).astype(np.float16)
    gate_up = run_q4(ctx, x, packed, k, 2 * n_inter)
    check(oracle, gate_up, x, packed, k, 2 * n_inter, f"gate_up {m}x{k}x{2 * n_inter}")
    dg, do = ctx.upload(np.ascontiguousarray(gate_up).view(np.uint16)), ctx.alloc(m * n_inter * 2)
    ctx.swiglu(dg.ptr, do.ptr, m, width=n_inter)
    ctx.synchronize()
    two = do.read(np.uint16, (m, n_inter))
    dg.free()
    do.free()
    fused = run_q4_swiglu(ctx, x, packed, k, n_inter, ldy=n_inter + 8)
    assert np.isnan(fused[:, n_inter:].astype(np.float32)).all()  # columns past n_inter are not written
    assert np.array_equal(fused[:, :n_inter].view(np.uint16), two)
    ref = mr.swiglu(gate_up, n_inter).astype(np.float64)
    got = fused[:, :n_inter].astype(np.float64)
    step = np.maximum(np.spacing(np.maximum(np.abs(got), np.abs(ref)).astype(np.float16)).astype(np.float64), 2.0 ** -24)
    assert (np.abs(got - ref) / step).max() <= 1


def test_q4_rows_do_not_depend_on_the_launch_shape(ctx, oracle):
    """Three kernels serve one projection, chosen by the launch's size: up to 512 output blocks of
    32 x 32 the one-wavefront-per-block kernel, then the tiled kernel with 64-row tiles (fewer
    than 160 tiles of 128 x 128), then 128-row tiles.  Every output element is computed the same
    way in all three (the same K blocks and MFMA order), so rows 0..63 of a 64-row, a 300-row and
    an 1100-row launch are equal bit for bit -- the model's batch invariance rests on this -- for
    the plain and the fused gate/up projections."""
    rng = np.random.default_rng(5)
    k, n = 256, 4096
    packed = random_compact(rng, n, k)
    x = rng.standard_normal((1100, k)).astype(np.float16)
    big = run_q4(ctx, x, packed, k, n)          # 9 x 32 = 288 tiles: 128-row tiles
    mid = run_q4(ctx, x[:300], packed, k, n)    # 3 x 32 = 96 tiles: 64-row tiles
    small = run_q4(ctx, x[:64], packed, k, n)   # 2 x 128 = 256 blocks: one wavefront per block
    check(oracle, big, x, packed, k, n, "q4 1100 rows")
    check(oracle, small, x[:64], packed, k, n, "q4 64 rows")
    assert np.array_equal(big[:64].view(np.uint16), small.view(np.uint16))
    assert np.array_equal(mid[:64].view(np.uint16), small.view(np.uint16))
    big_f = run_q4_swiglu(ctx, x, packed, k, n // 2)
    mid_f = run_q4_swiglu(ctx, x[:300], packed, k, n // 2)
    small_f = run_q4_swiglu(ctx, x[:64], packed, k, n // 2)  # 2 x 64 = 128 blocks
    assert np.array_equal(big_f[:64].view(np.uint16), small_f.view(np.uint16))
    assert np.array_equal(mid_f[:64].view(np.uint16), small_f.view(np.uint16))


def test_q4_chunked_k_rows_do_not_depend_on_the_launch_shape(ctx, oracle):
    """K = 3072 spans three chunks of 1024 columns, summed in chunk order by every kernel: the
    direct kernel with one wavefront per chunk meeting in LDS (64 rows: 64 output blocks x 3
    chunks), the direct kernel with one wavefront folding the chunks in turn (300 rows: 320
    blocks, too many chunk wavefronts), the 64-row tiled kernel (1100 rows) and the 128-row tiled
    kernel (2600 rows: 168 tiles of 128 x 128), both with a second accumulator set.  Rows 0..63
    agree bit for bit."""
    rng = np.random.default_rng(6)
    k, n = 3072, 1024
    packed = random_compact(rng, n, k)
    x = rng.standard_normal((2600, k)).astype(np.float16)
    small = run_q4(ctx, x[:64], packed, k, n)
    check(oracle, small, x[:64], packed, k, n, "q4 chunked 64 rows")
    for m in (300, 1100, 2600):
        got = run_q4(ctx, x[:m], packed, k, n)
        assert np.array_equal(got[:64].view(np.uint16), small.view(np.uint16)), m
    check(oracle, got[:200], x[:200], packed, k, n, "q4 chunked 2600 rows (first 200)")


def test_q4_matmul_invalid_arguments(ctx, qattn):
    buf = ctx.alloc(1 << 16)
    good = dict(m=4, k=64, n=8, w_bytes=qattn.lib().qattn_q4_compact_bytes(64, 8), ldx=64, ldy=8, x_off=0)
    for bad in (dict(k=48), dict(w_bytes=100), dict(ldx=60), dict(ldy=12), dict(x_off=8), dict(n=0)):
        a = dict(good, **bad)
        with pytest.raises(qattn.QattnError) as e:
            ctx.q4_matmul(buf.ptr + a["x_off"], a["m"], a["k"], buf.ptr, a["w_bytes"], a["n"], buf.ptr,
                          ldx=a["ldx"], ldy=a["ldy"])
        assert e.value.code == qattn.EINVAL, bad
    # the fused entry point: n_inter a multiple of 64, y rows of n_inter, the weight 2 n_inter rows
    w128 = qattn.lib().qattn_q4_compact_bytes(64, 128)
    for n_inter, ldy, w_bytes in ((32, 64, w128), (96, 96, qattn.lib().qattn_q4_compact_bytes(64, 192)), (64, 56, w128),
                                  (64, 64, w128 - 20)):
        with pytest.raises(qattn.QattnError) as e:
            ctx.q4_matmul_swiglu(buf.ptr, 4, 64, buf.ptr, w_bytes, n_inter, buf.ptr, ldy=ldy)
        assert e.value.code == qattn.EINVAL, (n_inter, ldy, w_bytes)
    buf.free()
