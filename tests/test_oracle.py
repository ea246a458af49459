"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Every oracle function is checked against something other than its own formula: the reference's
own test vectors, published known answers, numpy / torch implementations, closed forms and
invariants that a dropped term, wrong sign, wrong index or transposed operand would break.
"""
import math

import numpy as np
import pytest

MASK_CAUSAL, MASK_PREFIX_LOCAL = 0, 1


def f16(a):
    return np.asarray(a, dtype=np.uint16).view(np.float16).astype(np.float64)


def to_bits(x):
    return np.asarray(x, dtype=np.float16).view(np.uint16)


# ---------------------------------------------------------------------------------------------
# fp16 codec  (reference: src/math/f16.ts:4-25, src/gguf/quantization.ts:2-9)
# ---------------------------------------------------------------------------------------------

def test_half_decoder_reference_kats(oracle):
    # tests/quantization.test.ts:5-9 of the reference
    for fn in (oracle.f16_to_f32, oracle.ref_half_to_float):
        assert fn(0x3C00) == 1.0
        assert fn(0xC000) == -2.0
        assert fn(0x0000) == 0.0


def test_half_decoder_exhaustive_vs_numpy(oracle):
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float64)
    got = np.array([oracle.f16_to_f32(int(i)) for i in h])
    ref = np.array([oracle.ref_half_to_float(int(i)) for i in h])
    fin = np.isfinite(want)
    assert np.array_equal(got[fin], want[fin]) and np.array_equal(ref[fin], want[fin])
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))


def test_half_encoder_round_trip_and_numpy(oracle):
    h = np.arange(65536, dtype=np.uint16)
    vals = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(vals)
    assert all(oracle.f32_to_f16(float(v)) == int(i) for i, v in zip(h[fin], vals[fin]))
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(20000) * np.exp(rng.uniform(-25, 12, 20000))).astype(np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert all(oracle.f32_to_f16(float(a)) == int(b) for a, b in zip(x, want))


def test_half_encoder_ties_to_even(oracle):
    # 1 + 2^-11 lies exactly between 1 and 1 + 2^-10: RNE keeps the even mantissa (1.0);
    # 1 + 3*2^-11 lies between 1+2^-10 (odd) and 1+2^-9 (even): rounds up.
    assert oracle.f32_to_f16(1.0 + 2.0 ** -11) == 0x3C00
    assert oracle.f32_to_f16(1.0 + 3 * 2.0 ** -11) == 0x3C02
    assert oracle.f32_to_f16(65504.0) == 0x7BFF
    assert oracle.f32_to_f16(65519.0) == 0x7BFF
    assert oracle.f32_to_f16(65520.0) == 0x7C00
    assert oracle.f32_to_f16(2.0 ** -25) == 0x0000          # half of the smallest subnormal: even
    assert oracle.f32_to_f16(3 * 2.0 ** -25) == 0x0002       # 1.5 ulp -> 2 (even)
    assert oracle.f32_to_f16(float("nan")) & 0x7C00 == 0x7C00


def test_reference_encoder_rounds_ties_up_and_nan_to_inf(oracle):
    # f16.ts:16-17 adds 0x2000 whenever bit 12 is set: ties go up in magnitude, not to even.
    assert oracle.ref_float_to_half(1.0 + 2.0 ** -11) == 0x3C01
    assert oracle.ref_float_to_half(-(1.0 + 2.0 ** -11)) == 0xBC01
    assert oracle.ref_float_to_half(float("nan")) == 0x7C00          # f16.ts:15
    assert oracle.ref_float_to_half(1.0) == 0x3C00
    assert oracle.ref_float_to_half(65520.0) == 0x7C00
    # Off ties it agrees with IEEE RNE (numpy): sample values with no tie bit pattern.
    rng = np.random.default_rng(3)
    x = rng.standard_normal(5000).astype(np.float32)
    bits = x.view(np.uint32)
    off_tie = (bits & 0x1FFF) != 0x1000
    want = x.astype(np.float16).view(np.uint16)
    got = np.array([oracle.ref_float_to_half(float(v)) for v in x])
    assert np.array_equal(got[off_tie], want[off_tie])


# ---------------------------------------------------------------------------------------------
# generator
# ---------------------------------------------------------------------------------------------

def test_splitmix64_published_vectors(oracle):
    # Published SplitMix64 outputs for seed 1234567 (Vigna's splitmix64.c test sequence).
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423,
            4593380528125082431, 16408922859458223821]
    assert [oracle.lib().orc_rand_u64(1234567, i) for i in range(5)] == want


def test_normal_draws_are_standard_normal(oracle):
    from scipy import stats
    x = f16(oracle.normal_f16(oracle.seed(9, 9, 0), 200000))
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    assert stats.kstest(x, "norm").pvalue > 1e-3
    # even and odd indices (cos and sin halves of each Box-Muller pair) are uncorrelated
    assert abs(np.corrcoef(x[0::2], x[1::2])[0, 1]) < 0.01


def test_seed_layout(oracle):
    assert oracle.seed(0, 0, 0) == 0x51574E3300000000
    assert oracle.seed(4, 27, 2) == 0x51574E3300000000 | (4 << 16) | (27 << 8) | 2


def test_rope_table_closed_form(oracle):
    c, s = oracle.rope_table(5)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    assert c[1, 0] == np.float32(math.cos(1.0)) and s[1, 0] == np.float32(math.sin(1.0))
    # i = 32 -> theta^(-1/2) = 1e-3 (model.ts:78: exponent is -i/64)
    assert abs(float(s[4, 32]) - math.sin(4e-3)) < 1e-9
    assert abs(float(c[3, 63]) - math.cos(3 * 1e6 ** (-63 / 64))) < 1e-7


def test_qk_norm_rope_matches_complex_rotation(oracle):
    rng = np.random.default_rng(11)
    T = 9
    x = to_bits(rng.standard_normal((T, 3 * 128)) * 3.0)
    cu = np.array([0, 4, 9], dtype=np.int32)
    y = oracle.qk_norm_rope(x.copy(), cu, heads=3)
    xf = f16(x).reshape(T, 3, 128)
    rms = np.sqrt((xf ** 2).mean(-1, keepdims=True) + 1e-6)
    n = xf / rms
    pos = np.array([0, 1, 2, 3, 0, 1, 2, 3, 4])  # positions restart per sequence
    ang = pos[:, None] * 1e6 ** (-np.arange(64) / 64.0)
    z = (n[..., :64] + 1j * n[..., 64:]) * np.exp(1j * ang)[:, None, :]
    want = np.concatenate([z.real, z.imag], axis=-1)
    got = f16(y).reshape(T, 3, 128)
    assert np.max(np.abs(got - want)) <= 2.0 ** -10 * np.max(np.abs(want)) * 1.01
    # position 0 is the bare RMSNorm
    assert np.array_equal(y.reshape(T, 3, 128)[0], to_bits(n[0]))


def test_qk_norm_rope_relative_position_property(oracle):
    # <rope(q, m), rope(k, n)> depends only on m - n.
    rng = np.random.default_rng(5)
    q = rng.standard_normal(128)
    k = rng.standard_normal(128)
    rows = np.stack([q if i % 2 == 0 else k for i in range(16)])
    x = to_bits(rows)
    y = f16(oracle.qk_norm_rope(x.copy(), np.array([0, 16], np.int32), heads=1))
    d1 = y[4] @ y[1]   # q at 4, k at 1: distance 3
    d2 = y[10] @ y[7]  # q at 10, k at 7: distance 3
    assert abs(d1 - d2) < 0.02 * 128 ** 0.5


def test_gen_lengths_range(oracle):
    L = oracle.gen_lengths(oracle.seed(1, 0, 3), 1000)
    assert L.min() >= 10 and L.max() <= 150 and len(set(L.tolist())) > 100


# ---------------------------------------------------------------------------------------------
# mask  (reference: ops.ts:205-209, 219-220)
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("L", [1, 2, 50, 175, 176, 177, 431, 432, 433, 500, 607, 608, 609, 1500, 5000])
def test_mask_pair_count_closed_form(oracle, L):
    n = min(L, 608)
    assert oracle.mask_pairs(L) == n * (n + 1) // 2 + max(0, L - 608) * 608
    assert oracle.mask_pairs(L, MASK_CAUSAL) == L * (L + 1) // 2


def test_mask_known_pairs(oracle):
    r = oracle.retained
    assert r(607, 176, 5000) and r(608, 175, 5000) and r(608, 177, 5000)
    assert not r(608, 176, 5000)            # first excluded key
    assert r(5000 - 1, 5000 - 432, 5000) and not r(4999, 4999 - 432, 5000)
    assert not r(10, 11, 5000) and not r(10, 3, 10)   # causal; q >= S


@pytest.mark.parametrize("L,P,W", [(700, 176, 432), (300, 7, 50), (129, 0, 33), (90, 64, 1), (40, 176, 432)])
def test_mask_bits_vs_numpy_definition(oracle, L, P, W):
    q = np.arange(L)[:, None]
    k = np.arange(L)[None, :]
    want = (k <= q) & ((k < P) | (q - k < W))
    bits = oracle.mask_bits(L, MASK_PREFIX_LOCAL, P, W)
    got = np.unpackbits(bits.view(np.uint8), axis=1, bitorder="little")[:, :L].astype(bool)
    assert np.array_equal(got, want)


def test_reference_tile_skip_never_drops_a_retained_key(oracle):
    # ops.ts:207-209 skips 16-key tiles using the tile's first query; prove it is conservative
    # and that it does skip at long lengths.
    for S in (608, 700, 1500):
        skipped = 0
        for q0 in range(0, S, 16):
            for kb in range(0, min(S, q0 + 16), 16):
                if oracle.ref_tile_skipped(S, q0, kb):
                    skipped += 1
                    for q in range(q0, min(S, q0 + 16)):
                        for k in range(kb, kb + 16):
                            assert not oracle.retained(q, k, S)
        assert (skipped > 0) == (S > 608)  # below 609 tokens the mask is plain causal


# ---------------------------------------------------------------------------------------------
# exact attention
# ---------------------------------------------------------------------------------------------

def _rand_qkv(rng, T, scale=1.0):
    q = to_bits(rng.standard_normal((T, 2048)) * scale)
    k = to_bits(rng.standard_normal((T, 1024)) * scale)
    v = to_bits(rng.standard_normal((T, 1024)))
    return q, k, v


def test_exact_constant_v_gives_constant(oracle):
    rng = np.random.default_rng(1)
    q, k, _ = _rand_qkv(rng, 40)
    v = to_bits(np.full((40, 1024), 0.75))
    o = oracle.attention_exact(q, k, v, [0, 40])
    assert np.allclose(o, 0.75, atol=1e-12)


def test_exact_zero_q_gives_mean_of_retained_v(oracle):
    rng = np.random.default_rng(2)
    T = 700
    _, k, v = _rand_qkv(rng, T)
    q = np.zeros((T, 2048), dtype=np.uint16)
    o = oracle.attention_exact(q, k, v, [0, T], rows=[0, 5, 607, 608, 699])
    vf = f16(v).reshape(T, 8, 128)
    for i, t in enumerate([0, 5, 607, 608, 699]):
        keys = [kk for kk in range(t + 1) if kk < 176 or t - kk < 432]
        want = vf[keys].mean(0)                        # [8,128]
        want = np.repeat(want, 2, axis=0)              # q head h reads kv head h // 2
        assert np.allclose(o[i], want, atol=1e-12)


def test_exact_first_row_is_v0_with_gqa_mapping(oracle):
    rng = np.random.default_rng(3)
    q, k, v = _rand_qkv(rng, 8)
    o = oracle.attention_exact(q, k, v, [0, 8], rows=[0])[0]
    vf = f16(v[0]).reshape(8, 128)
    for h in range(16):
        assert np.array_equal(o[h], vf[h // 2])


def test_exact_single_dominant_key(oracle):
    rng = np.random.default_rng(4)
    T = 30
    q, k, v = _rand_qkv(rng, T, scale=0.01)
    kf = f16(k).reshape(T, 8, 128).copy()
    kf[17] = 8.0
    k = to_bits(kf.reshape(T, 1024))
    q = to_bits(np.full((T, 2048), 8.0))
    o = oracle.attention_exact(q, k, v, [0, T], rows=[29])[0]
    vf = f16(v).reshape(T, 8, 128)
    assert np.allclose(o, np.repeat(vf[17], 2, axis=0), atol=1e-9)


@pytest.mark.parametrize("lengths,P,W", [([50], 176, 432), ([13, 1, 70, 33], 176, 432), ([700, 9], 176, 432),
                                          ([200], 20, 60)])
def test_exact_vs_torch_sdpa_float64(oracle, lengths, P, W):
    import torch
    rng = np.random.default_rng(sum(lengths))
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    T = int(cu[-1])
    q, k, v = _rand_qkv(rng, T)
    got = oracle.attention_exact(q, k, v, cu, MASK_PREFIX_LOCAL, P, W)
    qf = torch.from_numpy(f16(q).reshape(T, 16, 128))
    kf = torch.from_numpy(f16(k).reshape(T, 8, 128)).repeat_interleave(2, dim=1)
    vf = torch.from_numpy(f16(v).reshape(T, 8, 128)).repeat_interleave(2, dim=1)
    for s in range(len(lengths)):
        a, b = int(cu[s]), int(cu[s + 1])
        L = b - a
        qi = torch.arange(L)[:, None]
        ki = torch.arange(L)[None, :]
        m = (ki <= qi) & ((ki < P) | (qi - ki < W))
        want = torch.nn.functional.scaled_dot_product_attention(
            qf[a:b].transpose(0, 1), kf[a:b].transpose(0, 1), vf[a:b].transpose(0, 1),
            attn_mask=m).transpose(0, 1).numpy()
        assert np.max(np.abs(got[a:b] - want)) < 1e-10


def test_exact_varlen_equals_solo_and_isolation(oracle):
    rng = np.random.default_rng(6)
    lengths = [17, 64, 5]
    cu = np.array([0, 17, 81, 86], dtype=np.int32)
    q, k, v = _rand_qkv(rng, 86)
    packed = oracle.attention_exact(q, k, v, cu)
    solo = oracle.attention_exact(q[17:81].copy(), k[17:81].copy(), v[17:81].copy(), [0, 64])
    assert np.array_equal(packed[17:81], solo)
    k2, v2 = k.copy(), v.copy()
    k2[81:] = to_bits(rng.standard_normal((5, 1024)))
    v2[:17] = to_bits(rng.standard_normal((17, 1024)))
    pert = oracle.attention_exact(q, k2, v2, cu)
    assert np.array_equal(pert[17:81], packed[17:81])


def test_exact_interleaved_v_layout(oracle):
    # The reference reads V in place from qkvRaw: stride 4096, offset 3072 (model.ts:95).
    rng = np.random.default_rng(8)
    q, k, v = _rand_qkv(rng, 20)
    raw = np.zeros((20, 4096), dtype=np.uint16)
    raw[:, 3072:] = v
    a = oracle.attention_exact(q, k, v, [0, 20])
    b = oracle.attention_exact(q, k, raw, [0, 20], v_offset=3072)
    assert np.array_equal(a, b)


# ---------------------------------------------------------------------------------------------
# f16-faithful restatement of the reference's tiled kernel
# ---------------------------------------------------------------------------------------------

def test_tiled16_first_row_exact_and_two_key_f16_average(oracle):
    rng = np.random.default_rng(9)
    _, k, v = _rand_qkv(rng, 2)
    q = np.zeros((2, 2048), dtype=np.uint16)
    o = oracle.attention_tiled16(q, k, v, [0, 2]).reshape(2, 16, 128)
    for h in range(16):
        assert np.array_equal(o[0, h], v[0].reshape(8, 128)[h // 2])
    # row 1, Q = 0: weights (1, 1), den 2, total = f16(v0 + v1), O = f16(total / 2)
    v16 = v.view(np.float16).reshape(2, 8, 128)
    want = ((v16[0] + v16[1]) / np.float16(2)).astype(np.float16)
    assert np.array_equal(o[1].view(np.float16), np.repeat(want, 2, axis=0))


@pytest.mark.parametrize("lengths", [[50], [33, 100, 7], [700]])
def test_tiled16_vs_exact_within_f16_accumulation_error(oracle, lengths):
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    q, k, v = oracle.gen_qkv(0, 0, cu)
    ex = oracle.attention_exact(q, k, v, cu)
    tl = f16(oracle.attention_tiled16(q, k, v, cu)).reshape(ex.shape)
    err = np.abs(tl - ex)
    assert err.max() < 1e-2
    cos = (tl * ex).sum(-1) / (np.linalg.norm(tl, axis=-1) * np.linalg.norm(ex, axis=-1))
    assert cos.min() > 0.9995


def test_tiled16_varlen_equals_padded_reference_layout(oracle):
    # The reference pads every request to the batch maximum (embedding-engine.ts:62-69) and runs
    # sequence = max; valid rows must not depend on the padding, so the per-sequence restatement
    # equals the padded one on valid rows.
    rng = np.random.default_rng(10)
    lens = [20, 37]
    q, k, v = _rand_qkv(rng, 57)
    packed = oracle.attention_tiled16(q, k, v, [0, 20, 57])
    S = 37
    qp = np.zeros((2 * S, 2048), np.uint16); kp = np.zeros((2 * S, 1024), np.uint16)
    vp = np.zeros((2 * S, 1024), np.uint16)
    qp[:20], kp[:20], vp[:20] = q[:20], k[:20], v[:20]
    qp[S:], kp[S:], vp[S:] = q[20:], k[20:], v[20:]
    # padded batch: each sequence occupies S rows; valid rows are the first len rows.
    padded = oracle.attention_tiled16(qp, kp, vp, [0, S, 2 * S])
    # In the padded layout sequence 0 sees its padding rows as keys > q (masked) -- same result.
    assert np.array_equal(padded[:20], packed[:20])
    assert np.array_equal(padded[S:], packed[20:])


# ---- last-token pool + L2 norm (ops.ts:347-379) -------------------------------------------------

def test_pool_closed_forms(oracle):
    # A row of 3, 4, zeros -> 0.6, 0.8, zeros; a constant row c of width W -> sign(c)/sqrt(W).
    x = np.zeros((3, 1024), np.float16)
    x[0, :2] = [3, 4]
    x[1, :] = -0.5
    x[2, :] = 2.0
    out = oracle.pool_last_l2(x, [0, 1, 2, 3])
    assert np.allclose(out[0, :2], [0.6, 0.8], rtol=0, atol=1e-15) and not out[0, 2:].any()
    assert np.allclose(out[1], -1 / math.sqrt(1024), rtol=0, atol=1e-15)
    assert np.allclose(out[2], 1 / math.sqrt(1024), rtol=0, atol=1e-15)


def test_pool_reads_the_last_row_of_each_sequence(oracle):
    # Rows differ in where their mass is, so pooling any other row (the first, or the next
    # sequence's) gives a different unit vector.
    lengths = [1, 4, 2, 7]
    cu = np.concatenate([[0], np.cumsum(lengths)])
    x = np.zeros((cu[-1], 64), np.float16)
    for t in range(cu[-1]):
        x[t, t % 64] = 1.0 + t
    out = oracle.pool_last_l2(x, cu)
    for i in range(len(lengths)):
        last = cu[i + 1] - 1
        want = np.zeros(64)
        want[last % 64] = 1.0
        assert np.array_equal(out[i], want)


def test_pool_unit_norm_and_scale_invariance(oracle):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((40, 2048)).astype(np.float16)
    cu = [0, 9, 9, 25, 40]  # includes an empty sequence
    out = oracle.pool_last_l2(x, cu)
    norms = np.sqrt(np.sum(out * out, axis=1))
    assert np.allclose(norms[[0, 2, 3]], 1.0, rtol=0, atol=1e-12)
    assert not out[1].any()  # empty sequence: zeros
    # scaling a row by a power of two is exact in fp16 and leaves the unit vector unchanged
    assert np.array_equal(oracle.pool_last_l2(x * np.float16(8), cu), out)
    # width restricts the columns
    part = oracle.pool_last_l2(x, cu, width=1024)
    assert np.allclose(np.sqrt(np.sum(part[[0, 2, 3]] ** 2, axis=1)), 1.0, atol=1e-12)


def test_pool_zero_row_gives_nan_as_the_reference(oracle):
    # inverseSqrt(0) is +inf in the reference and 0 * inf = NaN: no epsilon (ops.ts:362-363).
    out = oracle.pool_last_l2(np.zeros((2, 16), np.float16), [0, 2])
    assert np.isnan(out).all()


# ---- Q4_0 tile32-compact packing and dequant-GEMM (format.ts:64-96, quant-matmul.ts) ----------

def _q40_block(scale_bits, quants):
    b = bytearray(18)
    b[0:2] = bytes(scale_bits)
    for i in range(16):
        b[2 + i] = quants[i] | (quants[i + 16] << 4)
    return bytes(b)


def test_pack_q40_tile32_reference_vector(oracle):
    # The reference's own test (tests/prepacked-format.test.ts:13-22): two one-row parts.
    first = _q40_block([0x00, 0x3C], [i & 15 for i in range(32)])
    second = _q40_block([0x00, 0x40], [15 - (i & 15) for i in range(32)])
    packed, k, n = oracle.pack_q40_tile32([(32, 1, first), (32, 1, second)])
    assert (k, n) == (32, 2) and packed.size == 32 * 20
    assert list(packed[0:8]) == [0x00, 0x3C, 0x00, 0x00, 0x00, 0x11, 0x22, 0x33]
    assert list(packed[20:28]) == [0x00, 0x40, 0x00, 0x00, 0xFF, 0xEE, 0xDD, 0xCC]
    assert not packed[40:].any()  # rows 2..31 of the tile are zero


def test_q40_weights_closed_form(oracle):
    # Scale 1.0 (0x3C00) and quants q -> q - 8; scale 2.0 (0x4000) and 15 - q -> 2 * (7 - q).
    first = _q40_block([0x00, 0x3C], [i & 15 for i in range(32)])
    second = _q40_block([0x00, 0x40], [15 - (i & 15) for i in range(32)])
    packed, k, n = oracle.pack_q40_tile32([(32, 1, first), (32, 1, second)])
    w = oracle.q40_compact_weights(packed, k, n).astype(np.float64)
    assert np.array_equal(w[0], [(i & 15) - 8 for i in range(32)])
    assert np.array_equal(w[1], [2 * (7 - (i & 15)) for i in range(32)])


def test_q40_tile_order_across_tiles_and_k_blocks(oracle):
    # 70 rows (3 tiles, the last partial) x 96 columns (3 K blocks): every (row, k block) gets its
    # own scale, so a transposed tile / block / row index gives different weights.
    rng = np.random.default_rng(5)
    n, k = 70, 96
    rows = []
    for r in range(n):
        for kb in range(k // 32):
            scale = np.array([1 + r + 0.25 * kb], np.float16).view(np.uint8)
            rows.append(_q40_block(list(scale), list(rng.integers(0, 16, 32))))
    raw = b"".join(rows)
    packed, _, _ = oracle.pack_q40_tile32([(k, 40, raw[:40 * 3 * 18]), (k, 30, raw[40 * 3 * 18:])])
    assert packed.size == 3 * 3 * 32 * 20
    w = oracle.q40_compact_weights(packed, k, n).astype(np.float64)
    src = np.frombuffer(raw, np.uint8).reshape(n, 3, 18)
    for r in (0, 31, 32, 45, 69):
        for kb in range(3):
            scale = float(src[r, kb, 0:2].copy().view(np.float16)[0])
            q = src[r, kb, 2:18]
            want = np.concatenate([(q & 15), (q >> 4)]).astype(np.float64) - 8
            assert np.array_equal(w[r, 32 * kb:32 * kb + 32], np.float16(want * scale).astype(np.float64))


def test_q4_matmul_against_dense_product(oracle):
    rng = np.random.default_rng(9)
    m, k, n = 5, 64, 33
    blocks = []
    for r in range(n):
        for kb in range(2):
            blocks.append(_q40_block(list(np.array([rng.uniform(0.01, 0.1)], np.float16).view(np.uint8)),
                                     list(rng.integers(0, 16, 32))))
    packed, _, _ = oracle.pack_q40_tile32([(k, n, b"".join(blocks))])
    x = rng.standard_normal((m, k)).astype(np.float16)
    w = oracle.q40_compact_weights(packed, k, n).astype(np.float64)
    y = oracle.q4_matmul(x, packed, k, n)
    for i in range(m):
        for j in range(n):
            assert abs(y[i, j] - sum(float(x[i, c]) * w[j, c] for c in range(k))) < 1e-12
