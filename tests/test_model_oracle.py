"""CPU checks of the model-forward oracle (oracle/model_ref.py) before it judges the device:
the reference's own Q6_K vector, two independent restatements of the Q6_K decoder, closed forms of
RMSNorm and SwiGLU, and invariants of the whole forward that a wrong stage order, norm or residual
would break."""
import numpy as np
import pytest

import model_ref as mr


def test_q6k_reference_vector():
    # tests/quantization.test.ts:35-41: codes 0 (-> -32), all scales 1, d = 1 -> every value -32.
    blk = np.zeros(210, np.uint8)
    blk[192:208] = 1
    blk[208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    table = np.tile(blk, 4)                      # one 1024-wide row = 4 blocks
    assert np.all(mr.q6k_rows(table, [0]) == -32)


def test_q6k_decoders_agree():
    # quantization.ts:46-70 (vectorised) against the shader's index arithmetic (ops.ts:390-401).
    rng = np.random.default_rng(3)
    table = mr.q6k_table(rng, 6)
    ids = [0, 5, 2]
    assert np.array_equal(mr.q6k_rows(table, ids), mr.q6k_rows_shader_form(table, ids))


def test_q6k_single_fields():
    # One block, d = 2, scale j of the 16 = j + 1: value 128h + 32quad + l is 2 * scale * (q - 32)
    # with the code assembled from one low nibble and two high bits chosen here per element.
    blk = np.zeros(210, np.uint8)
    blk[192:208] = np.arange(1, 17, dtype=np.uint8)
    blk[208:210] = np.frombuffer(np.float16(2.0).tobytes(), np.uint8)
    blk[0] = 0x5A      # ql[0]: low nibble 10 (h0 quad0 l0), high nibble 5 (h0 quad2 l0)
    blk[32] = 0x3C     # ql[32]: low nibble 12 (h0 quad1 l0), high nibble 3 (h0 quad3 l0)
    blk[128] = 0b11100100  # qh[0]: quad0 bits 00, quad1 01, quad2 10, quad3 11
    row = mr.q6k_rows(np.tile(blk, 4), [0])[0]
    assert row[0] == 2 * 1 * ((10 | 0 << 4) - 32)
    assert row[32] == 2 * 3 * ((12 | 1 << 4) - 32)
    assert row[64] == 2 * 5 * ((5 | 2 << 4) - 32)
    assert row[96] == 2 * 7 * ((3 | 3 << 4) - 32)
    assert row[16] == 2 * 2 * (0 - 32)          # l = 16 takes scale 8h + 1
    assert row[128] == 2 * 9 * (0 - 32)         # h = 1 takes scales from 8


def test_embed_rounds_like_the_shader():
    rng = np.random.default_rng(4)
    table = mr.q6k_table(rng, 3)
    exact = mr.q6k_rows(table, [1])
    got = mr.embed(table, [1])
    assert got.dtype == np.float16
    # the f32 product is exact (d: 11 bits, scale: 8, code: 6), so this is round-to-nearest f16
    assert np.array_equal(got, exact.astype(np.float16))


def test_rmsnorm_closed_forms():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((8, 1024)).astype(np.float16)
    ones = np.ones(1024, np.float32)
    xn, out = mr.rmsnorm(x, None, ones)
    assert np.array_equal(xn, x)                          # no residual: x untouched
    rms = np.sqrt(np.mean(out.astype(np.float64) ** 2, axis=1))
    assert np.allclose(rms, 1.0, atol=2e-3)               # unit gain: unit RMS (fp16 rounding)
    c = np.full((1, 1024), 3.0, np.float16)
    _, oc = mr.rmsnorm(c, None, ones, eps=0.0)
    assert np.all(oc == 1.0)                              # a constant row normalises to 1
    r = rng.standard_normal((8, 1024)).astype(np.float16)
    xr, out_r = mr.rmsnorm(x, r, 2 * ones)
    assert np.array_equal(xr, (x.astype(np.float64) + r.astype(np.float64)).astype(np.float16))
    _, out_sum = mr.rmsnorm(xr, None, 2 * ones)
    assert np.max(np.abs(out_r.astype(np.float64) - out_sum.astype(np.float64))) <= 2e-2  # gain 2


def test_swiglu_closed_forms():
    g = np.array([0.0, 1.0, 10.0, -20.0, 2.0], np.float16)
    u = np.array([5.0, 1.0, 1.0, 1.0, 0.0], np.float16)
    out = mr.swiglu(np.concatenate([g, u])[None, :], width=5)[0].astype(np.float64)
    assert out[0] == 0.0 and out[4] == 0.0
    assert abs(out[1] - 0.7310585786300049) <= 2 ** -11      # silu(1) = 1 / (1 + e^-1)
    assert abs(out[2] - 10.0) <= 2 ** -7                     # silu(g) -> g for large g
    assert abs(out[3]) <= 1e-7                               # silu(g) -> 0 for very negative g


@pytest.fixture(scope="module")
def small_model():
    return mr.synthetic_weights(11, 2, vocab=96)


def _zero_projections(w):
    z = dict(w)
    layers = []
    for lw in w["layers"]:
        lz = dict(lw)
        for name in ("attn_qkv", "attn_output", "ffn_gate_up", "ffn_down"):
            packed, k, n = lw[name]
            p = np.array(packed, copy=True).reshape(-1, 20)
            p[:, 0:2] = 0                                       # every block scale 0
            lz[name] = (p.reshape(-1), k, n)
        layers.append(lz)
    z["layers"] = layers
    return z


def test_forward_with_zero_projections_is_the_normalised_embedding(small_model):
    # Every projection 0 -> every residual delta 0: x stays the embedding and the pooled row is
    # the last token's embedding through the final norm (output_norm gain), L2-normalised.
    w = _zero_projections(small_model)
    cu = np.array([0, 3, 10], np.int32)
    ids = np.arange(10, dtype=np.int32) * 7 % 96
    got = mr.forward(w, ids, cu)
    for i in range(2):
        e = mr.embed(w["token_embd"], [ids[cu[i + 1] - 1]])
        _, n = mr.rmsnorm(e, None, w["output_norm"])
        v = n[0].astype(np.float64)
        assert np.allclose(got[i], v / np.linalg.norm(v), atol=1e-12)


def test_forward_sequences_are_independent(small_model):
    # Attention stays inside each packed sequence: changing sequence 1's tokens leaves 0 and 2.
    cu = np.array([0, 6, 20, 29], np.int32)
    rng = np.random.default_rng(6)
    ids = rng.integers(0, 96, 29).astype(np.int32)
    a = mr.forward(small_model, ids, cu)
    ids2 = ids.copy()
    ids2[6:20] = (ids2[6:20] + 1) % 96
    b = mr.forward(small_model, ids2, cu)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[2], b[2])
    assert not np.array_equal(a[1], b[1])
    # and a sequence alone gives what it gives inside the batch
    solo = mr.forward(small_model, ids[20:29], np.array([0, 9], np.int32))
    assert np.array_equal(solo[0], a[2])
