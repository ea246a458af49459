"""CPU checks of the committed golden fixtures (tests/golden/, written by make_golden.py).

- The reference's own vectors (binary16 KATs, tests/quantization.test.ts:5-9) hold for the
  oracle's decoders.  The packer vectors (tests/embedding-engine.test.ts:5-36) are driven through
  the Node engine by tests/js/engine.test.js.
- The oracle still generates the exact Q/K/V bytes the fixture hashes name.
- The golden attention rows are pinned twice: the oracle reproduces them bit for bit, and an
  independent numpy float64 brute force (its own mask predicate, restated from
  src/webgpu/ops.ts:205-220 of the reference) lands within half an fp16 ulp of them.
"""
import hashlib
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
HQ, HKV, HD = 16, 8, 128


def load_json(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def golden():
    with np.load(os.path.join(GOLDEN, "attention_golden.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).astype("<u2", copy=False).tobytes()).hexdigest()


def test_manifest_matches_fixture_files():
    with open(os.path.join(GOLDEN, "MANIFEST.sha256")) as f:
        lines = [ln.split() for ln in f if ln.strip()]
    assert len(lines) == 3
    for digest, name in lines:
        with open(os.path.join(GOLDEN, name), "rb") as g:
            assert hashlib.sha256(g.read()).hexdigest() == digest, name


def test_reference_f16_decode_kats(oracle):
    cases = load_json("reference_vectors.json")["f16_decode"]["cases"]
    assert len(cases) == 3
    for bits, want in cases:
        assert oracle.f16_to_f32(bits) == want
        assert oracle.ref_half_to_float(bits) == want


@pytest.mark.parametrize("config", [0, 1, 2, 3, 4])
def test_generator_bytes_match_fixture_hashes(oracle, config):
    from golden.make_golden import config_lengths, cu_of
    hashes = load_json("generator_sha256.json")
    lengths = config_lengths(config)
    if config == 1:
        assert lengths == hashes["cfg1_lengths"]
        assert all(10 <= n <= 150 for n in lengths) and len(lengths) == 16
    cu = cu_of(lengths)
    for layer in ([0, 27] if config >= 2 else [0]):
        q, k, v = oracle.gen_qkv(config, layer, cu)
        for name, a in (("q", q), ("k", k), ("v", v)):
            assert sha(a) == hashes["arrays"][f"cfg{config}/layer{layer}/{name}"], (config, layer, name)


def brute_force_rows(q, k, v, cu, rows, P=176, W=432):
    """float64 softmax(mask(q k^T) / sqrt(128)) v for the given rows, in numpy."""
    f = lambda a: a.view(np.float16).astype(np.float64)
    out = np.empty((len(rows), HQ, HD))
    for i, r in enumerate(rows):
        s = int(np.searchsorted(cu, r, side="right") - 1)
        b, S = int(cu[s]), int(cu[s + 1] - cu[s])
        qp = r - b
        kp = np.arange(S)
        keep = (kp <= qp) & ((kp < min(S, P)) | (kp + min(S, W) > qp))
        keys = b + kp[keep]
        qr = f(q[r]).reshape(HQ, HD)
        kk = f(k[keys]).reshape(-1, HKV, HD)
        vv = f(v[keys]).reshape(-1, HKV, HD)
        for h in range(HQ):
            sc = kk[:, h // 2, :] @ qr[h] / np.sqrt(HD)
            w = np.exp(sc - sc.max())
            out[i, h] = (w[:, None] * vv[:, h // 2, :]).sum(0) / w.sum()
    return out


def half_ulp(x):
    """Half the fp16 spacing at |x| (normal range), the largest RNE rounding error."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -14)))
    return 2.0 ** (e - 11)


@pytest.mark.parametrize("config", [0, 1, 2, 3, 4])
def test_golden_rows_oracle_bit_exact_and_brute_force(oracle, golden, config):
    from golden.make_golden import config_lengths, cu_of
    cu = cu_of(config_lengths(config))
    assert np.array_equal(golden[f"cfg{config}_cu"], cu)
    rows = golden[f"cfg{config}_rows"]
    want = golden[f"cfg{config}_out"]
    q, k, v = oracle.gen_qkv(config, 0, cu)
    exact = oracle.attention_exact(q, k, v, cu, 1, 176, 432, rows=rows)
    assert np.array_equal(exact.reshape(len(rows), -1).astype(np.float16).view(np.uint16), want)
    # Independent float64 restatement: within half an fp16 ulp (plus f64 noise) of the fixture.
    sub = rows if len(rows) <= 16 else rows[:: max(1, len(rows) // 16)]
    idx = np.searchsorted(rows, sub) if np.all(np.diff(rows) > 0) else np.arange(len(sub))
    bf = brute_force_rows(q, k, v, cu, sub).reshape(len(sub), -1)
    g = want[idx].view(np.float16).astype(np.float64)
    assert np.all(np.abs(bf - g) <= half_ulp(bf) * (1 + 1e-6) + 1e-12)


def test_golden_cfg0_first_row_is_v0(golden):
    # Row 0 attends only to key 0: O = V[0] for every query head, read from KV head h // 2.
    from golden.make_golden import cu_of
    import oracle as orc
    q, k, v = orc.gen_qkv(0, 0, cu_of([50]))
    row0 = golden["cfg0_out"][0].reshape(HQ, HD)
    assert np.array_equal(row0, np.repeat(v[0].reshape(HKV, HD), 2, axis=0))


def test_golden_tiled16_restatement_hash(oracle, golden):
    from golden.make_golden import cu_of
    cu = cu_of([50])
    q, k, v = oracle.gen_qkv(0, 0, cu)
    tiled = oracle.attention_tiled16(q, k, v, cu)
    assert sha(tiled) == bytes(golden["cfg0_tiled16_sha256"]).decode()
