"""GPU runs of BASELINE configs 0-4 (layer 0) against the committed golden rows.

The golden rows (tests/golden/attention_golden.npz) are the exact attention output rounded to
fp16; tests/test_golden.py pins them against the oracle and an independent numpy brute force.
Each comparison allows the 2e-3 bar plus the fixture's own half-ulp rounding, and asks for
per-row cosine >= 0.9999.  Inputs come from the oracle generator, whose bytes match the fixture's
SHA-256 hashes; one case uses the device generator instead.
"""
import hashlib
import json
import os

import numpy as np
import pytest

from test_gpu_parity import ATOL, MIN_COS, Case, f16

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def golden():
    with np.load(os.path.join(GOLDEN, "attention_golden.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="module")
def hashes():
    with open(os.path.join(GOLDEN, "generator_sha256.json")) as f:
        return json.load(f)["arrays"]


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).astype("<u2", copy=False).tobytes()).hexdigest()


def compare_golden(got_bits, want_bits, label):
    got, want = f16(got_bits), f16(want_bits)
    err = np.abs(got - want)
    e = np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -14)))
    allow = ATOL + 2.0 ** (e - 11)
    cos = (got * want).sum(-1) / np.maximum(np.linalg.norm(got, axis=-1) *
                                           np.linalg.norm(want, axis=-1), 1e-300)
    print(f"[{label}] max|err| {err.max():.3e}  min cos {cos.min():.7f}", flush=True)
    assert np.isfinite(got).all(), label
    assert np.all(err <= allow), (label, err.max())
    assert cos.min() >= MIN_COS, (label, cos.min())


# (config, flags, mask, o_last).  Configs 0-2 never exceed 608 tokens, where the prefix/local
# mask equals full causal, so both mask kinds must reproduce the same golden rows; (2, 0, 0, False)
# is exactly the launch bench.py times for its 16 x 500 line (causal kind, no flags, no o_last).
@pytest.mark.parametrize("config,flags,mask,o_last", [
    (0, 0, 1, True), (1, 0, 1, True), (2, 0, 1, True), (3, 0, 1, True), (3, 1, 1, True),
    (4, 0, 1, True), (4, 1, 1, True), (2, 0, 0, False), (1, 0, 0, False)])
def test_config_rows_match_golden(ctx, qattn, oracle, golden, hashes, config, flags, mask, o_last):
    cu = golden[f"cfg{config}_cu"].astype(np.int32)
    rows = golden[f"cfg{config}_rows"]
    print(f"golden cfg{config} flags {flags} mask {mask} o_last {o_last}: lengths "
          f"{np.diff(cu).tolist()[:4]}... rows {len(rows)}", flush=True)
    q, k, v = oracle.gen_qkv(config, 0, cu)
    for name, a in (("q", q), ("k", k), ("v", v)):
        assert sha(a) == hashes[f"cfg{config}/layer0/{name}"], name
    case = Case(ctx, qattn, q, k, v, cu, mask=mask, o_last=o_last, flags=flags)
    got = case.run()
    compare_golden(got[rows], golden[f"cfg{config}_out"], f"cfg{config} flags {flags} mask {mask}")
    if not o_last:
        case.free()
        return
    last = case.last()
    ends = cu[1:] - 1
    # o_last holds exactly the last output row of each sequence.
    assert np.array_equal(last, got[ends])
    hit = np.isin(rows, ends)
    if hit.any():
        compare_golden(last[np.searchsorted(ends, rows[hit])], golden[f"cfg{config}_out"][hit],
                       f"cfg{config} last rows")
    case.free()


def test_device_generator_config2_matches_golden(ctx, qattn, golden):
    # The whole device path: qattn_gen_qkv makes the 16x500 inputs on the GPU, then attention.
    cu = golden["cfg2_cu"].astype(np.int32)
    T = int(cu[-1])
    bq, bk, bv = ctx.alloc(T * 4096), ctx.alloc(T * 2048), ctx.alloc(T * 2048)
    bo, bl = ctx.alloc(T * 4096), ctx.alloc(16 * 4096)
    ctx.gen_qkv(2, 0, cu, bq.ptr, bk.ptr, bv.ptr)
    desc = qattn.make_desc(bq.ptr, bk.ptr, bv.ptr, bo.ptr, cu, 1, 176, 432, o_last=bl.ptr)
    ctx.prefill(desc)
    last = bl.read(np.uint16, (16, 2048))
    compare_golden(last, golden["cfg2_out"], "cfg2 device generator")
    for b in (bq, bk, bv, bo, bl):
        b.free()
