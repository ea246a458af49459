"""Seeded random sweeps on the GPU, beside the hand-picked cases of test_gpu_parity / test_gpu_q4.

Attention: random ragged packings (1-16 sequences, up to 12,000 tokens, single tokens to 4,000-
token sequences), causal or prefix/local masks with random prefix and window, split-K or
batch-invariant plans, compact or qkvRaw value layout, with or without last-token rows.  Each case
is checked against the f64 oracle on sampled rows (every sequence's first and last row plus
random ones) to the north-star bar, its last-token rows against its output rows, and its
executed mask (qattn_debug_run_mask) against the reference predicate bit for bit.

Q4_0 GEMM: random shapes (M 1-3,000, K 32-4,096 in steps of 32, N 1-4,100; the plain and the
fused gate/up + SwiGLU projection), checked on sampled rows against the oracle's exact product
within the fp32-summation bound, and for row invariance: the first rows of a shorter launch of the
same rows equal the longer launch's bit for bit, whichever kernels the two sizes take.
"""
import numpy as np
import pytest

from test_gpu_parity import Case, compare, cu_of
from test_gpu_q4 import check, random_compact, run_q4, run_q4_swiglu

pytestmark = pytest.mark.gpu

ATTN_SEEDS = list(range(10))
GEMM_SEEDS = list(range(8))
MASK_LENS = (0, 1, 7, 64, 176, 200, 431, 432, 1000)


def _attn_case(seed):
    rng = np.random.default_rng(2026 + seed)
    nseq = int(rng.integers(1, 17))
    lengths = []
    for _ in range(nseq):
        L = int(rng.integers(1000, 4001)) if rng.random() < 0.25 else int(rng.integers(1, 701))
        if sum(lengths) + L > 12000:
            break
        lengths.append(L)
    lengths = lengths or [int(rng.integers(1, 701))]
    mask = int(rng.random() < 0.6)
    P = W = 0
    if mask == 1:
        while P == 0 and W == 0:
            P, W = int(rng.choice(MASK_LENS)), int(rng.choice(MASK_LENS))
    return dict(lengths=lengths, mask=mask, P=P, W=W, flags=int(rng.integers(0, 2)),
                v_layout="qkvraw" if rng.random() < 0.5 else "compact", o_last=bool(rng.random() < 0.5),
                rows_seed=int(rng.integers(0, 1 << 30)))


@pytest.mark.timeout(300)
@pytest.mark.parametrize("seed", ATTN_SEEDS)
def test_attention_random_packing(ctx, qattn, oracle, seed):
    c = _attn_case(seed)
    cu = cu_of(c["lengths"])
    T = int(cu[-1])
    print(f"sweep {seed}: {len(c['lengths'])} seqs {c['lengths'][:6]}{'...' if len(c['lengths']) > 6 else ''} "
          f"T={T} mask {c['mask']} P {c['P']} W {c['W']} flags {c['flags']} {c['v_layout']} "
          f"o_last {c['o_last']}", flush=True)
    q, k, v = oracle.gen_qkv(1, seed, cu)
    case = Case(ctx, qattn, q, k, v, cu, c["mask"], c["P"], c["W"], v_layout=c["v_layout"],
                o_last=c["o_last"], flags=c["flags"])
    got = case.run()
    rng = np.random.default_rng(c["rows_seed"])
    ends = [int(cu[i + 1]) - 1 for i in range(len(c["lengths"]))]
    rows = np.unique(np.concatenate([cu[:-1], ends, rng.integers(0, T, size=min(T, 200))]).astype(np.int64))
    exact = oracle.attention_exact(q, k, v, cu, c["mask"], c["P"], c["W"], rows=rows)
    compare(got[rows], exact, f"sweep {seed} ({len(rows)} rows)")
    if c["o_last"]:
        assert np.array_equal(case.last(), got[ends])
    run = ctx.run(case.desc)
    bits = run.mask_bits()
    for s, L in enumerate(c["lengths"]):
        want = oracle.mask_bits(L, c["mask"], c["P"], c["W"])
        got_bits = bits[:, cu[s]:cu[s + 1], :want.shape[1]]
        assert np.array_equal(got_bits, np.broadcast_to(want, got_bits.shape)), (seed, s, L)
    run.destroy()
    case.free()


def _gemm_case(seed):
    rng = np.random.default_rng(4242 + seed)
    m = int(rng.choice([int(rng.integers(1, 65)), int(rng.integers(65, 600)), int(rng.integers(600, 3001))]))
    k = 32 * int(rng.integers(1, 129))
    swiglu = bool(rng.random() < 0.35)
    n = 64 * int(rng.integers(1, 49)) if swiglu else int(rng.integers(1, 4101))
    return rng, m, k, n, swiglu


@pytest.mark.timeout(300)
@pytest.mark.parametrize("seed", GEMM_SEEDS)
def test_q4_random_shape(ctx, oracle, seed):
    rng, m, k, n, swiglu = _gemm_case(seed)
    n_rows = 2 * n if swiglu else n
    print(f"q4 sweep {seed}: M {m} K {k} N {n}{' swiglu' if swiglu else ''}", flush=True)
    packed = random_compact(rng, n_rows, k)
    x = rng.standard_normal((m, k)).astype(np.float16)
    rows = np.unique(np.concatenate([[0, m - 1], rng.integers(0, m, size=min(m, 48))]))
    m2 = int(rng.integers(1, m + 1))
    if swiglu:
        # the fused launch equals the two launches it replaces (projection, then qattn_swiglu) bit
        # for bit; the projection is checked against the oracle on the sampled rows
        y = run_q4_swiglu(ctx, x, packed, k, n)
        gate_up = run_q4(ctx, x, packed, k, 2 * n)
        check(oracle, gate_up[rows], x[rows], packed, k, 2 * n, f"q4 sweep {seed} gate/up")
        dg, do = ctx.upload(np.ascontiguousarray(gate_up).view(np.uint16)), ctx.alloc(m * n * 2)
        ctx.swiglu(dg.ptr, do.ptr, m, width=n)
        ctx.synchronize()
        assert np.array_equal(y.view(np.uint16), do.read(np.uint16, (m, n))), seed
        dg.free()
        do.free()
        y2 = run_q4_swiglu(ctx, x[:m2], packed, k, n)
    else:
        y = run_q4(ctx, x, packed, k, n)
        check(oracle, y[rows], x[rows], packed, k, n, f"q4 sweep {seed}")
        y2 = run_q4(ctx, x[:m2], packed, k, n)
    assert np.array_equal(y2.view(np.uint16), y[:m2].view(np.uint16)), (seed, m2)
