"""The model forward on the GPU (qattn_embed_q6k, qattn_rmsnorm, qattn_swiglu, qattn_model_plan_*)
against the CPU restatement (oracle/model_ref.py) on identical synthetic weights and token ids.

Bars: the embedding rows bit-exact (the shader's f32 product is exact before one f16 rounding);
residual add, RMSNorm and SwiGLU within one fp16 step of the f64 restatement (fp32 arithmetic and
summation order inside the row); the whole forward -- fp16 activations between 9 stages per layer
-- per-row cosine >= 0.9999 and max |error| <= 2e-3 on the L2-normalised f32 embeddings."""
import numpy as np
import pytest

import model_ref as mr

pytestmark = pytest.mark.gpu


def ulps(a, b):
    """Distance in fp16 steps of the larger magnitude (at least the subnormal step)."""
    a = np.asarray(a, np.float16).astype(np.float64)
    b = np.asarray(b, np.float16).astype(np.float64)
    step = np.maximum(np.spacing(np.maximum(np.abs(a), np.abs(b)).astype(np.float16)).astype(np.float64), 2.0 ** -24)
    return np.abs(a - b) / step


class DeviceModel:
    """Synthetic weights uploaded once; the qattn_model over them."""

    def __init__(self, ctx, weights, flags=0):
        self.ctx = ctx
        self.bufs = []
        up = lambda a: self._keep(ctx.upload(np.ascontiguousarray(a)))
        self.embd = up(weights["token_embd"])
        self.out_norm = up(weights["output_norm"])
        self.layers = []
        for lw in weights["layers"]:
            d = {}
            for name in ("attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm"):
                d[name] = up(lw[name]).ptr
            for name in ("attn_qkv", "attn_output", "ffn_gate_up", "ffn_down"):
                packed = lw[name][0]
                d[name] = (up(packed).ptr, packed.nbytes)
            self.layers.append(d)
        self.model = ctx.model((self.embd.ptr, weights["token_embd"].nbytes), self.out_norm.ptr, self.layers,
                               flags=flags)

    def _keep(self, b):
        self.bufs.append(b)
        return b

    def free(self):
        self.model.destroy()
        for b in self.bufs:
            b.free()


@pytest.fixture(scope="module")
def weights():
    return mr.synthetic_weights(21, 2, vocab=300)


@pytest.fixture(scope="module")
def dmodel(ctx, weights):
    m = DeviceModel(ctx, weights)
    yield m
    m.free()


def test_embed_q6k_bit_exact(ctx, weights):
    table = weights["token_embd"]
    ids = np.array([0, 299, 17, 17, 150, 3], np.int32)
    dids, dtab, dout = ctx.upload(ids), ctx.upload(table), ctx.alloc(len(ids) * 1024 * 2)
    try:
        ctx.embed_q6k(dids.ptr, len(ids), dtab.ptr, table.nbytes, dout.ptr)
        got = dout.read(np.float16, (len(ids), 1024))
        want = mr.embed(table, ids)
        assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
        # an id outside the table gives a zero row, never a read past it
        bad = ctx.upload(np.array([300, -1, 5], np.int32))
        ctx.embed_q6k(bad.ptr, 3, dtab.ptr, table.nbytes, dout.ptr)
        got = dout.read(np.float16, (3, 1024))
        assert np.all(got[:2] == 0) and np.array_equal(got[2], mr.embed(table, [5])[0])
        bad.free()
    finally:
        for b in (dids, dtab, dout):
            b.free()


@pytest.mark.parametrize("with_residual", [False, True])
def test_rmsnorm_matches_oracle(ctx, with_residual):
    rng = np.random.default_rng(7)
    rows = 37
    x = (3 * rng.standard_normal((rows, 1024))).astype(np.float16)
    r = rng.standard_normal((rows, 1024)).astype(np.float16)
    w = (1 + 0.1 * rng.standard_normal(1024)).astype(np.float32)
    dx, dr, dw, do = ctx.upload(x), ctx.upload(r), ctx.upload(w), ctx.alloc(rows * 1024 * 2)
    try:
        ctx.rmsnorm(dx.ptr, dw.ptr, do.ptr, rows, residual_ptr=dr.ptr if with_residual else None)
        gx, go = dx.read(np.float16, (rows, 1024)), do.read(np.float16, (rows, 1024))
        wx, wo = mr.rmsnorm(x, r if with_residual else None, w)
        assert ulps(gx, wx).max() <= 1
        assert ulps(go, wo).max() <= 1
    finally:
        for b in (dx, dr, dw, do):
            b.free()


def test_swiglu_matches_oracle(ctx):
    rng = np.random.default_rng(8)
    rows = 19
    gu = (2 * rng.standard_normal((rows, 6144))).astype(np.float16)
    dg, do = ctx.upload(gu), ctx.alloc(rows * 3072 * 2)
    try:
        ctx.swiglu(dg.ptr, do.ptr, rows)
        got = do.read(np.float16, (rows, 3072))
        assert ulps(got, mr.swiglu(gu)).max() <= 1
    finally:
        dg.free()
        do.free()


def _run(ctx, dmodel, ids, cu, max_tokens=1024, max_seqs=16):
    plan = dmodel.model.plan(max_tokens, max_seqs)
    out = ctx.alloc(max(1, len(cu) - 1) * 1024 * 4)
    try:
        plan.run(ids, cu, out.ptr)
        ctx.synchronize()
        return out.read(np.float32, (len(cu) - 1, 1024))
    finally:
        out.free()
        plan.destroy()


def _check_embeddings(got, want):
    want = np.asarray(want, np.float64)
    err = np.abs(got.astype(np.float64) - want)
    cos = np.sum(got * want, axis=1) / (np.linalg.norm(got, axis=1) * np.linalg.norm(want, axis=1))
    assert err.max() <= 2e-3, f"max |err| {err.max():.3e}"
    assert cos.min() >= 0.9999, f"min cosine {cos.min():.6f}"
    return err.max(), cos.min()


@pytest.mark.parametrize("lengths", [[5, 32, 43, 1], [700], [9, 640, 60]], ids=["ragged", "sparse700", "mixed"])
def test_model_forward_matches_oracle(ctx, weights, dmodel, lengths):
    rng = np.random.default_rng(sum(lengths))
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    ids = rng.integers(0, weights["vocab"], int(cu[-1])).astype(np.int32)
    got = _run(ctx, dmodel, ids, cu)
    want = mr.forward(weights, ids, cu)
    e, c = _check_embeddings(got, want)
    print(f"lengths {lengths}: max|err| {e:.3e}, min cos {c:.7f}")


@pytest.mark.timeout(400)
def test_model_forward_28_layers_matches_oracle(ctx):
    """The model's real depth (LAYERS = 28, model.ts:21, 91-104): fp16 activations between the
    nine stages of every layer must not drift past the bar over 28 layers.  A mixed packing with
    a sequence longer than prefix + window (the sparse mask's long-range rows) and a short one."""
    weights = mr.synthetic_weights(28, 28, vocab=300)
    m = DeviceModel(ctx, weights)
    try:
        lengths = [5, 64, 200, 700]
        rng = np.random.default_rng(28)
        cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
        ids = rng.integers(0, weights["vocab"], int(cu[-1])).astype(np.int32)
        print(f"28-layer forward {lengths}", flush=True)
        got = _run(ctx, m, ids, cu)
        want = mr.forward(weights, ids, cu)
        e, c = _check_embeddings(got, want)
        print(f"28 layers, lengths {lengths}: max|err| {e:.3e}, min cos {c:.7f}", flush=True)
    finally:
        m.free()


def test_model_rows_do_not_depend_on_the_batch(ctx, weights):
    """With the batch-invariant attention plan, a request's embedding is the same bits alone and
    in batches whose projections take other kernels: alone (120 tokens) the output and down
    projections run the one-wavefront-per-block kernel; in 700- and 2,600-token batches they
    split their K chunks over workgroups (fp32 partials in the plan's workspace, summed in chunk
    order); in a 4,200-token batch (beyond the split range) they sum the chunks in registers."""
    m = DeviceModel(ctx, weights, flags=1)
    rng = np.random.default_rng(12)
    probe = rng.integers(0, weights["vocab"], 120).astype(np.int32)
    try:
        ref = None
        for total in (120, 700, 2600, 4200):
            rest = total - 120
            lengths = [120] + ([rest // 2, rest - rest // 2] if rest else [])
            cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
            ids = np.concatenate([probe, rng.integers(0, weights["vocab"], rest).astype(np.int32)])
            print(f"batch of {total} tokens: {lengths}", flush=True)
            got = _run(ctx, m, ids, cu, max_tokens=4200, max_seqs=4)[0]
            if ref is None:
                ref = got.copy()
                _check_embeddings(got[None], mr.forward(weights, probe, np.array([0, 120], np.int32)))
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), total
    finally:
        m.free()


def test_model_plan_reuse_and_rejects(ctx, qattn, weights, dmodel):
    rng = np.random.default_rng(9)
    plan = dmodel.model.plan(400, 4)
    out = ctx.alloc(4 * 1024 * 4)
    try:
        batches = [np.array([0, 100, 130], np.int32), np.array([0, 7, 8, 300, 400], np.int32)]
        ids = [rng.integers(0, 300, int(cu[-1])).astype(np.int32) for cu in batches]
        results = []
        for i in (0, 1, 0):
            plan.run(ids[i], batches[i], out.ptr)
            ctx.synchronize()
            results.append(out.read(np.float32, (len(batches[i]) - 1, 1024)).copy())
        assert np.array_equal(results[0], results[2])       # re-planned back: the same bits
        _check_embeddings(results[1], mr.forward(weights, ids[1], batches[1]))
        with pytest.raises(qattn.QattnError):                # token id past the vocabulary
            plan.run(np.full(130, 300, np.int32), batches[0], out.ptr)
        with pytest.raises(qattn.QattnError):                # more tokens than the plan holds
            plan.run(np.zeros(401, np.int32), np.array([0, 401], np.int32), out.ptr)
        with pytest.raises(qattn.QattnError):                # more sequences than the plan holds
            plan.run(np.zeros(5, np.int32), np.arange(6, dtype=np.int32), out.ptr)
        plan.run(ids[0], batches[0], out.ptr)                # still usable
        ctx.synchronize()
        assert np.array_equal(out.read(np.float32, (2, 1024)), results[0])
    finally:
        out.free()
        plan.destroy()


def test_model_profile_stages(ctx, qattn, weights, dmodel):
    rng = np.random.default_rng(10)
    cu = np.array([0, 200, 260], np.int32)
    ids = rng.integers(0, 300, 260).astype(np.int32)
    plan = dmodel.model.plan(260, 2)
    out = ctx.alloc(2 * 1024 * 4)
    try:
        plan.run(ids, cu, out.ptr)
        ctx.synchronize()
        ref = out.read(np.float32, (2, 1024)).copy()
        ms = plan.profile(ids, cu, out.ptr)
        assert list(ms) == list(qattn.STAGES)
        # the gate/up projection and SwiGLU are one launch, timed as ffn_up_gate; swiglu is empty
        assert all(v > 0 for k, v in ms.items() if k != "swiglu") and ms["swiglu"] >= 0
        assert np.array_equal(out.read(np.float32, (2, 1024)), ref)
    finally:
        out.free()
        plan.destroy()
