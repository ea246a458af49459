"""GPU tests of the Node path (engine -> runtime -> N-API -> libqattn.so) under `node`.

The operator parity case feeds oracle-generated inputs through the N-API addon and checks the
output here against the f64 oracle with the same bar as the C-ABI parity tests.
"""
import os
import shutil
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_node_gpu_path(oracle, tmp_path):
    lengths = [33, 150, 1, 64, 97]
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    q, k, v = oracle.gen_qkv(1, 5, cu)
    for name, arr in (("q", q), ("k", k), ("v", v), ("cu", cu)):
        arr.tofile(str(tmp_path / f"{name}.bin"))
    r = subprocess.run(["node", "--expose-gc", os.path.join(HERE, "js", "gpu.test.js"), str(tmp_path)],
                       capture_output=True, text=True, timeout=180,
                       env=dict(os.environ, QATTN_EXPECT_GPU="1"))
    print(r.stdout, r.stderr[-2000:])
    assert r.returncode == 0, r.stdout + r.stderr
    o = np.fromfile(str(tmp_path / "o.bin"), dtype=np.uint16).view(np.float16).astype(np.float64)
    exact = oracle.attention_exact(q, k, v, cu)
    o = o.reshape(exact.shape)
    err = np.abs(o - exact).max()
    cos = ((o * exact).sum(-1) / (np.linalg.norm(o, axis=-1) * np.linalg.norm(exact, axis=-1))).min()
    print(f"node path: max|err| {err:.3e} min cos {cos:.7f}")
    assert err <= 2e-3 and cos >= 0.9999


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_node_model_path(tmp_path):
    """The whole forward through Node: a synthetic 2-layer .wgpack, the engine's micro-batch of
    ragged requests, embeddings against the forward oracle (same bar as test_gpu_model)."""
    import json

    import model_ref as mr
    import wgpack
    weights = mr.synthetic_weights(31, 2, vocab=300)
    wgpack.write_model(str(tmp_path / "model.wgpack"), weights)
    rng = np.random.default_rng(12)
    eos = 299
    lists = [rng.integers(0, eos, n).tolist() + [eos] for n in (3, 40, 129, 6, 200)]
    (tmp_path / "requests.json").write_text(json.dumps({"eos": eos, "lists": lists}))
    r = subprocess.run(["node", os.path.join(HERE, "js", "model.gpu.js"), str(tmp_path)],
                       capture_output=True, text=True, timeout=180)
    print(r.stdout, r.stderr[-2000:])
    assert r.returncode == 0, r.stdout + r.stderr
    got = np.fromfile(str(tmp_path / "emb.bin"), dtype=np.float32).reshape(len(lists), 1024)
    cu = np.concatenate([[0], np.cumsum([len(t) for t in lists])]).astype(np.int32)
    want = mr.forward(weights, np.concatenate(lists).astype(np.int32), cu)
    err = np.abs(got - want).max()
    cos = (np.sum(got * want, axis=1) / (np.linalg.norm(got, axis=1) * np.linalg.norm(want, axis=1))).min()
    print(f"node model path: max|err| {err:.3e} min cos {cos:.7f}")
    assert err <= 2e-3 and cos >= 0.9999


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_engine_benchmark_script_runs():
    """js/bench-engine.js (the engine's end-to-end timing on a synthetic model of the real
    shapes) at 2 layers and one timed round: every workload reports, with unit-norm embeddings."""
    import json
    script = os.path.join(HERE, "..", "qwen3-embedding-webgpu-prepacked_amd", "js", "bench-engine.js")
    r = subprocess.run(["node", script, "2", "1"],
                       capture_output=True, text=True, timeout=240)
    print(r.stdout, r.stderr[-2000:])
    assert r.returncode == 0, r.stdout + r.stderr
    lines = [json.loads(l) for l in r.stdout.splitlines() if l.startswith("{")]
    assert [l["workload"] for l in lines] == ["16x500", "64x500", "1x5000"]
    assert all(l["embeddings_unit_norm"] and l["requests_per_s"] > 0 for l in lines)
    # 64 requests: four micro-batches, each after the first enqueued while the one before it ran
    assert lines[1]["micro_batches"] == 4 and lines[1]["enqueued_while_previous_running"] == 3
