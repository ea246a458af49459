"""Runs the Node engine / N-API boundary tests (CPU) under `node`."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_node_engine_and_boundary():
    env = dict(os.environ, QATTN_EXPECT_GPU="0")
    try:
        import torch
        if torch.cuda.is_available():
            env["QATTN_EXPECT_GPU"] = "1"
    except Exception:
        pass
    r = subprocess.run(["node", os.path.join(HERE, "js", "engine.test.js")], capture_output=True,
                       text=True, timeout=120, env=env)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_node_prepacked_format():
    r = subprocess.run(["node", os.path.join(HERE, "js", "prepacked.test.js")], capture_output=True,
                       text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_node_packer_equals_oracle_packer(oracle, tmp_path):
    # Two parts (70 and 33 rows, K = 96) of seeded GGML Q4_0 bytes, packed by js/prepacked.js and by
    # the oracle's restatement of format.ts:64-96: identical bytes.
    import numpy as np
    rng = np.random.default_rng(17)
    k = 96
    a = rng.integers(0, 256, size=70 * 3 * 18, dtype=np.uint8)
    b = rng.integers(0, 256, size=33 * 3 * 18, dtype=np.uint8)
    (tmp_path / "a.bin").write_bytes(a.tobytes())
    (tmp_path / "b.bin").write_bytes(b.tobytes())
    mod = os.path.join(HERE, "..", "qwen3-embedding-webgpu-prepacked_amd", "js", "prepacked.js")
    script = (
        f"const fmt = require({mod!r}); const fs = require('fs');"
        f"const rd = (f) => new Uint8Array(fs.readFileSync(f));"
        f"const p = fmt.packQ40Tile32('w', [{{name: 'a', k: {k}, n: 70, bytes: rd({str(tmp_path / 'a.bin')!r})}},"
        f"  {{name: 'b', k: {k}, n: 33, bytes: rd({str(tmp_path / 'b.bin')!r})}}]);"
        f"fs.writeFileSync({str(tmp_path / 'out.bin')!r}, Buffer.from(p.bytes));")
    r = subprocess.run(["node", "-e", script], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    got = np.frombuffer((tmp_path / "out.bin").read_bytes(), np.uint8)
    want, _, n = oracle.pack_q40_tile32([(k, 70, a.tobytes()), (k, 33, b.tobytes())])
    assert n == 103 and np.array_equal(got, want)


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
@pytest.mark.parametrize("config,lengths,kind,groups", [
    (0, [50], 1, None), (1, [40, 33, 1], 0, None),
    # the sparse skip: the last query tiles of a 700-token sequence (rows 640..699), two heads
    (3, [700], 1, [[0, t, h] for t in (40, 41, 42, 43) for h in (0, 13)])])
def test_node_cpu_baseline_equals_c_restatement(oracle, tmp_path, config, lengths, kind, groups):
    # oracle/tiled16.js (the Node CPU baseline bench.py times) against orc_attention_tiled16 (the C
    # restatement of the same WGSL): bit for bit on every computed row.
    import json
    import numpy as np
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    q, k, v = oracle.gen_qkv(config, 0, cu)
    for name, a in (("q", q), ("k", k), ("v", v)):
        a.tofile(str(tmp_path / f"{name}.bin"))
    meta = {"cu": cu.tolist(), "kind": kind, "prefix": 176, "window": 432}
    if groups:
        meta["sample"] = groups
    (tmp_path / "meta.json").write_text(json.dumps(meta))
    js = os.path.join(HERE, "..", "oracle", "tiled16.js")
    r = subprocess.run(["node", js, "run", str(tmp_path)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    got = np.fromfile(str(tmp_path / "o.bin"), np.uint16).reshape(-1, 16, 128)
    want = oracle.attention_tiled16(q, k, v, cu, kind=kind).reshape(got.shape)
    if not groups:
        assert np.array_equal(got, want)
        return
    for s, t, h in groups:
        rows = slice(int(cu[s]) + 16 * t, min(int(cu[s]) + 16 * t + 16, int(cu[s + 1])))
        assert np.array_equal(got[rows, h], want[rows, h]), (t, h)


def test_bench_config1_lengths_equal_the_oracle_generator(oracle):
    import importlib.util
    spec = importlib.util.spec_from_file_location("bench", os.path.join(HERE, "..", "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    assert bench.config1_lengths() == oracle.gen_lengths(oracle.seed(1, 0, 3), 16).tolist()


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_node_model_loader():
    r = subprocess.run(["node", os.path.join(HERE, "js", "model.test.js")], capture_output=True,
                       text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_node_half_decode_is_ieee_binary16(tmp_path):
    # runtime.js's binary16 -> f32 table (the decode of every result the Node runtime reads back)
    # against numpy's IEEE conversion, on all 65,536 bit patterns: subnormals, signed zeros,
    # infinities and NaNs included.
    import numpy as np
    mod = os.path.join(HERE, "..", "qwen3-embedding-webgpu-prepacked_amd", "js", "runtime.js")
    out = tmp_path / "dec.bin"
    script = (
        f"const {{ halvesToFloat32 }} = require({mod!r});"
        f"const bits = new Uint16Array(65536); for (let i = 0; i < 65536; i += 1) bits[i] = i;"
        f"const f = halvesToFloat32(bits);"
        f"require('fs').writeFileSync({str(out)!r}, Buffer.from(f.buffer));")
    r = subprocess.run(["node", "-e", script], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    got = np.frombuffer(out.read_bytes(), np.float32)
    want = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))  # -0.0 kept
