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
