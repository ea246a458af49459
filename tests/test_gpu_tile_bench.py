"""The tile-body microbenchmark (csrc/tile_body_bench.hip) builds, rejects bad arguments without
touching the GPU, and runs each schedule to a finite rate on the device."""
import os
import re
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(REPO, "qwen3-embedding-webgpu-prepacked_amd", "tile_body_bench")

pytestmark = pytest.mark.skipif(not os.path.exists(BIN), reason="tile_body_bench not built (make tile-bench)")


@pytest.mark.parametrize("args", [[], ["3", "8", "1"], ["0", "0", "1"], ["0", "8", "3"], ["1", "8", "4"]])
def test_bad_arguments_exit_before_the_device(args):
    r = subprocess.run([BIN] + args, capture_output=True, text=True, timeout=60)
    assert r.returncode == 2, (args, r.stdout, r.stderr)


@pytest.mark.gpu
@pytest.mark.timeout(120)
@pytest.mark.parametrize("mode,per_cu", [(0, 2), (1, 3), (2, 3)])
def test_schedules_run(mode, per_cu):
    print(f"tile_body_bench {mode} 17 {per_cu}", flush=True)
    r = subprocess.run([BIN, str(mode), "17", str(per_cu)], capture_output=True, text=True, timeout=90)
    assert r.returncode == 0, (r.stdout, r.stderr)
    m = re.search(r"([0-9.]+) TFLOP/s \(([0-9.]+) of 2.5 PF\)", r.stdout)
    assert m, r.stdout
    assert 0.0 < float(m.group(2)) < 1.0, r.stdout
