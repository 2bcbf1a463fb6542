"""bench.py on the device, on the tiny model: the JSON line, and the destination check in every order
of warm-up and timed steps."""

import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TINY = "tiny-llama2-tp1dp8-tp4dp2"


def _bench(*args):
    print(f"case bench.py {' '.join(args)}", flush=True)
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--workload", TINY, "--no-cpu-baseline",
                        "--no-e2e", "--no-copy-ceiling", *args], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


@pytest.mark.gpu
@pytest.mark.parametrize("extra", [(), ("--megatron-buffers",), ("--tensors",)])
@pytest.mark.parametrize("warmup", [0, 1])
def test_bench_line_checks_the_destination(gpu_device, warmup, extra):
    """Without a warm-up the destination is checked after the timed steps, not before any launch."""
    d = _bench("--warmup", str(warmup), "--steps", "2", *extra)
    assert d["warmup"] == warmup and d["steps"] == 2 and d["n_gpus"] == 1
    assert d["config"]["verified_bit_exact"] is True
    assert d["ms_per_step"] > 0 and d["value"] > 0
