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
    """The destination is checked after the timed steps, with a warm-up or without one."""
    d = _bench("--warmup", str(warmup), "--steps", "2", *extra)
    assert d["warmup"] == warmup and d["steps"] == 2 and d["n_gpus"] == 1
    assert d["config"]["verified_bit_exact"] is True
    assert d["ms_per_step"] > 0 and d["value"] > 0


@pytest.mark.gpu
def test_shape_sweep_times_every_shape_on_the_same_allocations(gpu_device):
    d = _bench("--shape-sweep", "default;units=4,chunk_index=0;units=2", "--steps", "2", "--warmup", "1",
               "--rounds", "2")
    assert d["verified_bit_exact"] is True and d["rounds"] == 2
    assert [r["shape"] for r in d["shapes"]] == ["default", {"units": 4, "chunk_index": 0}, {"units": 2}]
    assert [(r["launch"]["units_per_lane"], r["launch"]["chunk_index"]) for r in d["shapes"]] == \
        [(1, 1), (4, 0), (2, 1)]
    assert all(len(r["ms"]) == 2 and r["best_ms"] > 0 for r in d["shapes"])


@pytest.mark.gpu
def test_rank_shares_line(gpu_device):
    """--rank-shares: every destination rank's share is written alone and checked, then timed."""
    d = _bench("--rank-shares", "--steps", "2", "--warmup", "1")
    assert d["verified_bit_exact"] is True and d["bf16_remainder_segments"] == 0
    assert [r["rank"] for r in d["shares"]] == list(range(8))
    assert all(r["segments"] > 0 and r["ms"] > 0 for r in d["shares"])
    assert sum(r["payload_bytes"] for r in d["shares"]) > 0
    assert d["whole_plan_ms"] > 0 and d["sum_of_shares_ms"] >= d["max_share_ms"] > 0


@pytest.mark.gpu
def test_ipc_line(gpu_device):
    """--ipc: the switch from a child process's exported granules, checked after the timed steps."""
    d = _bench("--ipc", "--ipc-granule-bytes", str(3 << 22), "--steps", "2", "--warmup", "1")
    assert d["config"]["verified_bit_exact"] is True and d["config"]["exporter_exit_status"] == 0
    assert d["config"]["granules"] > 4 and d["ms_per_step"] > 0
    assert set(d["config"]["mapped_vs_owned"]) == {"mapped", "owned", "verified_bit_exact"}
    assert d["config"]["mapped_vs_owned"]["verified_bit_exact"] is True


@pytest.mark.gpu
def test_ipc_staged_line(gpu_device):
    """--ipc --low-memory: one staged switch from a child's granules, each source arena freed by the
    child after its launch, the destination checked afterwards."""
    d = _bench("--ipc", "--low-memory", "--ipc-granule-bytes", str(3 << 22))
    c = d["config"]
    assert c["verified_bit_exact"] is True and c["exporter_exit_status"] == 0
    assert [sorted(s) for s in c["stages_ms"]] == [["allocate", "execute", "release"]] * 3
    assert len(c["device_used_before_each_release_bytes"]) == 3 and d["steps"] == 1


@pytest.mark.gpu
def test_share_rank_line(gpu_device):
    """--share-rank: one destination rank's share on the tensors it touches alone, checked."""
    d = _bench("--share-rank", "3", "--steps", "2", "--warmup", "1")
    c = d["config"]
    assert c["verified_bit_exact"] is True and c["rank"] == 3
    assert 0 < c["destination_tensors"] and 0 < c["source_tensors"] and d["ms_per_step"] > 0
    assert c["read_local_bytes"] + c["read_remote_bytes"] == c["read_bytes"]


@pytest.mark.gpu
def test_copy_shapes_line(gpu_device):
    """--copy-calibration-gib with --shape-sweep: a contiguous copy in each launch shape, checked."""
    d = _bench("--copy-calibration-gib", "0.25", "--shape-sweep", "default;units=2;persistent=1", "--rounds", "2",
               "--steps", "1", "--warmup", "1")
    assert [r["shape"] for r in d["shapes"]] == ["default", {"units": 2}, {"persistent": 1}]
    assert all(len(r["ms"]) == 2 and r["best_TBps"] > 0 for r in d["shapes"])


@pytest.mark.gpu
def test_adopt_line(gpu_device):
    """--adopt: a Group-ZeRO switch between shared states with instance 0 copied and taken over, each
    checked, and the taken-over launch moving a third less (instance 0's last partial granule aside)."""
    d = _bench("--workload", "tiny-llama2-groupzero-1-2", "--adopt", "--ipc-granule-bytes", str(1 << 16),
               "--steps", "2", "--warmup", "1")
    c = d["config"]
    assert c["granules_taken_over_per_fp32_arena"] > 0
    for k in ("copied", "taken_over"):
        assert c[k]["verified_bit_exact"] is True and c[k]["reshard_end_to_end"]["verified_bit_exact"] is True
    assert abs(c["taken_over"]["traffic_bytes"] / c["copied"]["traffic_bytes"] - 2 / 3) < 0.01
    assert c["taken_over"]["new_state_allocated_bytes"] < c["copied"]["new_state_allocated_bytes"]
    assert c["taken_over"]["both_states_allocated_bytes"] < c["copied"]["both_states_allocated_bytes"]


@pytest.mark.gpu
def test_lost_ranks_line(gpu_device):
    """--lost-ranks: the Group-ZeRO switch plain and with rank 1's state poisoned and read from the
    other instance, both checked, moving the same bytes."""
    d = _bench("--workload", "tiny-llama2-groupzero-2-1", "--lost-ranks", "1", "--steps", "2", "--warmup", "1")
    c = d["config"]
    assert c["lost_ranks"] == [1]
    assert c["plain"]["verified_bit_exact"] is True and c["lost"]["verified_bit_exact"] is True
    assert c["plain"]["traffic_bytes"] == c["lost"]["traffic_bytes"]


@pytest.mark.gpu
def test_low_memory_shared_states_line(gpu_device):
    """--low-memory --shared-states: staged switches between states held in granules, checked."""
    d = _bench("--low-memory", "--shared-states", "--ipc-granule-bytes", str(1 << 20), "--steps", "2", "--warmup", "1")
    c = d["config"]
    assert c["verified_bit_exact"] is True and "granules" in c["workload"]
    assert [sorted(s) for s in c["last_switch_stages_ms"]] == [["allocate", "execute", "release"]] * 3


@pytest.mark.gpu
def test_lost_ranks_refuses_a_switch_without_a_second_copy(gpu_device):
    """--lost-ranks on a switch that is not Group ZeRO exits 2 with a message: there is no other
    optimizer instance to read a lost rank's state from."""
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--workload", TINY, "--lost-ranks", "1",
                        "--steps", "1", "--warmup", "0"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "Group-ZeRO" in r.stderr and r.stdout.strip() == ""
