"""bench.py on the CPU: the parts of its contract that need no GPU."""

import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy  # noqa: E402
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model  # noqa: E402
from elasticmegatron_amd.transfer.transfer import TransferManager, adoptable_granules  # noqa: E402


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=300)


def test_more_than_one_gpu_is_refused_with_a_reason():
    r = _run("--gpus", "2")
    assert r.returncode == 2 and "one GPU" in r.stderr and r.stdout == ""


def test_shape_sweep_settings_are_checked_before_any_device_work():
    assert bench.parse_shapes("default;units=4,chunk_index=0; lanes=256") == [{}, {"units": 4, "chunk_index": 0},
                                                                              {"lanes": 256}]
    for bad in ("lanes=96", "units=3", "lanes=128,units=4", "foo=1", "units", "units=x"):
        r = _run("--shape-sweep", bad)
        assert r.returncode == 2 and "--shape-sweep" in r.stderr and r.stdout == "", bad


def test_launch_shape_flags_are_checked_before_any_device_work():
    r = _run("--lanes", "96")
    assert r.returncode == 2 and "invalid choice" in r.stderr and r.stdout == ""
    r = _run("--units", "3")
    assert r.returncode == 2 and "invalid choice" in r.stderr and r.stdout == ""
    r = _run("--help")
    assert r.returncode == 0 and all(f in r.stdout for f in ("--lanes", "--units", "--persistent", "--megatron-buffers",
                                                              "--low-memory", "--tensors", "--rank-shares",
                                                              "--warm-tables"))
    r = _run("--warm-tables", "2")
    assert r.returncode == 2 and "invalid choice" in r.stderr and r.stdout == ""
    assert bench.parse_shapes("warm_tables=0") == [{"warm_tables": 0}]


@pytest.mark.skipif(__import__("torch").cuda.is_available(), reason="checks the behaviour without a GPU")
def test_without_a_gpu_it_says_so():
    r = _run("--steps", "1", "--warmup", "0")
    assert r.returncode == 1 and "needs a GPU" in r.stderr and r.stdout == ""


@pytest.mark.parametrize("name", sorted(bench.workloads()))
def test_every_workload_lays_out(name):
    desc, spec_fn, src, dst, *opt = bench.workloads()[name]
    spec = spec_fn()
    if opt and opt[0]:   # re-padded: one model space per padded vocabulary
        spec_src = spec.with_padded_vocab(spec.padded_vocab_for_tp(src.tensor_model_parallel_size))
        spec_dst = spec.with_padded_vocab(spec.padded_vocab_for_tp(dst.tensor_model_parallel_size))
        ls, ld = build_virtual_model(spec_src).layout(src), build_virtual_model(spec_dst).layout(dst)
    else:
        space = build_virtual_model(spec)
        ls, ld = space.layout(src), space.layout(dst)
    assert ls.fp32_numel > 0 and ld.fp32_numel > 0 and desc


@pytest.mark.parametrize("traffic_file", sorted(f for f in os.listdir(os.path.join(ROOT, "profiles"))
                                                if f.endswith(".traffic.json")))
def test_committed_traffic_describes_the_current_plan(traffic_file):
    """Each committed PMC summary was measured on the plan its workload lowers to today (same
    algorithmic bytes), so bench.py quotes it; a stale one would be ignored, and this fails first."""
    name = traffic_file[:-len(".traffic.json")]
    workload, _, variant = name.partition(".")
    desc, spec_fn, src, dst, *opt = bench.workloads()[workload]
    spec = spec_fn()
    backup = ParallelStrategy.is_redundant_backup(src, dst)
    if opt and opt[0]:
        ls = build_virtual_model(spec.with_padded_vocab(spec.padded_vocab_for_tp(src.tensor_model_parallel_size))).layout(src)
        ld = build_virtual_model(spec.with_padded_vocab(spec.padded_vocab_for_tp(dst.tensor_model_parallel_size))).layout(dst)
    else:
        space = build_virtual_model(spec)
        ls, ld = space.layout(src), space.layout(dst)
    kind = "transfer" if backup is None else ("backup_up" if backup else "backup_down")
    if variant == "taken_over":   # bench.py --adopt: 1 GiB granules, instance 0 taken over
        g = 1 << 30
        n = adoptable_granules(ls, ld, g, kind)
        plan = TransferManager().compile_granules(ls, ld, g, g, kind, adopt_granules=n)
    else:
        assert variant == ""
        plan = TransferManager().compile(ls, ld, kind)
    with open(os.path.join(ROOT, "profiles", traffic_file)) as f:
        rec = json.load(f)
    assert bench.committed_traffic(name, "cast" if backup is None else None, plan.traffic_bytes) == \
        rec["hbm_bytes_per_launch"]
    # Within 0.2% of the algorithmic bytes: the measured traffic also holds the plan's chunk table
    # (4 bytes per 4 KB chunk, about 0.05%) and the segment descriptors.
    assert abs(rec["hbm_bytes_per_launch"] / plan.traffic_bytes - 1) < 2e-3
    assert bench.committed_traffic(name, "cast" if backup is None else None, plan.traffic_bytes + 1) is None


@pytest.mark.parametrize("src,dst", [(ParallelStrategy(8, 2, 1), ParallelStrategy(8, 1, 1)),
                                     (ParallelStrategy(4, 1, 1),
                                      ParallelStrategy(8, 1, 1, num_distributed_optimizer_instances=2))])
def test_cpu_baseline_covers_every_parameter(src, dst):
    """The CPU leg runs Oracle-1 over every parameter of the switch and sums their times."""
    import numpy as np
    import torch

    from elasticmegatron_amd.megatron_manager.training_state import TrainingState
    from elasticmegatron_amd.resharding.model_spec import tiny_llama2
    from tests.helpers import SEED, new_arenas, piece_fill_numpy

    spec = tiny_llama2()
    ls = build_virtual_model(spec).layout(src)
    host = new_arenas(ls, fill=0)
    piece_fill_numpy(ls.pieces(), host, SEED)
    a = TrainingState(ls, *[torch.from_numpy(x.view(np.float32)) for x in host[:3]],
                      torch.from_numpy(host[3].view(np.int16)).view(torch.bfloat16))
    out = bench.cpu_baseline(spec, ls, src, dst, ParallelStrategy.is_redundant_backup(src, dst), a)
    assert out["kind"] == "port" and out["cores"] == os.cpu_count()
    assert f"all {len(ls.place)} parameters ({spec.num_params()} elements)" in out["sample"]
    assert out["value"] > 0 and out["full_switch_ms"] > 0
    payload = TransferManager().compile(ls, ls.space.layout(dst),
                                        "transfer" if dst.num_distributed_optimizer_instances == 1
                                        else "backup_up").payload_bytes
    assert f"{payload / 1e9:.1f} GB payload" in out["sample"]


def test_each_line_names_its_own_workload():
    """The headline metric belongs to the headline switch only; every other workload's line names its
    own switch, so that a line quoted on its own says what it measured."""
    assert bench.metric_for(bench.HEADLINE, bench.workloads()[bench.HEADLINE][0]) == bench.METRIC
    seen = set()
    for name, (desc, *_) in bench.workloads().items():
        m = bench.metric_for(name, desc)
        if name != bench.HEADLINE:
            assert m != bench.METRIC and desc in m and m.endswith("1 GPU"), name
        seen.add(m)
    assert len(seen) == len(bench.workloads())
    gz = bench.metric_for("llama2-7b-groupzero-1-2", bench.workloads()["llama2-7b-groupzero-1-2"][0])
    assert "Group ZeRO" in gz and "TP1DP8" not in gz
