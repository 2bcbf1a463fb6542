"""GPU: emrs_plan_prepare, the meta-device pre-build of a plan's device tables.

A prepared plan's first execution needs no upload, so it can be the first
call captured into a HIP graph; the graph replays bit-exact, with eager work
and a check between replays.  Prepare itself uploads, so under capture it is
refused and records nothing.  ElasticMegatronManager.reshard(is_meta_device=True)
prepares the plan on the state's GPU without allocating any state, and the
real switch that follows is bit-exact.
"""

import pytest
import torch

from elasticmegatron_amd import ElasticMegatronManager, _native
from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy as PS
from elasticmegatron_amd.megatron_manager.training_state import TrainingState
from elasticmegatron_amd.resharding.model_spec import tiny_llama2
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.transfer import TransferManager
from tests.helpers import SEED, small_llama2

pytestmark = pytest.mark.gpu


def _scramble(state):
    for t in (state.main, state.exp_avg, state.exp_avg_sq):
        t.view(torch.int32).fill_(-1)
    state.param.view(torch.int16).fill_(-1)


def test_prepared_plan_is_captured_on_its_first_call(gpu_device):
    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(8, 2, 1)), space.layout(PS(8, 1, 1))
    a = TrainingState.allocate(ls, gpu_device)
    b = TrainingState.allocate(ld, gpu_device)
    a.fill_synthetic(SEED)
    tm = TransferManager()
    # The library meets the device outside any capture first (device properties, kernel code).
    other = space.layout(PS(8, 4, 1))
    tm.execute(tm.compile(ls, other), a, TrainingState.allocate(other, gpu_device))
    plan = tm.compile(ls, ld)
    marker = torch.zeros(1, device=gpu_device)
    torch.cuda.synchronize()

    print("case prepare under capture", flush=True)
    graph0 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph0):
        marker.fill_(1.0)
        with pytest.raises(_native.EmrsError) as e:
            tm.prepare(plan, gpu_device)
    assert e.value.code == -9 and "capturing" in str(e.value)

    print("case prepare, then capture the first execution", flush=True)
    tm.prepare(plan, gpu_device)
    tm.prepare(plan, gpu_device)  # a second prepare finds the tables in place
    _scramble(b)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        tm.execute(plan, a, b)
    torch.cuda.synchronize()
    assert b.verify_synthetic(SEED)[0] > 0   # captured, not run
    for r in range(3):
        _scramble(b)
        marker.fill_(float(r))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert b.verify_synthetic(SEED)[0] == 0, r


def test_meta_device_reshard_prepares_the_plan(gpu_device):
    seq = [dict(world_size=8, tensor_model_parallel_size=2, pipeline_model_parallel_size=1),
           dict(world_size=8, tensor_model_parallel_size=4, pipeline_model_parallel_size=1)]
    for low_memory in (False, True):
        print(f"case meta-device reshard, low_memory={low_memory}", flush=True)
        mgr = ElasticMegatronManager(seq, tiny_llama2(), device=gpu_device, low_memory=low_memory)
        mgr.training_state.fill_synthetic(SEED)
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated(gpu_device)
        assert mgr.reshard(seq[1], is_meta_device=True) is None
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated(gpu_device) == before   # no state allocated
        new = mgr.reshard(seq[1], verify=True)
        assert mgr.last_verification.bit_exact
        assert new.verify_synthetic(SEED)[0] == 0


def test_prepared_per_tensor_plan(gpu_device):
    """A per-tensor plan (more than 128 buffers a side) prepared ahead: its tables are in place, and
    the first execution, which still uploads the pointer table of its bases, is bit-exact."""
    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(8, 1, 1)), space.layout(PS(8, 4, 1))
    tm = TransferManager()
    plan = tm.compile_tensors(ls, ld)
    assert len(plan.src) > 128
    print("case prepare a per-tensor plan", flush=True)
    tm.prepare(plan, gpu_device)
    a = TrainingState.allocate(ls, gpu_device)
    b = TrainingState.allocate(ld, gpu_device)
    a.fill_synthetic(SEED)
    _scramble(b)
    tm.execute_tensors(plan, plan.src.views(a), plan.dst.views(b))
    torch.cuda.synchronize()
    assert b.verify_synthetic(SEED)[0] == 0


def _capture_first_execute(tm, plan, a, b, gpu_device):
    """Capture the plan's first execution after a meta pass and replay it bit-exact, with eager work
    on the destination between replays."""
    _scramble(b)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        tm.execute(plan, a, b)
    torch.cuda.synchronize()
    assert b.verify_synthetic(SEED)[0] > 0   # captured, not run
    for r in range(3):
        _scramble(b)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert b.verify_synthetic(SEED)[0] == 0, r


def test_capture_after_the_chunk_table_was_turned_on(gpu_device):
    """Prepared with the chunk table off, then turned on: the captured first execution finds its
    segments by search (the table cannot be built under capture) and replays bit-exact."""
    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(8, 2, 1)), space.layout(PS(8, 1, 1))
    a = TrainingState.allocate(ls, gpu_device)
    b = TrainingState.allocate(ld, gpu_device)
    a.fill_synthetic(SEED)
    tm = TransferManager()
    other = space.layout(PS(8, 4, 1))
    tm.execute(tm.compile(ls, other), a, TrainingState.allocate(other, gpu_device))
    plan = tm.compile(ls, ld)
    print("case prepare without the chunk table, capture with it", flush=True)
    try:
        _native.set_tuning(chunk_index=False)
        tm.prepare(plan, gpu_device)
        _native.set_tuning(chunk_index=True)
        _capture_first_execute(tm, plan, a, b, gpu_device)
        # Outside a capture the next call builds the table, and the result is the same.
        _scramble(b)
        tm.execute(plan, a, b)
        torch.cuda.synchronize()
        assert b.verify_synthetic(SEED)[0] == 0
    finally:
        _native.set_tuning()


@pytest.mark.parametrize("kind", ["transfer", "backup_up"])
def test_manager_meta_passes_prepare(gpu_device, kind):
    """transfer_params / redundant_backup with is_meta_device=True upload the plan's tables, as
    reshard(is_meta_device=True) does: the first real execution can then be captured."""
    spec = small_llama2()
    if kind == "transfer":
        src, dst = PS(8, 2, 1), PS(8, 1, 2)
    else:
        src, dst = PS(4, 1, 1), PS(8, 1, 1, num_distributed_optimizer_instances=2)
    mgr = ElasticMegatronManager([src, dst], spec, device=gpu_device, release_source=False)
    a = mgr.training_state
    a.fill_synthetic(SEED)
    # The library meets the device outside any capture first.
    warm = mgr.space_for(PS(8, 4, 1)).layout(PS(8, 4, 1))
    mgr.transfer_manager.execute(mgr.transfer_manager.compile(a.layout, warm), a,
                                 TrainingState.allocate(warm, gpu_device))
    ld = mgr.space_for(dst).layout(dst)
    b = TrainingState.allocate(ld, gpu_device, param=a.param if kind != "transfer" else None)
    print(f"case meta pass of {kind}, then capture", flush=True)
    if kind == "transfer":
        mgr.transfer_params(a, b, None, True)
        plan = mgr.transfer_manager.compile(a.layout, ld)
    else:
        mgr.redundant_backup(a, b, True, is_meta_device=True)
        plan = mgr.transfer_manager.compile(a.layout, ld, "backup_up")
    if kind == "transfer":
        _capture_first_execute(mgr.transfer_manager, plan, a, b, gpu_device)
        return
    # Group ZeRO writes only the fp32 arenas (the bf16 params are shared): check those.
    for t in (b.main, b.exp_avg, b.exp_avg_sq):
        t.view(torch.int32).fill_(-1)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        mgr.transfer_manager.execute(plan, a, b)
    for r in range(2):
        for t in (b.main, b.exp_avg, b.exp_avg_sq):
            t.view(torch.int32).fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert b.verify_synthetic(SEED, bf16=False)[0] == 0, r
