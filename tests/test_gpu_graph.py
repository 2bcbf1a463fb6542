"""GPU: a reshard captured in a HIP graph and replayed.

After its first execution a plan's device table is uploaded (and, for a plan
over more than 128 buffers, its pointer table is kept), so an execution with
the same base pointers is the table pre-read and the copy launch, with no allocation, no memset and
no host synchronisation: it can be captured.  Each replay, with eager work
on the same memory between replays, must give the same bit-exact result as
an eager execution.
"""

import pytest
import torch

from elasticmegatron_amd import ParallelStrategy as PS
from elasticmegatron_amd.megatron_manager.training_state import TrainingState
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.transfer import TransferManager
from tests.helpers import SEED, small_llama2

pytestmark = pytest.mark.gpu


def _scramble(state):
    for t in (state.main, state.exp_avg, state.exp_avg_sq):
        t.fill_(float("nan"))
    state.param.zero_()


@pytest.mark.parametrize("per_tensor", [False, True], ids=["arenas", "per-tensor"])
def test_captured_reshard_replays_bit_exact(gpu_device, per_tensor):
    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(8, 1, 1)), space.layout(PS(8, 4, 1))
    space.register_reshard(ls.strategy, ld.strategy)
    tm = TransferManager()
    a = TrainingState.allocate(ls, gpu_device)
    b = TrainingState.allocate(ld, gpu_device)
    a.fill_synthetic(SEED)
    if per_tensor:
        plan = tm.compile_tensors(ls, ld)
        assert len(plan.src) > 128   # the pointer-table path
        src_v, dst_v = plan.src.views(a), plan.dst.views(b)

        def run():
            tm.execute_tensors(plan, src_v, dst_v)
    else:
        plan = tm.compile(ls, ld)

        def run():
            tm.execute(plan, a, b)

    run()                      # first execution: uploads the tables
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    torch.cuda.synchronize()
    for k in range(4):
        print(f"case graph replay {k} ({'per-tensor' if per_tensor else 'arenas'})", flush=True)
        _scramble(b)           # eager work on the destination between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        bad, first = b.verify_synthetic(SEED)
        assert bad == 0, (k, first)
    # The source changes between replays too: the captured launch reads the memory, not a copy.
    a.fill_synthetic(SEED + 1)
    graph.replay()
    torch.cuda.synchronize()
    bad, first = b.verify_synthetic(SEED + 1)
    assert bad == 0, first


def test_captured_taken_over_group_zero_switch_replays_bit_exact(gpu_device):
    """A Group-ZeRO scale-up between states in 64 KiB granules (hundreds of buffers a side, the
    pointer-table path) whose new state holds the old one's instance 0: captured once, replayed
    with the new state's own granules scrambled in between, and with the source refilled (which
    also rewrites the taken-over head, the same memory)."""
    from elasticmegatron_amd.transfer.ipc_manager import SharedTrainingState
    from elasticmegatron_amd.transfer.transfer import adoptable_granules

    g = 1 << 16
    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(4, 1, 1)), space.layout(PS(8, 1, 1, num_distributed_optimizer_instances=2))
    n = adoptable_granules(ls, ld, g, "backup_up")
    tm = TransferManager()
    plan = tm.compile_granules(ls, ld, g, g, "backup_up", adopt_granules=n)
    a = SharedTrainingState.allocate(ls, gpu_device, g)
    a.fill_synthetic(SEED)
    b = SharedTrainingState.allocate(ld, gpu_device, g, param_granules=[a.tensors[x] for x in a.buffers.granules_of(3)],
                                     adopted=a.leading_fp32_granules(n))
    own = [b.tensors[x] for k in range(3) for x in b.buffers.granules_of(k)[n:]]
    assert len(plan.dst) > 128

    def run():
        tm.execute_states(plan, a, b)

    run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    torch.cuda.synchronize()
    for k in range(3):
        print(f"case graph replay {k} (Group ZeRO, instance 0 taken over)", flush=True)
        for t in own:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        bad, first = b.verify_synthetic(SEED)
        assert bad == 0, (k, first)
    a.fill_synthetic(SEED + 1)
    graph.replay()
    torch.cuda.synchronize()
    bad, first = b.verify_synthetic(SEED + 1)
    assert bad == 0, first


def test_capture_refuses_calls_that_would_allocate(gpu_device):
    """A first call on the device (table upload) or a call whose base pointers differ from the
    plan's first call (its own pointer table) cannot be replayed from a graph: under capture it
    fails with EMRS_ERR_CAPTURE and records nothing; the same calls run eagerly afterwards."""
    from elasticmegatron_amd import _native

    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(8, 1, 1)), space.layout(PS(8, 4, 1))
    space.register_reshard(ls.strategy, ld.strategy)
    tm = TransferManager()
    a = TrainingState.allocate(ls, gpu_device)
    b = TrainingState.allocate(ld, gpu_device)
    b2 = TrainingState.allocate(ld, gpu_device)
    a.fill_synthetic(SEED)
    tm.execute(tm.compile(ls, ld), a, b2)   # the library has met the device outside any capture
    plan = tm.compile_tensors(ls, ld)
    assert len(plan.src) > 128   # the pointer-table path
    src_v, dst_v, dst2_v = plan.src.views(a), plan.dst.views(b), plan.dst.views(b2)
    for st in (b, b2):
        _scramble(st)
    marker = torch.zeros(1, device=gpu_device)  # each graph records one fill, so it is not empty
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    print("case capture of a first call", flush=True)
    with torch.cuda.graph(graph):
        marker.fill_(1.0)
        with pytest.raises(_native.EmrsError) as e:
            tm.execute_tensors(plan, src_v, dst_v)
    assert e.value.code == -9 and "capturing" in str(e.value)
    graph.replay()
    torch.cuda.synchronize()
    assert b.verify_synthetic(SEED)[0] > 0   # nothing was recorded

    tm.execute_tensors(plan, src_v, dst_v)   # eager first call: tables for these bases
    torch.cuda.synchronize()
    assert b.verify_synthetic(SEED)[0] == 0

    graph2 = torch.cuda.CUDAGraph()
    print("case capture with other base pointers", flush=True)
    with torch.cuda.graph(graph2):
        marker.fill_(2.0)
        with pytest.raises(_native.EmrsError) as e:
            tm.execute_tensors(plan, src_v, dst2_v)
    assert e.value.code == -9
    graph2.replay()
    torch.cuda.synchronize()
    assert b2.verify_synthetic(SEED)[0] > 0
    tm.execute_tensors(plan, src_v, dst2_v)  # eagerly, a stream-ordered table of its own
    torch.cuda.synchronize()
    assert b2.verify_synthetic(SEED)[0] == 0

    # The compare entry point allocates: refused under capture as well.
    graph3 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph3):
        marker.fill_(3.0)
        with pytest.raises(_native.EmrsError) as e:
            tm.verify(a, b)
    assert e.value.code == -9
    graph3.replay()
    torch.cuda.synchronize()
    assert float(marker) == 3.0
    assert tm.verify(a, b).bit_exact
