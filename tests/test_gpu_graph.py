"""GPU: a reshard captured in a HIP graph and replayed.

After its first execution a plan's device table is uploaded (and, for a plan
over more than 128 buffers, its pointer table is kept), so an execution with
the same base pointers is one kernel launch with no allocation, no memset and
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
