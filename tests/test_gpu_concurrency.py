"""GPU: one plan used from two threads at once, each on its own stream.

The library documents that a plan may be executed and compared from several
threads and streams concurrently: its per-device tables are made, and its
launch records kept, under the plan's own lock.  Here both threads start on a
plan that has never run on the device, so both race to make its tables, and
then keep launching.  ctypes releases the interpreter lock around each call,
so the calls really overlap in the library.
"""

import threading

import pytest
import torch

from elasticmegatron_amd import ParallelStrategy as PS
from elasticmegatron_amd.megatron_manager.training_state import TrainingState
from elasticmegatron_amd.resharding.lowering import lower_transfer
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd import _native
from tests.helpers import SEED, small_llama2

pytestmark = pytest.mark.gpu


def _run_in_threads(fns):
    start = threading.Barrier(len(fns))
    errors = []

    def wrap(fn):
        try:
            start.wait()
            fn()
        except Exception as e:   # reported by the test thread
            errors.append(e)

    threads = [threading.Thread(target=wrap, args=(fn,)) for fn in fns]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a thread did not finish"
    assert errors == [], errors


def test_one_plan_executed_and_compared_from_two_threads(gpu_device):
    space = build_virtual_model(small_llama2())
    src, dst = PS(8, 2, 1), PS(8, 1, 2)
    space.register_reshard(src, dst)
    ls, ld = space.layout(src), space.layout(dst)
    table, groups, aux_groups = lower_transfer(ls, ld, with_groups=True)
    sizes = ([ls.fp32_numel * 4] * 3 + [ls.bf16_numel * 2], [ld.fp32_numel * 4] * 3 + [ld.bf16_numel * 2])
    plan = _native.Plan(table, *sizes)       # never run: both threads race to make its device tables
    a = TrainingState.allocate(ls, gpu_device)
    a.fill_synthetic(SEED)
    outs = [TrainingState.allocate(ld, gpu_device) for _ in range(2)]
    streams = [torch.cuda.Stream(device=gpu_device) for _ in range(2)]
    torch.cuda.synchronize()
    print("case one plan, two threads: execute", flush=True)

    def executor(b, st):
        def run():
            with torch.cuda.device(gpu_device):
                for _ in range(6):
                    plan.execute(a.arena_ptrs(), b.arena_ptrs(), st.cuda_stream)
                st.synchronize()
        return run

    _run_in_threads([executor(b, st) for b, st in zip(outs, streams)])
    for b in outs:
        bad, first = b.verify_synthetic(SEED)
        assert bad == 0, first

    print("case one plan, two threads: compare", flush=True)
    n_groups = 4 * len(space.all_virtual_params)
    results = [None, None]

    def comparer(i, b, st):
        def run():
            with torch.cuda.device(gpu_device):
                for _ in range(3):
                    results[i] = plan.compare(a.arena_ptrs(), b.arena_ptrs(), groups, aux_groups, n_groups,
                                              st.cuda_stream)
        return run

    outs[1].exp_avg.view(torch.int32)[1000] ^= 1        # one flipped bit in the second state
    torch.cuda.synchronize()
    _run_in_threads([comparer(i, b, st) for i, (b, st) in enumerate(zip(outs, streams))])
    assert int(results[0]["mismatches"].sum()) == 0
    assert int(results[1]["mismatches"].sum()) == 1
