"""Staged switches (one optimizer kind per launch), on the CPU.

A staged switch lets the caller allocate each destination fp32 arena just
before its stage and release the source arena right after it, as the
reference releases every optimizer tensor once it is sent
(transfer.py:182-228, resharding_metadata.py:58-65).  Its three stage plans
must partition the plan of the whole switch, each may touch only its own
arenas, and run in order they must write exactly what the whole plan writes,
even with the earlier stages' source arenas gone.
"""

import numpy as np
import pytest

from elasticmegatron_amd import ElasticMegatronManager, ParallelStrategy as PS
from elasticmegatron_amd.resharding import model_spec as ms
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.transfer import TransferManager
from tests.helpers import SEED, execute_numpy, new_arenas, piece_fill_numpy, small_llama2, small_llama3, small_mixtral

CASES = [
    (small_llama2, PS(8, 1, 1), PS(8, 4, 1), "transfer", "cast"),
    (small_llama2, PS(8, 1, 1), PS(8, 4, 1), "transfer", "copy"),
    (small_llama3, PS(8, 2, 2), PS(8, 4, 1), "transfer", "cast"),
    (small_mixtral, PS(8, 1, 1, expert_model_parallel_size=4), PS(8, 1, 1, expert_model_parallel_size=8),
     "transfer", "cast"),
    (small_llama2, PS(6, 1, 1), PS(12, 1, 1, num_distributed_optimizer_instances=2), "backup_up", "cast"),
]


def _rows(t):
    return sorted(map(tuple, t.tolist()))


@pytest.mark.parametrize("factory,src,dst,kind,bf16_source", CASES,
                         ids=["llama2-cast", "llama2-copy", "llama3", "mixtral", "groupzero"])
def test_stages_partition_the_switch(factory, src, dst, kind, bf16_source):
    space = build_virtual_model(factory())
    ls, ld = space.layout(src), space.layout(dst)
    if kind == "transfer":
        space.register_reshard(src, dst)
    tm = TransferManager(check_disjoint=True, bf16_source=bf16_source)
    full = tm.compile(ls, ld, kind)
    stages = tm.compile_staged(ls, ld, kind)
    assert _rows(np.concatenate([s.segments for s in stages])) == _rows(full.segments)
    assert sum(s.payload_bytes for s in stages) == full.payload_bytes
    assert sum(s.read_bytes for s in stages) == full.read_bytes
    for k, s in enumerate(stages):
        extra = {3} if k == 0 and kind == "transfer" else set()
        assert set(s.dst_refs) == {k} | extra
        assert set(s.src_refs) <= {k} | ({3} if bf16_source == "copy" and k == 0 else set())
    assert tm.compile_staged(ls, ld, kind) is stages  # cached

    # In order, with each stage's source arena wiped once it has run, the stages write what the
    # whole plan writes.
    a = new_arenas(ls)
    piece_fill_numpy(ls.pieces(), a, SEED)
    want = new_arenas(ld, fill=0)
    execute_numpy(full.segments, a, want)
    got = new_arenas(ld, fill=0)
    for k, s in enumerate(stages):
        execute_numpy(s.segments, a, got)
        a[k][:] = 0xDEADBEEF
    for x, y in zip(got, want):
        assert np.array_equal(x, y)


def test_low_memory_meta_reshard_prebuilds_the_stages():
    seq = [dict(world_size=8, tensor_model_parallel_size=1, pipeline_model_parallel_size=1),
           dict(world_size=8, tensor_model_parallel_size=4, pipeline_model_parallel_size=1)]
    mgr = ElasticMegatronManager(seq, ms.tiny_llama2(), device="cpu", low_memory=True)
    assert mgr.reshard(seq[1], is_meta_device=True) is None
    staged = [v for k, v in mgr.transfer_manager._plans.items() if k[0] == "staged"]
    assert len(staged) == 1 and len(staged[0]) == 3
