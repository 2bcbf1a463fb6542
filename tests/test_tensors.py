"""Per-tensor buffers: the arena plan re-based onto one buffer per stored tensor (CPU).

The reference holds one tensor per (rank, parameter, kind) and one bf16
parameter per model shard (resharding_metadata.py:19-40,
training_state.py:176-197).  Executed on separate per-tensor arrays, the
re-based plan must write exactly what the arena plan writes.
"""

import numpy as np
import pytest

from elasticmegatron_amd import _native
from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy as PS
from elasticmegatron_amd.resharding.layout import SEG_DUP
from elasticmegatron_amd.resharding.lowering import lower_redundant_backup, lower_transfer
from elasticmegatron_amd.resharding.tensors import TensorBuffers, rebase_on_tensors
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.transfer import TransferManager
from tests.helpers import SEED, SMALL_CASES, execute_numpy, new_arenas, piece_fill_numpy, small_llama2


def _split(bufs, arenas):
    return [arenas[a][o:o + n].copy() for a, o, n in zip(bufs.arena, bufs.offset, bufs.numel)]


def _join(bufs, tensors, arenas):
    for a, o, n, t in zip(bufs.arena, bufs.offset, bufs.numel, tensors):
        arenas[a][o:o + n] = t


def _cases():
    for name, factory, seq in SMALL_CASES:
        yield pytest.param(factory, seq[0], seq[1], id=name)


@pytest.mark.parametrize("factory,src,dst", list(_cases()))
@pytest.mark.parametrize("bf16_source", ["cast", "copy"])
def test_tensor_plan_writes_what_the_arena_plan_writes(factory, src, dst, bf16_source):
    space = build_virtual_model(factory())
    ls, ld = space.layout(src), space.layout(dst)
    table = lower_transfer(ls, ld, bf16_source=bf16_source)
    sb, db = TensorBuffers(ls), TensorBuffers(ld)
    # Every stored element belongs to exactly one tensor.
    for bufs, lay in ((sb, ls), (db, ld)):
        held = [vp for vp in space.all_virtual_params if lay.has_param(vp)]
        assert sum(bufs.numel) == 3 * sum(h.hi - h.lo for vp in held for h in lay.fp32_holders(vp)) + \
            sum(h.hi - h.lo for vp in held for h in lay.bf16_holders(vp))
        assert len(set(bufs.keys)) == len(bufs.keys)
    tt = rebase_on_tensors(table, sb, db)
    assert int((tt["len"] * tt["rows"]).sum()) == int((table["len"] * table["rows"]).sum())
    _native.Plan(tt, sb.nbytes(), db.nbytes(), check_disjoint=True)   # bounds and disjointness hold

    a = new_arenas(ls)
    piece_fill_numpy(ls.pieces(), a, SEED)
    want = new_arenas(ld, fill=0)
    execute_numpy(table, a, want)
    got_t = [np.zeros_like(t) for t in _split(db, want)]
    execute_numpy(tt, _split(sb, a), got_t)
    got = new_arenas(ld, fill=0)
    _join(db, got_t, got)
    for x, y in zip(got, want):
        assert np.array_equal(x, y)


def test_group_zero_tensor_plan():
    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(6, 1, 1)), space.layout(PS(12, 1, 1, num_distributed_optimizer_instances=2))
    table = lower_redundant_backup(ls, ld, scale_up=True)
    sb, db = TensorBuffers(ls), TensorBuffers(ld)
    tt = rebase_on_tensors(table, sb, db)
    # Duplicates survive the re-basing: the second instance is another tensor of the same kind.
    dup = tt[(tt["flags"] & SEG_DUP) != 0]
    assert len(dup) and (dup["aux_buf"] != dup["dst_buf"]).all()
    assert all(db.keys[int(a)][0] == db.keys[int(d)][0] for a, d in zip(dup["aux_buf"], dup["dst_buf"]))
    _native.Plan(tt, sb.nbytes(), db.nbytes(), check_disjoint=True)
    a = new_arenas(ls)
    piece_fill_numpy(ls.pieces(), a, SEED)
    want = new_arenas(ld, fill=0)
    execute_numpy(table, a, want)
    got_t = [np.zeros_like(t) for t in _split(db, want)]
    execute_numpy(tt, _split(sb, a), got_t)
    got = new_arenas(ld, fill=0)
    _join(db, got_t, got)
    for x, y in list(zip(got, want))[:3]:
        assert np.array_equal(x, y)


def test_keys_name_the_reference_tensors():
    space = build_virtual_model(small_llama2())
    lay = space.layout(PS(8, 2, 1))
    bufs = TensorBuffers(lay)
    kinds = {k[0] for k in bufs.keys}
    assert kinds == {"main", "exp_avg", "exp_avg_sq", "param"}
    name = "decoder.layers.0.mlp.linear_fc1.weight"
    ranks = sorted(k[1] for k in bufs.keys if k[0] == "main" and k[2] == name)
    assert ranks == list(range(8))           # every rank holds a DP piece of it
    assert sum(1 for k in bufs.keys if k[0] == "param" and k[2] == name) == 2   # one per TP shard
    b, local = bufs.locate(0, bufs.offset[5] + 3)
    assert (b, local) == (5, 3)


def test_pointer_table_path_is_exercised():
    """small_llama2 DP8 -> TP2 world 6 has more than 128 tensors on each side: the GPU tests that use it
    take the device-table path of emrs_plan_execute."""
    space = build_virtual_model(small_llama2())
    tm = TransferManager()
    tp = tm.compile_tensors(space.layout(PS(8, 1, 1)), space.layout(PS(6, 2, 1)))
    assert len(tp.src) > 128 and len(tp.dst) > 128
