"""Destination-rank shares of a plan: the sub-plan one GPU would run with one rank per GPU.

Run one after another on the same buffers, the shares must write exactly what
the whole plan writes (numpy model of the kernel), bit for bit, on every small
switch, both bf16 sources, re-padded vocabularies and Group-ZeRO switches.
Each share writes only its own rank's fp32 region; only the bf16 remainder
has a primary destination in the param arena.
"""

from dataclasses import replace

import numpy as np
import pytest

from elasticmegatron_amd import ParallelStrategy as PS
from elasticmegatron_amd.resharding.layout import ARENA_PARAM, SEG_DUP, SEG_ZERO_FILL
from elasticmegatron_amd.resharding.lowering import lower_redundant_backup, lower_transfer, payload_bytes, read_bytes
from elasticmegatron_amd.resharding.shares import destination_rank_shares, fp32_rank_of
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from tests.helpers import (REPAD_CASES, SEED, SMALL_CASES, execute_numpy, new_arenas, piece_fill_numpy, repad_spaces,
                           small_llama2, small_llama3)
from tests.test_group_zero import CASES as GZ_CASES


def _switches():
    for name, factory, seq in SMALL_CASES:
        for a, b in zip(seq, seq[1:]):
            yield pytest.param(factory, a, b, id=f"{name}-{a.tensor_model_parallel_size}x{a.pipeline_model_parallel_size}x"
                               f"{a.world_size}-{b.tensor_model_parallel_size}x{b.pipeline_model_parallel_size}x"
                               f"{b.world_size}")


def _check(ls, ld, table):
    shares, bf16 = destination_rank_shares(table, ld)
    assert len(shares) == ld.strategy.world_size
    for g, t in enumerate(shares):
        assert not np.any(t["flags"] & SEG_DUP & (fp32_rank_of(t["aux_off"], ld) != g))
        assert np.all(t["dst_buf"] != ARENA_PARAM)
        assert np.all(fp32_rank_of(t["dst_off"], ld) == g)
    assert np.all(bf16["dst_buf"] == ARENA_PARAM)
    # Same bytes written; a split duplicate reads its source once per share instead of once.
    parts = list(shares) + [bf16]
    assert sum(payload_bytes(t) for t in parts) == payload_bytes(table)
    assert sum(read_bytes(t) for t in parts) >= read_bytes(table)
    if not np.any(table["flags"] & SEG_DUP):
        assert sum(read_bytes(t) for t in parts) == read_bytes(table)

    a = new_arenas(ls)
    piece_fill_numpy(ls.pieces(), a, SEED)
    whole, pieces = new_arenas(ld), new_arenas(ld)
    execute_numpy(table, a, whole)
    for t in parts:
        execute_numpy(t, a, pieces)
    for w, p in zip(whole, pieces):
        assert np.array_equal(w, p)
    return shares, bf16


@pytest.mark.parametrize("factory,src,dst", list(_switches()))
@pytest.mark.parametrize("bf16_source", ["cast", "copy"])
def test_shares_write_what_the_plan_writes(factory, src, dst, bf16_source):
    space = build_virtual_model(factory())
    ls, ld = space.layout(src), space.layout(dst)
    table = lower_transfer(ls, ld, bf16_source=bf16_source)
    shares, bf16 = _check(ls, ld, table)
    if bf16_source == "cast":
        assert len(bf16) == 0  # every bf16 element rides on a main segment of some rank
    else:
        assert len(bf16) > 0


@pytest.mark.parametrize("factory,vocab,src,dst", REPAD_CASES)
def test_shares_of_a_repadded_switch(factory, vocab, src, dst):
    spec = replace(factory(), vocab_size=vocab)
    sa, sb = repad_spaces(spec, (src.tensor_model_parallel_size, dst.tensor_model_parallel_size))
    ls, ld = sa.layout(src), sb.layout(dst)
    table = lower_transfer(ls, ld)
    shares, bf16 = _check(ls, ld, table)
    zero = table[(table["flags"] & SEG_ZERO_FILL) != 0]
    if len(zero):
        assert sum(int(((t["flags"] & SEG_ZERO_FILL) != 0).sum()) for t in shares) + \
            int(((bf16["flags"] & SEG_ZERO_FILL) != 0).sum()) == len(zero)


@pytest.mark.parametrize("scale_up", [True, False], ids=["scale_up", "scale_down"])
@pytest.mark.parametrize("name,small,big", GZ_CASES, ids=[c[0] for c in GZ_CASES])
def test_shares_of_a_group_zero_switch(name, small, big, scale_up):
    from tests.helpers import small_llama2

    src, dst = (small, big) if scale_up else (big, small)
    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(src), space.layout(dst)
    table = lower_redundant_backup(ls, ld, scale_up=scale_up)
    shares, bf16 = _check(ls, ld, table)
    assert len(bf16) == 0
    if scale_up:
        # Each new instance's ranks pull their own copy: no share keeps a duplicate to another rank.
        assert np.any(table["flags"] & SEG_DUP)
        assert sum(len(t) for t in shares) > len(table)


def test_a_segment_across_ranks_is_cut_or_refused():
    """A one-row segment running on into the next rank's region is cut there, the source and the
    bf16 image shifting with it; a strided one spanning two regions is refused."""
    space = build_virtual_model(SMALL_CASES[0][1]())
    ls, ld = space.layout(PS(8, 2, 1)), space.layout(PS(8, 1, 1))
    row = lower_transfer(ls, ld)[:1].copy()
    row["rows"], row["src_stride"], row["dst_stride"], row["aux_stride"] = 1, 0, 0, 0
    row["dst_off"], row["len"], row["src_off"], row["aux_off"] = ld.rank_base[1] - 3, 5, 100, 200
    row["flags"] = 1  # with its bf16 image
    shares, bf16 = destination_rank_shares(row, ld)
    got = [(g, int(t["src_off"]), int(t["dst_off"]), int(t["len"]), int(t["aux_off"]))
           for g, ts in enumerate(shares) for t in ts]
    assert got == [(0, 100, ld.rank_base[1] - 3, 3, 200), (1, 103, ld.rank_base[1], 2, 203)]
    assert len(bf16) == 0
    strided = row.copy()
    strided["rows"], strided["len"], strided["src_stride"], strided["dst_stride"] = 2, 2, 4, 4
    strided["aux_stride"] = 4
    with pytest.raises(ValueError, match="one rank's fp32 region"):
        destination_rank_shares(strided, ld)


def test_compile_shares_builds_one_native_plan_per_rank():
    """TransferManager.compile_shares: one checked native plan per destination rank plus the bf16
    remainder, cached; the shares' bytes add up to the whole plan's."""
    from elasticmegatron_amd.transfer.transfer import TransferManager

    space = build_virtual_model(SMALL_CASES[0][1]())
    ls, ld = space.layout(PS(8, 2, 1)), space.layout(PS(8, 4, 1))
    tm = TransferManager()
    per_rank, bf16 = tm.compile_shares(ls, ld)
    assert tm.compile_shares(ls, ld)[0] is per_rank
    whole = tm.compile(ls, ld)
    assert len(per_rank) == 8 and len(bf16.segments) == 0
    assert sum(p.payload_bytes for p in per_rank) == whole.payload_bytes
    assert sum(p.read_bytes for p in per_rank) == whole.read_bytes
    for p in per_rank:
        assert p.native.stats().n_segments >= len(p.segments) > 0


def test_pull_bytes_add_up_to_the_reads():
    """Each share's reads split by source rank add up to its read bytes, and a TP4 -> TP4 identity
    switch reads almost all of it from the destination rank's own source shard: only the
    replicated (non-tensor-parallel) parameters come from TP rank 0's replica, as the reference
    sends them (resharding_tp.py:119-139)."""
    from elasticmegatron_amd.resharding.shares import pull_bytes

    space = build_virtual_model(SMALL_CASES[0][1]())
    for a, b in ((PS(8, 2, 1), PS(8, 1, 1)), (PS(8, 4, 1), PS(8, 4, 1))):
        ls, ld = space.layout(a), space.layout(b)
        table = lower_transfer(ls, ld)
        shares, _ = destination_rank_shares(table, ld)
        for g, t in enumerate(shares):
            fp32, param = pull_bytes(t, ls)
            assert int(fp32.sum()) + param == read_bytes(t)
            if a == b:
                assert 0.99 * int(fp32.sum()) < int(fp32[g])
                if g % 4 == 0:  # TP rank 0 holds the replica it reads
                    assert int(fp32.sum()) == int(fp32[g])


def test_pull_bytes_splits_a_read_across_source_ranks():
    """A one-row read that runs from one source rank's region into the next is split between the
    two; a strided read across a boundary is refused; zero fills read nothing."""
    from elasticmegatron_amd.resharding.shares import pull_bytes

    space = build_virtual_model(SMALL_CASES[0][1]())
    ls = space.layout(PS(8, 2, 1))
    row = np.zeros(1, dtype=lower_transfer(ls, space.layout(PS(8, 1, 1))).dtype)
    row["elem_bytes"], row["rows"], row["len"] = 4, 1, 10
    row["src_off"] = ls.rank_base[3] - 4
    fp32, param = pull_bytes(row, ls)
    assert fp32[2] == 16 and fp32[3] == 24 and int(fp32.sum()) == 40 and param == 0
    zero = row.copy()
    zero["flags"] = SEG_ZERO_FILL
    assert int(pull_bytes(zero, ls)[0].sum()) == 0
    strided = row.copy()
    strided["rows"], strided["len"], strided["src_stride"] = 2, 4, 8
    with pytest.raises(ValueError, match="strided"):
        pull_bytes(strided, ls)


@pytest.mark.parametrize("factory,src,dst", [
    pytest.param(small_llama2, PS(8, 2, 1), PS(8, 1, 2), id="llama2-tp2-pp2"),
    pytest.param(small_llama3, PS(8, 4, 1), PS(8, 1, 2), id="llama3-tp4-pp2"),
])
def test_share_over_tensors_touches_only_its_rank(factory, src, dst):
    """Rank g's share over per-tensor buffers (compile_share_tensors) writes only rank g's optimizer
    tensors and bf16 params of its model shard, and reads only source tensors.  Run with None for
    every tensor it does not touch (numpy model, each share on its own copy of the referenced
    source tensors), the shares together write what the whole plan writes."""
    from elasticmegatron_amd.transfer.transfer import TransferManager

    space = build_virtual_model(factory())
    space.register_reshard(src, dst)
    ls, ld = space.layout(src), space.layout(dst)
    tm = TransferManager()
    a = new_arenas(ls)
    piece_fill_numpy(ls.pieces(), a, SEED)
    whole = new_arenas(ld)
    execute_numpy(lower_transfer(ls, ld), a, whole)
    got = new_arenas(ld)
    for g in range(dst.world_size):
        plan = tm.compile_share_tensors(ls, ld, g)
        sb, db = plan.src, plan.dst
        for i in plan.dst_refs:
            key = db.keys[i]
            if db.arena[i] == ARENA_PARAM:
                assert key[0] == "param"
            else:
                assert key[1] == g, key   # (kind, rank, name): only rank g's own optimizer tensors
        src_bufs = [a[sb.arena[i]][sb.offset[i]:sb.offset[i] + sb.numel[i]].copy() if i in plan.src_refs else None
                    for i in range(len(sb))]
        unset = {4: 0xFFFFFFFF, 2: 0xFFFF}   # values the generator never gives
        dst_bufs = [np.full(db.numel[i], unset[whole[db.arena[i]].itemsize], dtype=whole[db.arena[i]].dtype)
                    if i in plan.dst_refs else None for i in range(len(db))]
        execute_numpy(plan.segments, src_bufs, dst_bufs)
        for i in plan.dst_refs:
            view = got[db.arena[i]][db.offset[i]:db.offset[i] + db.numel[i]]
            written = dst_bufs[i] != unset[dst_bufs[i].itemsize]
            assert np.all(view[written] == unset[view.itemsize])    # no element written by two shares
            view[written] = dst_bufs[i][written]
    for k in range(3):   # every stored fp32 element, from exactly the shares
        stored = whole[k] != 0xFFFFFFFF
        assert np.array_equal(got[k][stored], whole[k][stored])
    stored = whole[3] != 0xFFFF
    assert np.array_equal(got[3][stored], whole[3][stored])


def test_share_of_a_rank_outside_the_world_is_refused():
    from elasticmegatron_amd.transfer.transfer import TransferManager

    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(8, 2, 1)), space.layout(PS(8, 1, 2))
    tm = TransferManager()
    for bad in (-1, 8):
        with pytest.raises(ValueError):
            tm.compile_share_tensors(ls, ld, bad)


def test_partial_execution_checks_the_tensors_it_touches():
    """execute_tensors with None for untouched tensors: a touched tensor that is None, of the wrong
    size, or not in GPU memory is refused before anything runs."""
    import torch

    from elasticmegatron_amd.transfer.transfer import TransferManager

    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(8, 2, 1)), space.layout(PS(8, 1, 2))
    tm = TransferManager()
    plan = tm.compile_share_tensors(ls, ld, 5)
    src = [None] * len(plan.src)
    dst = [None] * len(plan.dst)
    with pytest.raises(ValueError, match="which is None"):
        tm.execute_tensors(plan, src, dst)
    for i in plan.src_refs:
        src[i] = torch.empty(plan.src.numel[i], dtype=torch.float32 if plan.src.arena[i] < 3 else torch.bfloat16)
    for i in plan.dst_refs:
        dst[i] = torch.empty(plan.dst.numel[i], dtype=torch.float32 if plan.dst.arena[i] < 3 else torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU memory"):
        tm.execute_tensors(plan, src, dst)
    i = plan.src_refs[0]          # the first tensor checked
    src[i] = torch.empty(plan.src.numel[i] + 1, dtype=src[i].dtype)
    with pytest.raises(ValueError, match="does not match"):
        tm.execute_tensors(plan, src, dst)


def test_shares_with_a_lost_rank_never_touch_its_tensors():
    """With one rank per GPU and a GPU lost, each surviving rank's share of a Group-ZeRO switch pulls
    the lost rank's shards from another instance: no share references a tensor of the lost rank
    (they may all be None), and the shares together write what the plain switch writes."""
    from elasticmegatron_amd.transfer.transfer import TransferManager

    space = build_virtual_model(small_llama2())
    src, dst, lost = PS(8, 1, 1, num_distributed_optimizer_instances=2), PS(4, 1, 1), 1
    ls, ld = space.layout(src), space.layout(dst)
    tm = TransferManager()
    a = new_arenas(ls)
    piece_fill_numpy(ls.pieces(), a, SEED)
    whole = new_arenas(ld)
    execute_numpy(lower_redundant_backup(ls, ld, False), a, whole)
    got = new_arenas(ld)
    for g in range(dst.world_size):
        plan = tm.compile_share_tensors(ls, ld, g, "backup_down", lost_ranks=[lost])
        sb, db = plan.src, plan.dst
        assert all(sb.keys[i][1] != lost for i in plan.src_refs), g
        src_bufs = [a[sb.arena[i]][sb.offset[i]:sb.offset[i] + sb.numel[i]].copy() if i in plan.src_refs else None
                    for i in range(len(sb))]
        dst_bufs = [np.zeros(db.numel[i], dtype=whole[db.arena[i]].dtype) if i in plan.dst_refs else None
                    for i in range(len(db))]
        execute_numpy(plan.segments, src_bufs, dst_bufs)
        for i in plan.dst_refs:
            got[db.arena[i]][db.offset[i]:db.offset[i] + db.numel[i]] = dst_bufs[i]
    for k in range(3):
        stored = whole[k] != 0xFFFFFFFF
        assert np.array_equal(got[k][stored], whole[k][stored])


def test_tensor_plan_with_a_lost_rank_never_references_its_tensors():
    """Over one buffer per stored tensor, a Group-ZeRO switch with a lost rank references none of
    the lost rank's tensors (they may be None) and writes what the plain switch writes."""
    from elasticmegatron_amd.transfer.transfer import TransferManager

    space = build_virtual_model(small_llama2())
    src, dst, lost = PS(8, 1, 1, num_distributed_optimizer_instances=2), PS(4, 1, 1), 2
    ls, ld = space.layout(src), space.layout(dst)
    plan = TransferManager().compile_tensors(ls, ld, "backup_down", lost_ranks=[lost])
    sb, db = plan.src, plan.dst
    assert all(sb.keys[i][1] != lost for i in plan.src_refs)
    assert any(sb.keys[i][1] == lost for i in range(len(sb)) if sb.arena[i] < 3)   # it has tensors to avoid
    a = new_arenas(ls)
    piece_fill_numpy(ls.pieces(), a, SEED)
    whole = new_arenas(ld)
    execute_numpy(lower_redundant_backup(ls, ld, False), a, whole)
    src_bufs = [a[sb.arena[i]][sb.offset[i]:sb.offset[i] + sb.numel[i]].copy() if i in plan.src_refs else None
                for i in range(len(sb))]
    dst_bufs = [np.zeros(db.numel[i], dtype=whole[db.arena[i]].dtype) for i in range(len(db))]
    execute_numpy(plan.segments, src_bufs, dst_bufs)
    for i in plan.dst_refs:
        assert np.array_equal(dst_bufs[i], whole[db.arena[i]][db.offset[i]:db.offset[i] + db.numel[i]]), db.keys[i]
