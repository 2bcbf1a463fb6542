"""Granule buffers: the arena plan re-based onto arenas cut into separate allocations (CPU).

A state handed to another process is held as granules of less than 2 GiB
(device memory is shared one allocation at a time).  Executed on separate
granule arrays, the re-based plan must write exactly what the arena plan
writes.  Small granules (a few KB, some not a power of two) put boundaries
inside one-row and strided segments, bf16 images and duplicates.
"""

import numpy as np
import pytest
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from elasticmegatron_amd import _native
from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy as PS
from elasticmegatron_amd.resharding.granules import GranuleBuffers
from elasticmegatron_amd.resharding.layout import SEG_CAST_BF16, SEG_DUP, SEGMENT_DTYPE
from elasticmegatron_amd.resharding.lowering import lower_redundant_backup, lower_transfer
from elasticmegatron_amd.resharding.tensors import rebase_on_tensors
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from tests.helpers import SEED, SMALL_CASES, execute_numpy, new_arenas, piece_fill_numpy, small_llama2
from tests.test_plan_properties import _lowered, switches

# Granule sizes as (source, destination) numbers of granules per fp32 arena; None: whole arenas.
GRANULES = [(37, 41), (23, None), (None, 29), (3, 64)]


def _granule_bytes(layout, k):
    """Bytes of a granule that cuts the layout's fp32 arenas into about ``k`` pieces."""
    if k is None:
        return None
    return -(-layout.fp32_numel * 4 // k // 256) * 256


def _split(bufs, arenas):
    return [arenas[a][o:o + n].copy() for a, o, n in zip(bufs.arena, bufs.offset, bufs.numel)]


def _join(bufs, parts, arenas):
    for a, o, n, t in zip(bufs.arena, bufs.offset, bufs.numel, parts):
        arenas[a][o:o + n] = t


def _run(ls, ld, table, gs, gd):
    sb, db = GranuleBuffers(ls, gs), GranuleBuffers(ld, gd)
    gt, origin = rebase_on_tensors(table, sb, db, return_origin=True)
    # Bounds (and, for the destinations, disjointness) hold in every granule.
    _native.Plan(gt, sb.nbytes(), db.nbytes(), check_disjoint=True)
    # Nothing is lost or added, and every piece keeps its input row's kind.
    assert int((gt["len"] * gt["rows"]).sum()) == int((table["len"] * table["rows"]).sum())
    assert np.array_equal(gt["flags"], table["flags"][origin])
    assert np.array_equal(gt["elem_bytes"], table["elem_bytes"][origin])
    per_origin = np.bincount(origin, weights=gt["len"] * gt["rows"], minlength=len(table))
    assert np.array_equal(per_origin, (table["len"] * table["rows"]).astype(np.float64))
    a = new_arenas(ls)
    piece_fill_numpy(ls.pieces(), a, SEED)
    want = new_arenas(ld, fill=0)
    execute_numpy(table, a, want)
    got_g = [np.zeros_like(t) for t in _split(db, want)]
    execute_numpy(gt, _split(sb, a), got_g)
    got = new_arenas(ld, fill=0)
    _join(db, got_g, got)
    for x, y in zip(got, want):
        assert np.array_equal(x, y)
    return gt, sb, db


def _cases():
    """Every small switch under every granule setting; the tiny model (39M parameters, the slowest
    under the numpy executor) under the first only."""
    for name, factory, seq in SMALL_CASES:
        for i, (ks, kd) in enumerate(GRANULES):
            if i and name.startswith("tiny"):
                continue
            yield pytest.param(factory, seq[0], seq[1], ks, kd, id=f"{name}-{ks}-{kd}")


@pytest.mark.parametrize("factory,src,dst,ks,kd", list(_cases()))
def test_granule_plan_writes_what_the_arena_plan_writes(factory, src, dst, ks, kd):
    space = build_virtual_model(factory())
    ls, ld = space.layout(src), space.layout(dst)
    table = lower_transfer(ls, ld)
    gt, sb, db = _run(ls, ld, table, _granule_bytes(ls, ks), _granule_bytes(ld, kd))
    if ks is not None and ks > 20:
        assert len(gt) > len(table)   # boundaries fell inside segments


def test_strided_segments_are_cut_between_rows():
    """A column split (TP 1 -> 4) moves strided rows; granule boundaries fall inside and between them."""
    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(8, 1, 1)), space.layout(PS(8, 4, 1))
    table = lower_transfer(ls, ld)
    assert (table["rows"] > 1).any()
    gt, _, _ = _run(ls, ld, table, 256 * 37, 256 * 41)
    assert (gt["rows"] > 1).any() and int(gt["rows"].sum()) >= int(table["rows"].sum())


def test_group_zero_duplicates_across_granules():
    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(6, 1, 1)), space.layout(PS(12, 1, 1, num_distributed_optimizer_instances=2))
    table = lower_redundant_backup(ls, ld, scale_up=True)
    gt, _, _ = _run(ls, ld, table, 4096, 8192)
    assert ((gt["flags"] & SEG_DUP) != 0).any()


def test_cast_images_land_in_param_granules():
    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(8, 1, 1)), space.layout(PS(8, 2, 1))
    gt, _, db = _run(ls, ld, lower_transfer(ls, ld), 1 << 16, 1 << 14)
    cast = gt[(gt["flags"] & SEG_CAST_BF16) != 0]
    assert len(cast) and all(db.arena[int(b)] == 3 for b in cast["aux_buf"])


def test_whole_arena_buffers_are_the_arena_plan():
    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(8, 1, 1)), space.layout(PS(8, 4, 1))
    table = lower_transfer(ls, ld)
    gt = rebase_on_tensors(table, GranuleBuffers(ls, None), GranuleBuffers(ld, None))
    assert np.array_equal(gt, table[table["len"] > 0])


def test_granule_geometry():
    space = build_virtual_model(small_llama2())
    lay = space.layout(PS(8, 2, 1))
    gb = GranuleBuffers(lay, 4096)
    assert [len(gb.granules_of(a)) for a in range(4)] == \
        [-(-lay.fp32_numel // 1024)] * 3 + [-(-lay.bf16_numel // 2048)]
    assert max(gb.nbytes()) == 4096 and len(set(gb.keys)) == len(gb)
    assert gb.locate(1, 1025) == (gb.first[1] + 1, 1)
    assert gb.boundaries(0, 0, 3000) == [1024, 2048]
    assert gb.boundaries(3, 2048, 4096) == []
    with pytest.raises(ValueError):
        GranuleBuffers(lay, 2 << 30)
    with pytest.raises(ValueError):
        GranuleBuffers(lay, 1000)


def test_split_pieces_fill_what_the_arena_fill_writes():
    space = build_virtual_model(small_llama2())
    lay = space.layout(PS(8, 2, 2))
    gb = GranuleBuffers(lay, 256 * 29)
    want = new_arenas(lay, fill=0)
    piece_fill_numpy(lay.pieces(), want, SEED)
    parts = [np.zeros_like(t) for t in _split(gb, want)]
    pcs = gb.split_pieces(lay.pieces())
    assert int(pcs["len"].sum()) == int(lay.pieces()["len"].sum())
    piece_fill_numpy(pcs, parts, SEED)
    got = new_arenas(lay, fill=0)
    _join(gb, parts, got)
    for x, y in zip(got, want):
        assert np.array_equal(x, y)


def test_empty_table():
    space = build_virtual_model(small_llama2())
    lay = space.layout(PS(8, 1, 1))
    gt, origin = rebase_on_tensors(np.zeros(0, dtype=SEGMENT_DTYPE), GranuleBuffers(lay, 4096),
                                   GranuleBuffers(lay, 4096), return_origin=True)
    assert len(gt) == 0 and len(origin) == 0


@st.composite
def _granule_switches(draw):
    spec, a, b = draw(switches())
    # Granule sizes in 256-byte steps, from a few KB (boundaries inside most segments) up to a
    # size that holds a whole arena; None keeps whole arenas on that side.
    sizes = st.one_of(st.none(), st.integers(1, 400).map(lambda k: 256 * k), st.integers(1, 64).map(lambda k: 4096 * k))
    return spec, a, b, draw(sizes), draw(sizes)


@settings(max_examples=25, deadline=None, suppress_health_check=[HealthCheck.filter_too_much, HealthCheck.too_slow])
@given(_granule_switches())
def test_random_granules_write_what_the_arena_plan_writes(sw):
    """Random models, switches and granule sizes on either side: the re-based plan, run on
    separate granule arrays, writes exactly what the arena plan writes."""
    spec, a, b, gs, gd = sw
    space = build_virtual_model(spec)
    la, lb, table = _lowered(space, a, b)
    if max(len(GranuleBuffers(la, gs)), len(GranuleBuffers(lb, gd))) > _native.EMRS_MAX_BUFFERS:
        # More granules on a side than a plan can address: refused when the plan is made.
        with pytest.raises(_native.EmrsError) as e:
            _run(la, lb, table, gs, gd)
        assert e.value.code == -7    # EMRS_ERR_TOO_MANY_BUFFERS
        return
    _run(la, lb, table, gs, gd)


@pytest.mark.parametrize("kind,src,dst", [
    ("transfer", PS(8, 2, 1), PS(8, 1, 1)),
    ("backup_up_bf16", PS(4, 1, 1), PS(8, 1, 1, num_distributed_optimizer_instances=2)),
], ids=["transfer", "groupzero-bf16-copy"])
def test_staged_granule_plans_split_the_granule_plan_by_kind(kind, src, dst):
    """A staged switch from a received state: stage k reads only the source granules of fp32 arena k
    (stage 0 also the bf16 params, when they are copied), writes only destination arena k (stage 0
    also the bf16 params), and the three stages in turn write what the whole granule plan writes."""
    from elasticmegatron_amd.transfer.transfer import TransferManager

    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(src), space.layout(dst)
    tm = TransferManager()
    gs = _granule_bytes(ls, 37)
    whole = tm.compile_granules(ls, ld, gs, None, kind)
    stages = tm.staged_for_states(ls, ld, gs, None, kind)
    assert tm.staged_for_states(ls, ld, gs, None, kind) is stages
    sb = whole.src
    for k, p in enumerate(stages):
        allowed = {k, 3} if k == 0 else {k}
        assert {sb.arena[i] for i in p.src_refs} <= allowed
        assert set(p.dst_refs) <= allowed and k in set(p.dst_refs)
    assert sum(p.payload_bytes for p in stages) == whole.payload_bytes
    assert sum(p.read_bytes for p in stages) == whole.read_bytes
    a = new_arenas(ls)
    piece_fill_numpy(ls.pieces(), a, SEED)
    want, got = new_arenas(ld, fill=0), new_arenas(ld, fill=0)
    execute_numpy(whole.segments, _split(sb, a), want)
    for p in stages:
        execute_numpy(p.segments, _split(sb, a), got)
    for x, y in zip(got, want):
        assert np.array_equal(x, y)
