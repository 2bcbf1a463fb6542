"""Lowering of a strategy switch to a flat table of copy segments.

The reference moves each parameter's optimizer state in three passes of
point-to-point messages: a DP gather onto the aligned source rank plus the
SwiGLU shuffle, the TP/PP/EP exchange, then the SwiGLU unshuffle and a DP
scatter (elastic_megatron/transfer/transfer.py:143-269, :291-341).  Every hop
is a same-dtype copy, so their composition is a fixed gather: each
destination element takes the value of one source element holding the same
(parameter, full-tensor index).  This module computes that gather directly,
in full-tensor coordinates:

* every holder (rank piece or model shard) is cut into at most three
  rectangles per band of its local tensor (partial first row, whole rows,
  partial last row), each a strided region of its arena;
* each destination rectangle is intersected with the source rectangles; an
  intersection is one strided segment, and whole-row intersections that are
  contiguous on both sides become one contiguous segment;
* source replicas are chosen as the reference chooses them: a parameter that
  is not tensor-parallel is sent by source TP rank 0 to every destination TP
  rank (resharding_tp.py:119-139).

The SwiGLU shuffle/unshuffle pair (resharding_metadata.py:98-178) needs no
pass of its own: it only makes the destination's ``[W_t; V_t]`` rows come
from the two matching row bands of the source, which the band geometry
expresses directly.

Group-ZeRO switches (transfer.py:343-388) copy whole optimizer shards: every
destination instance receives the shard of source instance 0 on scale-up
(migrate on the inter-instance master, then broadcast) and of its own
instance on scale-down (``TrainingState.param_migrate``,
training_state.py:40-60).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Iterable, List, Optional, Sequence, Tuple

import numpy as np

from .layout import (ARENA_PARAM, SEG_CAST_BF16, SEG_DUP, SEG_ZERO_FILL, SEGMENT_DTYPE, Geometry, Holder, StrategyLayout,
                     view2d)
from .resharding_tp import is_pow2


@dataclass(frozen=True)
class Rect:
    r0: int
    r1: int
    c0: int
    c1: int
    off: int      # arena element offset of (r0, c0)
    stride: int   # arena elements between rows


def holder_rects(h: Holder, geo: Geometry) -> List[Rect]:
    cl = geo.cols
    out: List[Rect] = []
    for lr0, lr1, fr0 in geo.bands():
        a, b = max(h.lo, lr0 * cl), min(h.hi, lr1 * cl)
        if a >= b:
            continue
        ra, ca = divmod(a, cl)
        rb, cb = divmod(b, cl)

        def emit(r: int, c0: int, c1: int, nrows: int) -> None:
            out.append(Rect(r - lr0 + fr0, r - lr0 + fr0 + nrows, c0 + geo.col_off, c1 + geo.col_off,
                            h.offset + r * cl + c0 - h.lo, cl))

        if ra == rb:
            emit(ra, ca, cb, 1)
            continue
        r = ra
        if ca > 0:
            emit(ra, ca, cl, 1)
            r = ra + 1
        if rb > r:
            emit(r, 0, cl, rb - r)
        if cb > 0:
            emit(rb, 0, cb, 1)
    return out


def _intersections(src: Sequence[Rect], dst: Sequence[Rect]) -> Iterable[Tuple[int, int, int, int, int, int]]:
    """(src_off, dst_off, len, rows, src_stride, dst_stride) for every overlapping pair."""
    src = sorted(src, key=lambda r: r.r0)
    starts = [r.r0 for r in src]
    import bisect

    for d in dst:
        hi = bisect.bisect_left(starts, d.r1)
        for s in src[:hi]:
            r0, r1 = max(s.r0, d.r0), min(s.r1, d.r1)
            if r0 >= r1:
                continue
            c0, c1 = max(s.c0, d.c0), min(s.c1, d.c1)
            if c0 >= c1:
                continue
            so = s.off + (r0 - s.r0) * s.stride + (c0 - s.c0)
            do = d.off + (r0 - d.r0) * d.stride + (c0 - d.c0)
            n, rows = c1 - c0, r1 - r0
            if rows == 1 or (n == s.stride and n == d.stride):
                yield so, do, n * rows, 1, 0, 0
            else:
                yield so, do, n, rows, s.stride, d.stride


class SegmentBuilder:
    """Accumulates segment rows, merging a contiguous continuation into the previous row."""

    def __init__(self):
        self.rows: List[Tuple] = []
        self.groups: List[int] = []  # parameter of each row; rows of different parameters never merge

    def add(self, sbuf: int, dbuf: int, eb: int, so: int, do: int, n: int, rows: int, ss: int, ds: int,
            aux: Optional[Tuple[int, int, int]] = None, zero: bool = False, group: int = 0,
            dup: bool = False) -> None:
        """``aux`` = (buffer, offset, row stride) of a second destination: the bf16
        image of the values, or with ``dup`` an unchanged copy."""
        if n <= 0 or rows <= 0:
            return
        flags, abuf, aoff, astr = ((SEG_DUP if dup else SEG_CAST_BF16), aux[0], aux[1], aux[2]) if aux else (0, 0, 0, 0)
        if zero:
            flags |= SEG_ZERO_FILL
            so, ss = 0, 0
        if self.rows and rows == 1 and self.groups[-1] == group:
            p = self.rows[-1]
            if (p[0] == sbuf and p[1] == dbuf and p[2] == eb and p[3] == flags and p[7] == 1
                    and (zero or p[4] + p[6] == so) and p[5] + p[6] == do
                    and (not aux or (p[10] == abuf and p[12] + p[6] == aoff))):
                self.rows[-1] = p[:6] + (p[6] + n,) + p[7:]
                return
        self.rows.append((sbuf, dbuf, eb, flags, so, do, n, rows, ss, ds, abuf, 0, aoff, astr if rows > 1 else 0))
        self.groups.append(group)

    def table(self) -> np.ndarray:
        arr = np.zeros(len(self.rows), dtype=SEGMENT_DTYPE)
        if self.rows:
            arr[:] = self.rows
        return arr

    def group_array(self) -> np.ndarray:
        return np.asarray(self.groups, dtype=np.int64)


def _src_replica(vp, holders: List[Holder]) -> List[Holder]:
    out = [h for h in holders if h.instance == 0]
    if not vp.tensor_parallel_attr.tensor_model_parallel:
        out = [h for h in out if h.tp_rank == 0]
    return out


def _rows_from(rects: Sequence[Rect], first_row: int) -> Iterable[Tuple[int, int, int, int]]:
    """(dst_off, len, rows, dst_stride) of the parts of ``rects`` at full rows >= first_row."""
    for d in rects:
        if d.r1 <= first_row:
            continue
        r0 = max(d.r0, first_row)
        off = d.off + (r0 - d.r0) * d.stride
        n, rows = d.c1 - d.c0, d.r1 - r0
        if rows == 1 or n == d.stride:
            yield off, n * rows, 1, 0
        else:
            yield off, n, rows, d.stride


def check_compatible(src_space, dst_space) -> None:
    """Two models that differ at most in the padded vocabulary (rows of the embedding and output layer)."""
    if src_space is dst_space:
        return
    a, b = src_space.all_virtual_params, dst_space.all_virtual_params
    if len(a) != len(b) or src_space.tied_embeddings != dst_space.tied_embeddings:
        raise ValueError("the two layouts are of different models")
    for x, y in zip(a, b):
        same_attr = (x.name == y.name and x.tensor_parallel_attr.tensor_model_parallel
                     == y.tensor_parallel_attr.tensor_model_parallel
                     and x.tensor_parallel_attr.partition_dim == y.tensor_parallel_attr.partition_dim)
        vocab = x.param_def.name in ("embedding.word_embeddings.weight", "output_layer.weight")
        same_shape = x.full_shape == y.full_shape or (vocab and x.full_shape[1:] == y.full_shape[1:])
        if not (same_attr and same_shape):
            raise ValueError(f"the two layouts are of different models ({x.name} vs {y.name})")


def lower_transfer(src: StrategyLayout, dst: StrategyLayout, include_fp32: bool = True,
                   include_bf16: bool = True, bf16_source: str = "cast", with_groups: bool = False):
    """Segments of a switch between two layouts of the same model.

    Buffers 0..2 are the fp32 arenas (main, exp_avg, exp_avg_sq) and buffer 3
    the bf16 param arena, on both sides.  ``bf16_source``:

    * ``"cast"`` (default): the destination bf16 params are the bf16 rounding
      of the destination main weights, written by the main segments as they
      copy (the reference's ``_copy_main_params_to_model_params`` + DP
      all-gather, training_state.py:176-197).  26 bytes of HBM traffic per
      parameter.
    * ``"copy"``: the bf16 params are copied from the source bf16 shards.
      28 bytes per parameter; equal bits when main = upcast(param).

    The two layouts may differ in the padded vocabulary (a re-padding switch;
    the reference keeps it fixed, virtual_param.py:480-481).  Rows the source
    has and the destination keeps are copied; new padding rows are written
    as zeros in all four tensors; dropped padding rows are not read.

    ``with_groups=True`` returns ``(table, groups, aux_groups)`` instead: no
    segment spans two parameters, and each segment's elements (and its bf16
    image) carry the group ``4 * parameter index + kind`` (kind 0 bf16 param,
    1 main, 2 exp_avg, 3 exp_avg_sq).  That table is for verification
    (:func:`emrs_plan_compare`); the executed one merges across parameters.
    """
    if bf16_source not in ("cast", "copy"):
        raise ValueError(bf16_source)
    # The reference computes every parameter's TP maps, and those accept powers of two only
    # (resharding_tp.py:98-99), whatever path built the layouts.
    for st in (src.strategy, dst.strategy):
        if not is_pow2(st.tensor_model_parallel_size):
            raise AssertionError("TP sizes must be powers of two")
    cast = include_bf16 and bf16_source == "cast"
    if cast and not include_fp32:
        raise ValueError("the bf16 cast rides on the fp32 main segments")
    check_compatible(src.space, dst.space)
    fp32 = SegmentBuilder()
    bf16 = SegmentBuilder()
    for vp in dst.space.all_virtual_params:
        # A tied output layer is filled from the source word embedding: the
        # reference broadcasts the new embedding state to it (transfer.py:103-141).
        sv = src.space.value_source(src.space.all_virtual_params[vp.global_index])
        if not (src.has_param(sv) and dst.has_param(vp)):
            continue  # tied output layer at destination PP 1 (transfer.py:324-330)
        gid = vp.global_index if with_groups else 0
        src_rows = view2d(sv.full_shape, sv.tensor_parallel_attr.partition_dim)[0]
        dst_rows = view2d(vp.full_shape, vp.tensor_parallel_attr.partition_dim)[0]
        new_rows = src_rows if dst_rows > src_rows else None
        if include_fp32:
            bf16_base = {h.tp_rank: h.offset for h in dst.bf16_holders(vp)} if cast else {}
            s_rects = [r for h in _src_replica(sv, src.fp32_holders(sv))
                       for r in holder_rects(h, src.geometry(sv, h.tp_rank))]
            covered = 0
            want = 0
            for h in dst.fp32_holders(vp):
                want += h.hi - h.lo
                d_rects = holder_rects(h, dst.geometry(vp, h.tp_rank))

                def aux_of(do, ds):
                    if cast and h.instance == 0:
                        return ARENA_PARAM, bf16_base[h.tp_rank] + do - h.offset + h.lo, ds
                    return None

                for so, do, n, rows, ss, ds in _intersections(s_rects, d_rects):
                    fp32.add(0, 0, 4, so, do, n, rows, ss, ds, aux_of(do, ds), group=gid)
                    covered += n * rows
                if new_rows is not None:
                    for do, n, rows, ds in _rows_from(d_rects, new_rows):
                        fp32.add(0, 0, 4, 0, do, n, rows, 0, ds, aux_of(do, ds), zero=True, group=gid)
                        covered += n * rows
            if covered != want:
                raise AssertionError(f"{vp.name}: fp32 plan covers {covered} of {want} elements")
            if cast:
                main_once = sum(h.hi - h.lo for h in dst.fp32_holders(vp) if h.instance == 0)
                if main_once != sum(h.hi - h.lo for h in dst.bf16_holders(vp)):
                    raise AssertionError(f"{vp.name}: bf16 cast would not cover every param element once")
        if include_bf16 and not cast:
            s_rects = [r for h in _src_replica(sv, src.bf16_holders(sv))
                       for r in holder_rects(h, src.geometry(sv, h.tp_rank))]
            covered = 0
            want = 0
            for h in dst.bf16_holders(vp):
                want += h.hi - h.lo
                d_rects = holder_rects(h, dst.geometry(vp, h.tp_rank))
                for so, do, n, rows, ss, ds in _intersections(s_rects, d_rects):
                    bf16.add(ARENA_PARAM, ARENA_PARAM, 2, so, do, n, rows, ss, ds, group=gid)
                    covered += n * rows
                if new_rows is not None:
                    for do, n, rows, ds in _rows_from(d_rects, new_rows):
                        bf16.add(ARENA_PARAM, ARENA_PARAM, 2, 0, do, n, rows, 0, ds, zero=True, group=gid)
                        covered += n * rows
            if covered != want:
                raise AssertionError(f"{vp.name}: bf16 plan covers {covered} of {want} elements")
    return _assemble(fp32.table(), bf16.table(), fp32.group_array(), bf16.group_array(), with_groups)


def _backup_sources(src: StrategyLayout, dst: StrategyLayout, vp, scale_up: bool, lost=frozenset(),
                    source_instance: int = 0):
    """(source holder, destination holder) of every fp32 run of ``vp`` in a Group-ZeRO switch: a
    new instance's shard comes from instance ``source_instance`` (the reference's ``group_src``,
    0 unless given) on a scale-up and from the same instance on a scale-down
    (transfer.py:343-388).  A shard whose rank is in ``lost`` is read from the first
    other optimizer instance that holds it on a rank not lost (every instance holds the whole
    optimizer state, partitioned alike)."""
    src_by, replicas = {}, {}
    for h in src.fp32_holders(vp):
        src_by[(h.instance, h.tp_rank, h.lo)] = h
        replicas.setdefault((h.tp_rank, h.lo, h.hi), []).append(h)
    out = []
    for h in dst.fp32_holders(vp):
        s = src_by.get((source_instance if scale_up else h.instance, h.tp_rank, h.lo))
        if s is None or s.hi != h.hi:
            raise AssertionError(f"{vp.name}: no matching source shard for a Group-ZeRO copy")
        if s.rank in lost:
            s = next((r for r in replicas[(s.tp_rank, s.lo, s.hi)] if r.rank not in lost), None)
            if s is None:
                raise ValueError(f"{vp.name}: every optimizer instance's copy of a shard is on a lost rank")
        out.append((s, h))
    return out


def in_place_prefix(src: StrategyLayout, dst: StrategyLayout, scale_up: bool) -> int:
    """Length of the head of a Group-ZeRO switch's fp32 arenas that the new state could take over
    from the old one unchanged: every destination run that starts below it sits at its source's
    offset, and it does not pass the end of either arena.  With PP = 1 it covers instance 0 (the
    leading ranks of both worlds); with PP > 1, instance 0 of the first stage."""
    if src.strategy.optimizer_data_parallel_size != dst.strategy.optimizer_data_parallel_size:
        raise AssertionError("Group-ZeRO switch must keep the optimizer DP size")
    end = min(src.fp32_numel, dst.fp32_numel)
    for vp in src.space.all_virtual_params:
        if src.has_param(vp) and dst.has_param(vp):
            for s, h in _backup_sources(src, dst, vp, scale_up):
                if s.offset != h.offset:
                    end = min(end, h.offset)
    return end


def lower_redundant_backup(src: StrategyLayout, dst: StrategyLayout, scale_up: bool, with_groups: bool = False,
                           copy_bf16: bool = False, in_place_below: int = 0, lost_ranks: Sequence[int] = (),
                           source_instance: int = 0):
    """fp32 segments of a Group-ZeRO switch (instances change, shards do not).

    On a scale-up every new instance of a shard is filled from instance 0's
    copy, or instance ``source_instance``'s (transfer.py:343-388).  The destinations of one source shard are
    taken in pairs, each pair as one duplicating segment: the shard is read
    once per two copies written.

    The model-parallel shards are the same on both sides, so the bf16 params
    normally carry over in place (the new state shares the old one's param
    arena).  ``copy_bf16`` is for a destination that cannot share it, such
    as one built from another process's state, which that process frees: the
    bf16 params are then copied shard by shard, the same bits the shared
    arena would hold (4 bytes of traffic per parameter).

    ``in_place_below``: fp32 elements of the new arenas below this offset are
    not written, because the new state holds the old one's memory there (it
    took over the old state's leading granules; at most
    :func:`in_place_prefix`, checked run by run).  A run that crosses the
    offset is copied from it on.  A scale-up to two instances then moves one
    read and one write per element instead of one read and two writes.

    ``lost_ranks``: source ranks whose fp32 state is gone (a failed GPU).  Every
    shard they held is read from another optimizer instance's copy instead,
    so nothing is read from them (an extension: the reference migrates each
    instance from itself).  A shard whose every copy is lost raises
    ValueError.  The bf16 params are the model shard's, held by every rank of
    its DP group, and are not affected.

    ``source_instance``: on a scale-up, the optimizer instance whose copy fills
    the new ones (the reference's ``group_src``, transfer.py:343-371).

    ``with_groups``: as for :func:`lower_transfer`.
    """
    space = src.space
    if src.strategy.optimizer_data_parallel_size != dst.strategy.optimizer_data_parallel_size:
        raise AssertionError("Group-ZeRO switch must keep the optimizer DP size")
    if not 0 <= source_instance < src.strategy.num_distributed_optimizer_instances:
        raise ValueError(f"source instance {source_instance} is not an optimizer instance of the source "
                         f"({src.strategy.num_distributed_optimizer_instances} instances)")
    lost = frozenset(int(r) for r in lost_ranks)
    if any(not 0 <= r < src.strategy.world_size for r in lost):
        raise ValueError(f"lost ranks must be ranks of the source world (0..{src.strategy.world_size - 1})")
    b = SegmentBuilder()
    bf16 = SegmentBuilder()
    for vp in space.all_virtual_params:
        if not (src.has_param(vp) and dst.has_param(vp)):
            continue
        g = vp.global_index if with_groups else 0
        # Destinations per source shard, in destination order.
        fills: Dict[int, Tuple[Holder, List[Holder]]] = {}
        for s, h in _backup_sources(src, dst, vp, scale_up, lost, source_instance):
            if h.offset < in_place_below:
                if s.offset != h.offset:
                    raise AssertionError(f"{vp.name}: a run below the in-place bound is not at its source's offset")
                cut = in_place_below - h.offset
                if cut < h.hi - h.lo:
                    b.add(0, 0, 4, s.offset + cut, in_place_below, h.hi - h.lo - cut, 1, 0, 0, group=g)
                continue
            fills.setdefault(id(s), (s, []))[1].append(h)
        for s, hs in fills.values():
            n = s.hi - s.lo
            for i in range(0, len(hs) - 1, 2):
                b.add(0, 0, 4, s.offset, hs[i].offset, n, 1, 0, 0, aux=(0, hs[i + 1].offset, 0), group=g, dup=True)
            if len(hs) % 2:
                b.add(0, 0, 4, s.offset, hs[-1].offset, n, 1, 0, 0, group=g)
        if copy_bf16:
            src_bf = {h.tp_rank: h for h in src.bf16_holders(vp)}
            for h in dst.bf16_holders(vp):
                s = src_bf.get(h.tp_rank)
                if s is None or (s.lo, s.hi) != (h.lo, h.hi):
                    raise AssertionError(f"{vp.name}: no matching source bf16 shard for a Group-ZeRO copy")
                bf16.add(ARENA_PARAM, ARENA_PARAM, 2, s.offset, h.offset, h.hi - h.lo, 1, 0, 0, group=g)
    return _assemble(b.table(), bf16.table(), b.group_array(), bf16.group_array(), with_groups)


# Largest interleaved piece: 64 MiB of fp32.  Timed on the same arenas in one process, pieces of
# 1, 16, 64 and 256 MiB took 31.10, 30.93, 30.91 and 30.90 ms on Llama-2-7B TP1DP8 -> TP4DP2
# (kinds one after another: 8% slower); 64 MiB leaves almost every segment whole.
INTERLEAVE_ELEMS = 1 << 24


def _split(table: np.ndarray, max_elems: int, groups: np.ndarray):
    """Cut segments into pieces of at most ``max_elems`` elements (whole rows for strided ones).

    Returns the pieces and the group of each.
    """
    out, out_g = [], []
    for s, g in zip(table, groups):
        n, rows = int(s["len"]), int(s["rows"])
        if n * rows <= max_elems:
            out.append(s)
            out_g.append(g)
            continue
        reads = not s["flags"] & SEG_ZERO_FILL
        aux = bool(s["flags"] & (SEG_CAST_BF16 | SEG_DUP))
        if rows == 1:
            for o in range(0, n, max_elems):
                p = s.copy()
                p["src_off"] += o if reads else 0
                p["dst_off"] += o
                p["aux_off"] += o if aux else 0
                p["len"] = min(max_elems, n - o)
                out.append(p)
                out_g.append(g)
            continue
        step = max(1, max_elems // n)
        for r in range(0, rows, step):
            p = s.copy()
            p["src_off"] += r * int(s["src_stride"])
            p["dst_off"] += r * int(s["dst_stride"])
            p["aux_off"] += r * int(s["aux_stride"])
            p["rows"] = min(step, rows - r)
            out.append(p)
            out_g.append(g)
    arr = np.array(out, dtype=SEGMENT_DTYPE) if out else np.zeros(0, dtype=SEGMENT_DTYPE)
    return arr, np.asarray(out_g, dtype=np.int64)


def _assemble(fp32: np.ndarray, bf16: np.ndarray, g32: np.ndarray, gbf: np.ndarray, with_groups: bool):
    """Replicate the fp32 segments over the three optimizer kinds; only main carries the bf16 cast.

    A duplicating segment duplicates within its own kind's arena.

    The kinds are interleaved segment by segment, in pieces of at most
    64 MiB: a main chunk that also writes the bf16 cast costs more than the
    others, and each XCD sweeps its own eighth of the plan, so every eighth
    must hold the same mix of kinds.  Running the kinds one after another
    instead costs 8% on Llama-2-7B.
    """
    base, gbase = _split(fp32, INTERLEAVE_ELEMS, g32)
    out = np.zeros(3 * len(base), dtype=SEGMENT_DTYPE)
    groups = np.zeros(3 * len(base), dtype=np.int64)
    for k in range(3):
        t = out[k::3]
        t[...] = base
        t["src_buf"] = k
        t["dst_buf"] = k
        groups[k::3] = 4 * gbase + 1 + k
        dup = (base["flags"] & SEG_DUP) != 0
        t["aux_buf"] = np.where(dup, k, t["aux_buf"])
        if k:
            t["flags"] &= ~np.uint32(SEG_CAST_BF16)
            for f in ("aux_buf", "aux_off", "aux_stride"):
                t[f] = np.where(dup, t[f], 0)
    table = np.concatenate([out, bf16])
    if not with_groups:
        return table
    groups = np.concatenate([groups, 4 * gbf])
    # The bf16 image counts to the parameter's bf16 group, a duplicate to its own kind.
    dup3 = (out["flags"] & SEG_DUP) != 0
    aux_groups = np.concatenate([np.where(dup3, groups[:len(out)], 4 * np.repeat(gbase, 3)), 4 * gbf])
    return table, groups.astype(np.uint32), aux_groups.astype(np.uint32)


def _units(table: np.ndarray) -> np.ndarray:
    return table["len"].astype(np.uint64) * table["rows"].astype(np.uint64)


def payload_bytes(table: np.ndarray) -> int:
    """Bytes written per execution (bf16 images and duplicates included)."""
    eb = table["elem_bytes"].astype(np.uint64)
    cast = ((table["flags"] & SEG_CAST_BF16) != 0).astype(np.uint64)
    dup = ((table["flags"] & SEG_DUP) != 0).astype(np.uint64)
    return int(np.sum(_units(table) * (eb + 2 * cast + eb * dup)))


def read_bytes(table: np.ndarray) -> int:
    """Bytes read per execution (zero fills read nothing)."""
    reads = (table["flags"] & SEG_ZERO_FILL) == 0
    return int(np.sum(_units(table) * table["elem_bytes"].astype(np.uint64) * reads.astype(np.uint64)))
