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
from typing import Iterable, List, Sequence, Tuple

import numpy as np

from .layout import (ARENA_PARAM, Geometry, Holder, SEGMENT_DTYPE, StrategyLayout)


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
    def __init__(self):
        self.rows: List[Tuple] = []

    def add(self, sbuf: int, dbuf: int, eb: int, so: int, do: int, n: int, rows: int, ss: int, ds: int) -> None:
        if n <= 0 or rows <= 0:
            return
        if self.rows and rows == 1:
            p = self.rows[-1]
            if (p[0] == sbuf and p[1] == dbuf and p[2] == eb and p[7] == 1
                    and p[4] + p[6] == so and p[5] + p[6] == do):
                self.rows[-1] = (p[0], p[1], p[2], 0, p[4], p[5], p[6] + n, 1, 0, 0)
                return
        self.rows.append((sbuf, dbuf, eb, 0, so, do, n, rows, ss, ds))

    def table(self) -> np.ndarray:
        arr = np.zeros(len(self.rows), dtype=SEGMENT_DTYPE)
        if self.rows:
            arr[:] = self.rows
        return arr


def _src_replica(vp, holders: List[Holder]) -> List[Holder]:
    out = [h for h in holders if h.instance == 0]
    if not vp.tensor_parallel_attr.tensor_model_parallel:
        out = [h for h in out if h.tp_rank == 0]
    return out


def lower_transfer(src: StrategyLayout, dst: StrategyLayout, include_fp32: bool = True,
                   include_bf16: bool = True) -> np.ndarray:
    """Segments of a switch between two layouts of the same model.

    Buffers 0..2 are the fp32 arenas (main, exp_avg, exp_avg_sq) and buffer 3
    the bf16 param arena, on both sides.
    """
    space = src.space
    assert dst.space is space
    fp32 = SegmentBuilder()
    bf16 = SegmentBuilder()
    for vp in space.all_virtual_params:
        if not (src.has_param(vp) and dst.has_param(vp)):
            continue  # tied output layer at PP 1 (transfer.py:324-330)
        if include_fp32:
            s_rects = [r for h in _src_replica(vp, src.fp32_holders(vp))
                       for r in holder_rects(h, src.geometry(vp, h.tp_rank))]
            covered = 0
            want = 0
            for h in dst.fp32_holders(vp):
                want += h.hi - h.lo
                d_rects = holder_rects(h, dst.geometry(vp, h.tp_rank))
                for so, do, n, rows, ss, ds in _intersections(s_rects, d_rects):
                    fp32.add(0, 0, 4, so, do, n, rows, ss, ds)
                    covered += n * rows
            if covered != want:
                raise AssertionError(f"{vp.name}: fp32 plan covers {covered} of {want} elements")
        if include_bf16:
            s_rects = [r for h in _src_replica(vp, src.bf16_holders(vp))
                       for r in holder_rects(h, src.geometry(vp, h.tp_rank))]
            covered = 0
            want = 0
            for h in dst.bf16_holders(vp):
                want += h.hi - h.lo
                d_rects = holder_rects(h, dst.geometry(vp, h.tp_rank))
                for so, do, n, rows, ss, ds in _intersections(s_rects, d_rects):
                    bf16.add(ARENA_PARAM, ARENA_PARAM, 2, so, do, n, rows, ss, ds)
                    covered += n * rows
            if covered != want:
                raise AssertionError(f"{vp.name}: bf16 plan covers {covered} of {want} elements")
    return _assemble(fp32.table(), bf16.table())


def lower_redundant_backup(src: StrategyLayout, dst: StrategyLayout, scale_up: bool) -> np.ndarray:
    """fp32 segments of a Group-ZeRO switch (instances change, shards do not)."""
    space = src.space
    if src.strategy.optimizer_data_parallel_size != dst.strategy.optimizer_data_parallel_size:
        raise AssertionError("Group-ZeRO switch must keep the optimizer DP size")
    b = SegmentBuilder()
    for vp in space.all_virtual_params:
        if not (src.has_param(vp) and dst.has_param(vp)):
            continue
        src_by = {(h.instance, h.tp_rank, h.lo): h for h in src.fp32_holders(vp)}
        for h in dst.fp32_holders(vp):
            inst = 0 if scale_up else h.instance
            s = src_by.get((inst, h.tp_rank, h.lo))
            if s is None or s.hi != h.hi:
                raise AssertionError(f"{vp.name}: no matching source shard for a Group-ZeRO copy")
            b.add(0, 0, 4, s.offset, h.offset, h.hi - h.lo, 1, 0, 0)
    return _assemble(b.table(), np.zeros(0, dtype=SEGMENT_DTYPE))


def _assemble(fp32: np.ndarray, bf16: np.ndarray) -> np.ndarray:
    parts = []
    for k in range(3):
        t = fp32.copy()
        t["src_buf"] = k
        t["dst_buf"] = k
        parts.append(t)
    parts.append(bf16)
    return np.concatenate(parts)


def payload_bytes(table: np.ndarray) -> int:
    return int(np.sum(table["len"].astype(np.uint64) * table["rows"] * table["elem_bytes"]))
