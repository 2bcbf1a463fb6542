"""Per-tensor buffers: the reference's own storage format at the transfer boundary.

The reference's executor reads and writes one tensor per (rank, parameter,
kind): the ``main_weight`` / ``exp_avg`` / ``exp_avg_sq`` of an
``OptimizerTensorInfo`` (resharding_metadata.py:19-40) and the bf16 model
parameter of each model-parallel shard (training_state.py:176-197).  The
arena layout of :mod:`.layout` packs those tensors into four buffers; this
module names every one of them and re-bases an arena plan onto a list of
separate tensors, so that a caller holding per-parameter tensors (one buffer
id per tensor) runs the same transfer without packing anything.

Buffer order on each side: every fp32 holder of every parameter for
``main``, then the same for ``exp_avg``, then ``exp_avg_sq``, then every bf16
holder; holders in arena order.
"""

from __future__ import annotations

import bisect
from typing import Dict, List, Tuple

import numpy as np

from .layout import ARENA_NAMES, ARENA_PARAM, SEG_CAST_BF16, SEG_DUP, SEG_ZERO_FILL, SEGMENT_DTYPE, StrategyLayout

FP32_KINDS = ("main", "exp_avg", "exp_avg_sq")


class TensorBuffers:
    """Every stored tensor of one layout, with its key, arena range and buffer id."""

    def __init__(self, layout: StrategyLayout):
        self.layout = layout
        space = layout.space
        fp32, bf16 = [], []
        for vp in space.all_virtual_params:
            if not layout.has_param(vp):
                continue
            for h in layout.fp32_holders(vp):
                fp32.append((h.offset, h.hi - h.lo, h.rank, vp.name))
            for h in layout.bf16_holders(vp):
                bf16.append((h.offset, h.hi - h.lo, layout.shard_keys[h.rank], vp.name))
        fp32.sort()
        bf16.sort()
        self.keys: List[Tuple] = []
        self.arena: List[int] = []
        self.offset: List[int] = []
        self.numel: List[int] = []
        for k, kind in enumerate(FP32_KINDS):
            for off, n, rank, name in fp32:
                self._add((kind, rank, name), k, off, n)
        for off, n, shard, name in bf16:
            self._add(("param", shard, name), ARENA_PARAM, off, n)
        # Per arena: sorted starts and the buffer id of each.
        self._starts: Dict[int, List[int]] = {}
        self._ids: Dict[int, List[int]] = {}
        for i, (a, off) in enumerate(zip(self.arena, self.offset)):
            self._starts.setdefault(a, []).append(off)
            self._ids.setdefault(a, []).append(i)
        for a in self._starts:
            order = np.argsort(self._starts[a], kind="stable")
            self._starts[a] = [self._starts[a][j] for j in order]
            self._ids[a] = [self._ids[a][j] for j in order]

    def _add(self, key, arena, off, n):
        self.keys.append(key)
        self.arena.append(arena)
        self.offset.append(off)
        self.numel.append(n)

    def __len__(self) -> int:
        return len(self.keys)

    def nbytes(self) -> List[int]:
        return [n * (2 if a == ARENA_PARAM else 4) for a, n in zip(self.arena, self.numel)]

    def locate(self, arena: int, off: int) -> Tuple[int, int]:
        """(buffer id, element offset in that buffer) of arena element ``off``."""
        starts = self._starts[arena]
        j = bisect.bisect_right(starts, off) - 1
        if j < 0:
            raise ValueError(f"{ARENA_NAMES[arena]} element {off} lies before every tensor")
        b = self._ids[arena][j]
        if off >= self.offset[b] + self.numel[b]:
            raise ValueError(f"{ARENA_NAMES[arena]} element {off} lies in padding")
        return b, off - self.offset[b]

    def locate_many(self, arenas: np.ndarray, offs: np.ndarray, extents: np.ndarray):
        """Vector form of :meth:`locate` for ranges [off, off + extent): (buffer ids, offsets,
        whether the whole range lies in that one tensor).  Rows whose arena has no tensors
        come back with ok = False."""
        arenas = np.asarray(arenas, dtype=np.int64)
        offs = np.asarray(offs, dtype=np.int64)
        ids = np.zeros(len(offs), dtype=np.int64)
        local = np.zeros(len(offs), dtype=np.int64)
        ok = np.zeros(len(offs), dtype=bool)
        numel = np.asarray(self.numel, dtype=np.int64)
        for a in np.unique(arenas):
            m = arenas == a
            if int(a) not in self._starts:
                continue
            starts = np.asarray(self._starts[int(a)], dtype=np.int64)
            idmap = np.asarray(self._ids[int(a)], dtype=np.int64)
            j = np.searchsorted(starts, offs[m], side="right") - 1
            valid = j >= 0
            jj = np.where(valid, j, 0)
            b = idmap[jj]
            loc = offs[m] - starts[jj]
            ids[m], local[m] = b, loc
            ok[m] = valid & (loc + np.asarray(extents)[m] <= numel[b])
        return ids, local, ok

    def boundaries(self, arena: int, lo: int, hi: int) -> List[int]:
        """Tensor starts strictly inside (lo, hi)."""
        starts = self._starts[arena]
        i = bisect.bisect_right(starts, lo)
        j = bisect.bisect_left(starts, hi)
        return starts[i:j]

    def views(self, state) -> list:
        """The tensors of ``state`` in buffer order, as views into its arenas."""
        arenas = state.arenas()
        return [arenas[a][o:o + n] for a, o, n in zip(self.arena, self.offset, self.numel)]


def rebase_on_tensors(table: np.ndarray, src: TensorBuffers, dst: TensorBuffers) -> np.ndarray:
    """The arena plan ``table`` re-expressed over per-tensor buffers.

    A one-row segment that runs across tensor boundaries (tensors of one
    parameter on consecutive ranks can be adjacent in an arena) is cut at
    every boundary on the source, destination and second-destination (bf16
    image or duplicate) sides; a strided segment always lies inside one
    tensor on each side.  Segments that need no cut are mapped in bulk.
    """
    table = table[(table["len"] > 0)]
    n = len(table)
    if n == 0:
        return np.zeros(0, dtype=SEGMENT_DTYPE)
    ln = table["len"].astype(np.int64)
    rows = table["rows"].astype(np.int64)
    zero = (table["flags"] & SEG_ZERO_FILL) != 0
    aux = (table["flags"] & (SEG_CAST_BF16 | SEG_DUP)) != 0
    ext_s = np.where(rows > 1, (rows - 1) * table["src_stride"].astype(np.int64), 0) + ln
    ext_d = np.where(rows > 1, (rows - 1) * table["dst_stride"].astype(np.int64), 0) + ln
    ext_a = np.where(rows > 1, (rows - 1) * table["aux_stride"].astype(np.int64), 0) + ln
    sb, so, s_ok = src.locate_many(table["src_buf"], table["src_off"], ext_s)
    db, do, d_ok = dst.locate_many(table["dst_buf"], table["dst_off"], ext_d)
    # The second destination's arena: the param arena for a bf16 image, the segment's own for a duplicate.
    ab, ao, a_ok = dst.locate_many(np.where(aux, table["aux_buf"], ARENA_PARAM), table["aux_off"], ext_a)
    fits = (zero | s_ok) & d_ok & (~aux | a_ok)
    out = table[fits].copy()
    f = np.flatnonzero(fits)
    out["src_buf"] = np.where(zero[f], 0, sb[f])
    out["src_off"] = np.where(zero[f], 0, so[f])
    out["dst_buf"], out["dst_off"] = db[f], do[f]
    out["aux_buf"] = np.where(aux[f], ab[f], out["aux_buf"])
    out["aux_off"] = np.where(aux[f], ao[f], out["aux_off"])
    rest = [_cut(s, src, dst) for s in table[~fits]]
    if rest:
        out = np.concatenate([out] + rest)
    return out


def _cut(s, src: TensorBuffers, dst: TensorBuffers) -> np.ndarray:
    """One segment that crosses tensor boundaries, cut at each of them."""
    n, rows = int(s["len"]), int(s["rows"])
    if rows > 1:
        raise AssertionError("a strided segment leaves its tensor")
    zero = bool(int(s["flags"]) & SEG_ZERO_FILL)
    aux = bool(int(s["flags"]) & (SEG_CAST_BF16 | SEG_DUP))
    sa, da, aa = int(s["src_buf"]), int(s["dst_buf"]), int(s["aux_buf"])
    so, do, ao = int(s["src_off"]), int(s["dst_off"]), int(s["aux_off"])
    pts = {0, n}
    if not zero:
        pts.update(b - so for b in src.boundaries(sa, so, so + n))
    pts.update(b - do for b in dst.boundaries(da, do, do + n))
    if aux:
        pts.update(b - ao for b in dst.boundaries(aa, ao, ao + n))
    cuts = sorted(pts)
    out = np.zeros(len(cuts) - 1, dtype=SEGMENT_DTYPE)
    for i, (c0, c1) in enumerate(zip(cuts, cuts[1:])):
        r = s.copy()
        if zero:
            r["src_buf"], r["src_off"] = 0, 0
        else:
            r["src_buf"], r["src_off"] = src.locate(sa, so + c0)
        r["dst_buf"], r["dst_off"] = dst.locate(da, do + c0)
        if aux:
            r["aux_buf"], r["aux_off"] = dst.locate(aa, ao + c0)
        r["len"] = c1 - c0
        out[i] = r
    return out
