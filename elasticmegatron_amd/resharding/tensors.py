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


def rebase_on_tensors(table: np.ndarray, src, dst, return_origin: bool = False):
    """The arena plan ``table`` re-expressed over separately allocated buffers.

    ``src`` and ``dst`` name the buffers and where each sits in its arena:
    one per stored tensor (:class:`TensorBuffers`) or consecutive granules of
    every arena (:class:`.granules.GranuleBuffers`); anything with their
    ``locate`` / ``locate_many`` / ``boundaries`` works.  A segment that runs
    across buffer boundaries on the source, destination or second-destination
    (bf16 image or duplicate) side is cut at every one of them: a one-row
    segment at the boundary, a strided one between rows, with a row that
    straddles a boundary taken out as a row of its own.  Segments that need
    no cut are mapped in bulk.

    With ``return_origin`` also returns, per output row, the index of the
    input row it came from (so that per-segment data such as verification
    groups can follow the cuts).
    """
    keep = np.flatnonzero(table["len"] > 0)
    table = table[keep]
    n = len(table)
    if n == 0:
        out = np.zeros(0, dtype=SEGMENT_DTYPE)
        return (out, np.zeros(0, dtype=np.int64)) if return_origin else out
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
    parts, origin = [out], [keep[f]]
    for i in np.flatnonzero(~fits):
        cut = _cut(table[i], src, dst)
        parts.append(cut)
        origin.append(np.full(len(cut), keep[i], dtype=np.int64))
    out = np.concatenate(parts)
    return (out, np.concatenate(origin).astype(np.int64)) if return_origin else out


def _sides(s):
    """(side, arena field, offset field, stride field) of every buffer a segment touches."""
    flags = int(s["flags"])
    out = []
    if not flags & SEG_ZERO_FILL:
        out.append(("src", "src_buf", "src_off", "src_stride"))
    out.append(("dst", "dst_buf", "dst_off", "dst_stride"))
    if flags & (SEG_CAST_BF16 | SEG_DUP):
        out.append(("dst", "aux_buf", "aux_off", "aux_stride"))
    return out


def _rows_of(s, r0: int, r1: int):
    """Rows [r0, r1) of a strided segment, as a segment of its own."""
    r = s.copy()
    for _, _, off, stride in (("", "", "src_off", "src_stride"), ("", "", "dst_off", "dst_stride"),
                              ("", "", "aux_off", "aux_stride")):
        r[off] = int(s[off]) + r0 * int(s[stride])
    if int(s["flags"]) & SEG_ZERO_FILL:
        r["src_off"] = s["src_off"]
    r["rows"] = r1 - r0
    return r


def _cut(s, src, dst) -> np.ndarray:
    """One segment that crosses buffer boundaries, cut at each of them."""
    n, rows = int(s["len"]), int(s["rows"])
    sets = {"src": src, "dst": dst}
    if rows > 1:
        # Walk down the rows: the leading rows clear of every side's next boundary form one
        # piece; a row that straddles a boundary is cut on its own.
        out, r = [], 0
        while r < rows:
            rest = _rows_of(s, r, rows)
            take = _clean_rows(rest, sets, n, rows - r)
            if take >= rows - r:
                out.append(_cut_or_keep(rest, src, dst))
                break
            take = max(take, 1)
            out.append(_cut_or_keep(_rows_of(s, r, r + take), src, dst))
            r += take
        return np.concatenate(out)
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


def _clean_rows(s, sets, n: int, rows: int) -> int:
    """How many leading rows of a strided segment lie clear of every buffer boundary."""
    clean = rows
    for side, buf, off, stride in _sides(s):
        o, st = int(s[off]), int(s[stride])
        b = sets[side].boundaries(int(s[buf]), o, o + (rows - 1) * st + n)
        if not b:
            continue
        if st == 0:     # every row reads the same elements: each is cut on its own
            return 0
        k, c = divmod(b[0] - o, st)
        clean = min(clean, k + 1 if c >= n else k)
    return clean


def _cut_or_keep(s, src, dst) -> np.ndarray:
    """``s`` re-based as one segment when it crosses no boundary, else cut."""
    n, rows = int(s["len"]), int(s["rows"])
    sets = {"src": src, "dst": dst}
    for side, buf, off, stride in _sides(s):
        o = int(s[off])
        ext = (rows - 1) * int(s[stride]) + n if rows > 1 else n
        if sets[side].boundaries(int(s[buf]), o, o + ext):
            return _cut(s, src, dst)
    r = s.copy()
    if int(s["flags"]) & SEG_ZERO_FILL:
        r["src_buf"], r["src_off"] = 0, 0
    else:
        r["src_buf"], r["src_off"] = src.locate(int(s["src_buf"]), int(s["src_off"]))
    r["dst_buf"], r["dst_off"] = dst.locate(int(s["dst_buf"]), int(s["dst_off"]))
    if int(s["flags"]) & (SEG_CAST_BF16 | SEG_DUP):
        r["aux_buf"], r["aux_off"] = dst.locate(int(s["aux_buf"]), int(s["aux_off"]))
    out = np.zeros(1, dtype=SEGMENT_DTYPE)
    out[0] = r
    return out
