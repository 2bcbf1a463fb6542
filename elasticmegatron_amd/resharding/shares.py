"""One destination rank's share of a copy plan.

With one rank per GPU, GPU g would run the part of the plan that writes the
fp32 shard it hosts: the segments whose destination lies in rank g's region of
the ``main`` / ``exp_avg`` / ``exp_avg_sq`` arenas, each with the fused bf16
cast of the pieces it writes.  In the reference each rank likewise receives
only into its own optimizer tensors (transfer.py:291-341; the receive side of
``Communicator``, communicator.py:61-96).

- A duplicating segment (Group ZeRO: one read, two instances) whose two
  destinations sit on different ranks becomes one plain copy per rank: each
  GPU pulls its own copy.
- Segments whose primary destination is the bf16 param arena (bf16 copied from
  the source's params, or the zero rows of a re-padded vocabulary) write no
  fp32 shard.  Every DP replica holds the whole bf16 shard, so they are
  returned apart, as the side the bf16 all-gather completes
  (training_state.py:176-197).

The lowering merges a contiguous continuation into the previous segment, so a
segment may run on from one rank's region into the next; such a segment is cut
at the boundary, one piece per rank.  The shares partition the plan's writes:
run one after another on the same buffers, they write exactly what the whole
plan writes.
"""

from __future__ import annotations

from typing import List, Tuple

import numpy as np

from .layout import ARENA_PARAM, SEG_CAST_BF16, SEG_DUP, SEG_ZERO_FILL, StrategyLayout


def _last_elem(off, rows, stride, n):
    """One past the last element a segment touches on one side (rows >= 1, len >= 1)."""
    return off + (rows - 1) * stride + n


def fp32_rank_of(offsets: np.ndarray, layout: StrategyLayout) -> np.ndarray:
    """Rank whose fp32 region holds each element offset (-1 for offsets in no rank's region)."""
    base = np.asarray(layout.rank_base, dtype=np.uint64)
    end = base + np.asarray(layout.rank_numel, dtype=np.uint64)
    r = np.searchsorted(base, offsets, side="right").astype(np.int64) - 1
    ok = (r >= 0) & (offsets < end[np.maximum(r, 0)])
    return np.where(ok, r, -1)


def _cut_at_rank_boundaries(table: np.ndarray, dst: StrategyLayout) -> np.ndarray:
    """The table with every one-row fp32 segment that crosses into another rank's region (on its
    destination, or on its duplicate's) cut into one piece per rank, in the plan's order."""
    n = table["len"]
    one_row = table["rows"] == 1
    fp32 = table["dst_buf"] != ARENA_PARAM
    dup = (table["flags"] & SEG_DUP) != 0
    lo, alo = table["dst_off"], table["aux_off"]
    cross = fp32_rank_of(lo, dst) != fp32_rank_of(lo + n - 1, dst)
    cross |= dup & (fp32_rank_of(alo, dst) != fp32_rank_of(alo + n - 1, dst))
    cut = np.nonzero(one_row & fp32 & cross)[0]
    if len(cut) == 0:
        return table
    base = np.asarray(dst.rank_base, dtype=np.uint64)
    second = SEG_CAST_BF16 | SEG_DUP
    parts, prev = [], 0
    for i in cut:
        s = table[i]
        m, d = int(s["len"]), int(s["dst_off"])
        edges = {0, m}
        edges.update(int(b) - d for b in base[(base > d) & (base < d + m)])
        if s["flags"] & SEG_DUP:
            a = int(s["aux_off"])
            edges.update(int(b) - a for b in base[(base > a) & (base < a + m)])
        edges = sorted(edges)
        pieces = np.repeat(table[i:i + 1], len(edges) - 1)
        start = np.asarray(edges[:-1], dtype=np.uint64)
        pieces["len"] = np.diff(np.asarray(edges, dtype=np.uint64))
        pieces["src_off"] += start
        pieces["dst_off"] += start
        if s["flags"] & second:
            pieces["aux_off"] += start
        parts += [table[prev:i], pieces]
        prev = i + 1
    parts.append(table[prev:])
    return np.concatenate(parts)


def destination_rank_shares(table: np.ndarray, dst: StrategyLayout) -> Tuple[List[np.ndarray], np.ndarray]:
    """(one segment table per destination rank, the bf16-arena segments) of a plan over arenas.

    Raises ``ValueError`` for a segment that writes outside every rank's fp32 region, or a
    strided one that spans two regions; a plan lowered from the layout holds neither.  Each
    table keeps the plan's order.
    """
    table = _cut_at_rank_boundaries(table, dst)
    n = table["len"]
    rows = table["rows"]
    fp32 = table["dst_buf"] != ARENA_PARAM
    lo = table["dst_off"]
    hi = _last_elem(lo, rows, table["dst_stride"], n)
    rank = fp32_rank_of(lo, dst)
    if np.any(fp32 & ((rank < 0) | (fp32_rank_of(hi - 1, dst) != rank))):
        raise ValueError("a segment's destination is not inside one rank's fp32 region")
    dup = (table["flags"] & SEG_DUP) != 0
    if np.any(dup & ((table["flags"] & SEG_CAST_BF16) != 0)):
        raise ValueError("a segment both duplicates and casts")
    aux_rank = np.full(len(table), -1, dtype=np.int64)
    if dup.any():
        if np.any(dup & ((~fp32) | (table["aux_buf"] == ARENA_PARAM))):
            raise ValueError("a duplicating segment writes the bf16 arena")
        alo = table["aux_off"][dup]
        ahi = _last_elem(alo, rows[dup], table["aux_stride"][dup], n[dup])
        ar = fp32_rank_of(alo, dst)
        if np.any((ar < 0) | (fp32_rank_of(ahi - 1, dst) != ar)):
            raise ValueError("a duplicate's destination is not inside one rank's fp32 region")
        aux_rank[dup] = ar
    split = dup & (aux_rank != rank)

    # Primary writes: the segment itself, a split duplicate losing its second destination.
    prim = table.copy()
    prim["flags"][split] &= ~np.uint32(SEG_DUP)
    prim["aux_buf"][split] = 0
    prim["aux_off"][split] = 0
    prim["aux_stride"][split] = 0
    # Second writes of split duplicates: a plain copy into the other instance.
    second = table[split].copy()
    second["dst_buf"] = second["aux_buf"]
    second["dst_off"] = second["aux_off"]
    second["dst_stride"] = second["aux_stride"]
    second["flags"] &= ~np.uint32(SEG_DUP)
    second["aux_buf"] = 0
    second["aux_off"] = 0
    second["aux_stride"] = 0

    # Each split duplicate's second copy goes right after its primary, so every share keeps the
    # plan's order.
    order = np.concatenate([np.arange(len(table), dtype=np.float64),
                            np.nonzero(split)[0].astype(np.float64) + 0.5])
    rows_all = np.concatenate([prim, second])
    rank_all = np.concatenate([np.where(fp32, rank, -1), aux_rank[split]])
    sort = np.argsort(order, kind="stable")
    rows_all, rank_all = rows_all[sort], rank_all[sort]
    shares = [rows_all[rank_all == g] for g in range(dst.strategy.world_size)]
    return shares, rows_all[rank_all < 0]


def pull_bytes(share: np.ndarray, src: StrategyLayout) -> Tuple[np.ndarray, int]:
    """(bytes the share reads from each source rank's fp32 region, bytes it reads from the bf16
    arena).  With one rank per GPU in both layouts, entry g is what GPU g reads from its own HBM
    when the share is GPU g's, and the rest is what it pulls from peers."""
    W = src.strategy.world_size
    out = np.zeros(W, dtype=np.int64)
    reads = share[(share["flags"] & SEG_ZERO_FILL) == 0]
    bf16 = reads["src_buf"] == ARENA_PARAM
    param = int((reads["len"][bf16] * reads["rows"][bf16] * reads["elem_bytes"][bf16]).sum())
    fp32 = reads[~bf16]
    base = np.asarray(src.rank_base, dtype=np.uint64)
    end = base + np.asarray(src.rank_numel, dtype=np.uint64)
    lo = fp32["src_off"]
    hi = _last_elem(lo, fp32["rows"], fp32["src_stride"], fp32["len"])
    r_lo, r_hi = fp32_rank_of(lo, src), fp32_rank_of(hi - 1, src)
    if np.any(r_lo < 0) or np.any(r_hi < 0):
        raise ValueError("a segment reads outside every rank's fp32 region")
    same = r_lo == r_hi
    np.add.at(out, r_lo[same], (fp32["len"][same] * fp32["rows"][same] * fp32["elem_bytes"][same]).astype(np.int64))
    for s in fp32[~same]:
        if int(s["rows"]) != 1:
            raise ValueError("a strided segment reads across a rank boundary")
        a, b = int(s["src_off"]), int(s["src_off"]) + int(s["len"])
        for g in range(W):
            n = min(b, int(end[g])) - max(a, int(base[g]))
            if n > 0:
                out[g] += n * int(s["elem_bytes"])
    return out, param
