"""Arenas cut into granules: the storage of a state that can be handed to another process.

Device memory can be shared with another process one allocation at a time,
and only allocations smaller than 2 GiB; one arena of a 7B model's state is
tens of GB.  A shareable state therefore holds each of its four arenas as
consecutive granules of ``granule_bytes`` (the last one shorter), each its
own allocation: arena element ``e`` lives in granule ``e // g`` at element
``e % g``, with ``g = granule_bytes / element bytes``.  This module names the
granules and locates arena ranges in them, so that
:func:`.tensors.rebase_on_tensors` can re-base an arena plan onto them.

With ``granule_bytes=None`` every arena is one buffer: the layout of an
ordinary :class:`~..megatron_manager.training_state.TrainingState`.

Buffer order: the granules of ``main``, then ``exp_avg``, ``exp_avg_sq`` and
the bf16 ``param`` arena.
"""

from __future__ import annotations

from typing import List, Optional, Tuple

import numpy as np

from .layout import ARENA_NAMES, ARENA_PARAM, PIECE_DTYPE, StrategyLayout

ELEM_BYTES = (4, 4, 4, 2)
GRANULE_ALIGN = 256          # bytes: keeps every element's 16-byte alignment class inside its granule
DEFAULT_GRANULE_BYTES = 1 << 30
MAX_SHARED_ALLOCATION = 2 << 30   # exclusive


class GranuleBuffers:
    """The granules of every arena of one layout, with their keys, arena ranges and buffer ids."""

    def __init__(self, layout: StrategyLayout, granule_bytes: Optional[int] = DEFAULT_GRANULE_BYTES):
        if granule_bytes is not None:
            if granule_bytes <= 0 or granule_bytes % GRANULE_ALIGN:
                raise ValueError(f"granule_bytes must be a positive multiple of {GRANULE_ALIGN}")
            if granule_bytes >= MAX_SHARED_ALLOCATION:
                raise ValueError("granules must stay under 2 GiB: larger allocations cannot be shared")
        self.layout = layout
        self.granule_bytes = granule_bytes
        self.arena_numel = (layout.fp32_numel,) * 3 + (layout.bf16_numel,)
        self.keys: List[Tuple[str, int]] = []
        self.arena: List[int] = []
        self.offset: List[int] = []
        self.numel: List[int] = []
        self.granule_numel: List[int] = []
        self.first: List[int] = []          # buffer id of each arena's first granule
        for a, n in enumerate(self.arena_numel):
            g = n if granule_bytes is None else granule_bytes // ELEM_BYTES[a]
            self.granule_numel.append(max(g, 1))
            self.first.append(len(self.keys))
            for i, lo in enumerate(range(0, n, max(g, 1))):
                self.keys.append((ARENA_NAMES[a], i))
                self.arena.append(a)
                self.offset.append(lo)
                self.numel.append(min(g, n - lo))

    def __len__(self) -> int:
        return len(self.keys)

    def nbytes(self) -> List[int]:
        return [n * ELEM_BYTES[a] for a, n in zip(self.arena, self.numel)]

    def granules_of(self, arena: int) -> range:
        """Buffer ids of one arena's granules, in order."""
        end = self.first[arena + 1] if arena + 1 < len(self.first) else len(self.keys)
        return range(self.first[arena], end)

    def locate(self, arena: int, off: int) -> Tuple[int, int]:
        """(buffer id, element offset in that buffer) of arena element ``off``."""
        if not 0 <= off < self.arena_numel[arena]:
            raise ValueError(f"{ARENA_NAMES[arena]} element {off} lies outside the arena")
        j = off // self.granule_numel[arena]
        return self.first[arena] + j, off - j * self.granule_numel[arena]

    def locate_many(self, arenas: np.ndarray, offs: np.ndarray, extents: np.ndarray):
        """Vector form of :meth:`locate` for ranges [off, off + extent): (buffer ids, offsets,
        whether the whole range lies in that one granule)."""
        arenas = np.asarray(arenas, dtype=np.int64)
        offs = np.asarray(offs, dtype=np.int64)
        ext = np.asarray(extents, dtype=np.int64)
        g = np.asarray(self.granule_numel, dtype=np.int64)[np.clip(arenas, 0, 3)]
        total = np.asarray(self.arena_numel, dtype=np.int64)[np.clip(arenas, 0, 3)]
        j = offs // g
        local = offs - j * g
        ids = np.asarray(self.first, dtype=np.int64)[np.clip(arenas, 0, 3)] + j
        ok = (arenas >= 0) & (arenas <= ARENA_PARAM) & (offs >= 0) & (local + ext <= g) & (offs + ext <= total)
        return ids, local, ok

    def boundaries(self, arena: int, lo: int, hi: int) -> List[int]:
        """Granule starts strictly inside (lo, hi)."""
        g = self.granule_numel[arena]
        first = lo // g + 1
        return list(range(first * g, min(hi, self.arena_numel[arena]), g)) if first * g < hi else []

    def split_pieces(self, pieces: np.ndarray) -> np.ndarray:
        """Synthetic-data pieces (emrs_piece records addressed by arena) re-addressed by granule:
        a piece that crosses a granule boundary is cut there, its second part continuing at the
        next local element."""
        out = []
        for p in pieces:
            a, off, n = int(p["buf"]), int(p["buf_off"]), int(p["len"])
            at = 0
            while at < n:
                b, loc = self.locate(a, off + at)
                take = min(n - at, self.numel[b] - loc)
                q = p.copy()
                q["buf"], q["buf_off"], q["len"] = b, loc, take
                q["local_start"] = int(p["local_start"]) + at
                out.append(q)
                at += take
        arr = np.zeros(len(out), dtype=PIECE_DTYPE)
        if out:
            arr[:] = out
        return arr
