"""Range algebra and the device-synchronised timer.

Mirrors ``Range``, ``ParamRange`` and ``Timer`` of the reference
(elastic_megatron/resharding/util.py:19-214): a half-open element range, a
box of at most two ranges over a parameter's shape, and a wall-clock timer
that synchronises the device on entry and exit.
"""

from __future__ import annotations

import time
from typing import List, Optional, Sequence, Tuple


class Timer:
    """Synchronised wall-clock timer (util.py:19-46).

    ``synchronize`` is called on entry and exit; by default it is
    ``torch.cuda.synchronize`` when a device is present.
    """

    def __init__(self, unit: str = "ms", synchronize=None):
        self.unit = unit
        self.elapsed = 0.0
        self._sync = synchronize
        self._start = None

    def _do_sync(self):
        if self._sync is not None:
            self._sync()
            return
        import torch

        if torch.cuda.is_available():
            torch.cuda.synchronize()

    def __enter__(self):
        self._do_sync()
        self._start = time.perf_counter_ns()
        return self

    def __exit__(self, exc_type, exc, tb):
        self._do_sync()
        ns = time.perf_counter_ns() - self._start
        if self.unit == "ms":
            self.elapsed = ns / 1e6
        elif self.unit == "s":
            self.elapsed = ns / 1e9
        else:
            self.elapsed = ns
        return False


class Range:
    """Half-open range [start, end) of element indices (util.py:49-103)."""

    __slots__ = ("start", "end", "size", "is_normalized")

    def __init__(self, start: int, end: int):
        self.start = int(start)
        self.end = int(end)
        self.size = self.end - self.start
        self.is_normalized = self.start == 0

    def normalize(self, global_offset: Optional[int] = None) -> "Range":
        if global_offset is None:
            global_offset = self.start
        assert global_offset <= self.start
        return Range(self.start - global_offset, self.end - global_offset)

    def chunk(self, split: int) -> List["Range"]:
        assert split >= 1 and self.size % split == 0, f"cannot split {self} into {split}"
        n = self.size // split
        return [Range(self.start + i * n, self.start + (i + 1) * n) for i in range(split)]

    def is_contain(self, other: "Range") -> bool:
        assert isinstance(other, Range)
        return other.start >= self.start and other.end <= self.end

    def intersect(self, other: "Range") -> Optional["Range"]:
        lo, hi = max(self.start, other.start), min(self.end, other.end)
        return Range(lo, hi) if lo < hi else None

    def get_sub_range_slices(self, sub_range: "Range") -> Tuple[slice]:
        assert self.is_normalized
        assert isinstance(sub_range, Range)
        if self == sub_range:
            return (slice(None),)
        assert self.is_contain(sub_range)
        return (slice(sub_range.start, sub_range.end),)

    def __len__(self):
        return self.size

    def __eq__(self, other):
        return isinstance(other, Range) and other.start == self.start and other.end == self.end

    def __hash__(self):
        return hash((self.start, self.end))

    def __str__(self):
        return "%d,%d [%d]" % (self.start, self.end, self.size)

    __repr__ = __str__


class ParamRange:
    """A box of at most two ``Range`` over a parameter's shape (util.py:106-214)."""

    __slots__ = ("shapes", "dims", "is_normalized", "size")

    def __init__(self, ranges: Optional[Sequence[Range]] = None, param_shape: Optional[Sequence[int]] = None):
        if param_shape is not None:
            self.shapes = [Range(0, int(n)) for n in param_shape]
        else:
            self.shapes = list(ranges)
        self.dims = len(self.shapes)
        assert self.dims <= 2
        self.is_normalized = all(r.is_normalized for r in self.shapes)
        size = 1
        for r in self.shapes:
            size *= r.size
        self.size = size

    def normalize(self, global_offsets: Optional[Sequence[int]] = None) -> "ParamRange":
        if global_offsets is None:
            global_offsets = [0] * self.dims
        assert len(global_offsets) == self.dims
        return ParamRange(ranges=[r.normalize(o) for r, o in zip(self.shapes, global_offsets)])

    def to_shape(self) -> Tuple[int, ...]:
        return tuple(r.size for r in self.shapes)

    def chunk(self, split: int, dim: int) -> List["ParamRange"]:
        assert 0 <= dim < self.dims
        out = []
        for view in self.shapes[dim].chunk(split):
            shapes = list(self.shapes)
            shapes[dim] = view
            out.append(ParamRange(ranges=shapes))
        return out

    def is_contain(self, other: "ParamRange") -> int:
        """Dim along which ``other`` is a sub-range with every other dim equal, else -1."""
        assert isinstance(other, ParamRange)
        if self.dims != other.dims:
            return -1
        sub_dim = -1
        for dim, mine in enumerate(self.shapes):
            theirs = other.shapes[dim]
            if mine == theirs:
                continue
            if sub_dim != -1:
                return -1
            if mine.is_contain(theirs):
                sub_dim = dim
        return sub_dim

    def get_sub_range_slices(self, sub_range: "ParamRange") -> Tuple[slice, ...]:
        assert self.is_normalized
        assert isinstance(sub_range, ParamRange)
        slices = [slice(None)] * self.dims
        if self == sub_range:
            return tuple(slices)
        sub_dim = self.is_contain(sub_range)
        assert sub_dim != -1
        slices[sub_dim] = slice(sub_range.shapes[sub_dim].start, sub_range.shapes[sub_dim].end)
        return tuple(slices)

    def __eq__(self, other):
        return (
            isinstance(other, ParamRange)
            and self.dims == other.dims
            and all(a == b for a, b in zip(self.shapes, other.shapes))
        )

    def __hash__(self):
        return hash((self.dims, tuple(self.shapes)))

    def __len__(self):
        return self.size

    def __str__(self):
        return "".join(f"dim{i} = {r}  " for i, r in enumerate(self.shapes))

    __repr__ = __str__
