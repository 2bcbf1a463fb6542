"""Index boxes of a parameter and the device-synchronised timer.

The planner describes which part of a parameter a rank holds with two value
types: ``Range``, a half-open interval of element indices along one
dimension, and ``ParamRange``, the product of one or two such intervals (a
1-D piece or a 2-D block of rows x columns).  Both are immutable values,
hashable and compared by their bounds, so they key dictionaries and caches.

Public names and behaviour follow the reference's ``Range``, ``ParamRange``
and ``Timer`` (elastic_megatron/resharding/util.py:19-214), which callers of
the planner use: ``normalize``, ``chunk``, ``is_contain``,
``get_sub_range_slices``, ``size``, ``is_normalized`` and ``elapsed``.
"""

from __future__ import annotations

import time
from dataclasses import dataclass
from typing import Callable, Iterable, List, Optional, Sequence, Tuple

# Seconds per unit of Timer.elapsed; anything else is reported in nanoseconds.
_TIMER_SCALE_NS = {"ms": 1e6, "s": 1e9}


def _device_sync() -> None:
    import torch

    if torch.cuda.is_available():
        torch.cuda.synchronize()


class Timer:
    """Wall-clock time of a ``with`` block, with the device drained at both ends.

    ``elapsed`` is in ``unit``: "ms", "s", or nanoseconds for any other value
    (the reference's units, util.py:19-46).  ``synchronize`` replaces the
    device drain, e.g. with a no-op on the CPU.
    """

    def __init__(self, unit: str = "ms", synchronize: Optional[Callable[[], None]] = None):
        self.unit = unit
        self.elapsed = 0.0
        self._drain = synchronize or _device_sync
        self._t0 = 0

    def __enter__(self) -> "Timer":
        self._drain()
        self._t0 = time.perf_counter_ns()
        return self

    def __exit__(self, *exc) -> bool:
        self._drain()
        ns = time.perf_counter_ns() - self._t0
        scale = _TIMER_SCALE_NS.get(self.unit)
        self.elapsed = ns / scale if scale else ns
        return False


@dataclass(frozen=True)
class Range:
    """Element indices ``start <= i < end`` along one dimension."""

    start: int
    end: int

    def __post_init__(self):
        object.__setattr__(self, "start", int(self.start))
        object.__setattr__(self, "end", int(self.end))

    @property
    def size(self) -> int:
        return self.end - self.start

    @property
    def is_normalized(self) -> bool:
        """True when the interval starts at index 0."""
        return self.start == 0

    def __len__(self) -> int:
        return self.size

    def shifted(self, by: int) -> "Range":
        return Range(self.start + by, self.end + by)

    def normalize(self, global_offset: Optional[int] = None) -> "Range":
        """The interval relative to ``global_offset`` (default: its own start),
        which must not lie past the start."""
        origin = self.start if global_offset is None else int(global_offset)
        if origin > self.start:
            raise AssertionError(f"offset {origin} lies past the start of {self}")
        return self.shifted(-origin)

    def chunk(self, split: int) -> List["Range"]:
        """``split`` consecutive equal parts; the size must divide evenly."""
        if split < 1 or self.size % split:
            raise AssertionError(f"{self} does not split into {split} equal parts")
        step = self.size // split
        return [Range(self.start + k * step, self.start + (k + 1) * step) for k in range(split)]

    def is_contain(self, other: "Range") -> bool:
        """True when ``other`` lies inside this interval."""
        if not isinstance(other, Range):
            raise AssertionError("is_contain needs a Range")
        return self.start <= other.start and other.end <= self.end

    def intersect(self, other: "Range") -> Optional["Range"]:
        """The common part of two intervals, or None when it is empty."""
        lo = max(self.start, other.start)
        hi = min(self.end, other.end)
        return Range(lo, hi) if hi > lo else None

    def get_sub_range_slices(self, sub_range: "Range") -> Tuple[slice]:
        """Index tuple selecting ``sub_range`` out of a tensor that holds this
        (normalized) interval: ``(slice(None),)`` when they are equal."""
        if not self.is_normalized or not isinstance(sub_range, Range):
            raise AssertionError("slices are taken from a normalized Range by a Range")
        if sub_range == self:
            return (slice(None),)
        if not self.is_contain(sub_range):
            raise AssertionError(f"{sub_range} is not inside {self}")
        return (slice(sub_range.start, sub_range.end),)

    def __str__(self) -> str:
        return f"[{self.start}:{self.end})"

    __repr__ = __str__


class ParamRange:
    """The box ``ranges[0] x ranges[1]`` (or one range) of a parameter.

    Built from explicit ranges, or from a shape as the whole parameter
    (every range starting at 0).  At most two dimensions.
    """

    __slots__ = ("_box",)

    def __init__(self, ranges: Optional[Iterable[Range]] = None,
                 param_shape: Optional[Sequence[int]] = None):
        if param_shape is not None:
            box = tuple(Range(0, n) for n in param_shape)
        else:
            box = tuple(ranges)
        if len(box) > 2:
            raise AssertionError("a ParamRange has at most two dimensions")
        object.__setattr__(self, "_box", box)

    def __setattr__(self, name, value):
        raise AttributeError("ParamRange is immutable")

    def __reduce__(self):
        return (ParamRange, (self._box,))

    @property
    def shapes(self) -> Tuple[Range, ...]:
        return self._box

    @property
    def dims(self) -> int:
        return len(self._box)

    @property
    def is_normalized(self) -> bool:
        return all(r.start == 0 for r in self._box)

    @property
    def size(self) -> int:
        n = 1
        for r in self._box:
            n *= r.size
        return n

    def __len__(self) -> int:
        return self.size

    def to_shape(self) -> Tuple[int, ...]:
        return tuple(r.size for r in self._box)

    def normalize(self, global_offsets: Optional[Sequence[int]] = None) -> "ParamRange":
        """Each range relative to its offset (default 0 in every dimension)."""
        offsets = [0] * self.dims if global_offsets is None else list(global_offsets)
        if len(offsets) != self.dims:
            raise AssertionError("one offset per dimension")
        return ParamRange(ranges=[r.normalize(o) for r, o in zip(self._box, offsets)])

    def chunk(self, split: int, dim: int) -> List["ParamRange"]:
        """``split`` equal boxes along ``dim``; the other dimension is kept whole."""
        if not 0 <= dim < self.dims:
            raise AssertionError(f"no dimension {dim} in {self}")
        return [ParamRange(ranges=self._box[:dim] + (part,) + self._box[dim + 1:])
                for part in self._box[dim].chunk(split)]

    def is_contain(self, other: "ParamRange") -> int:
        """The dimension along which ``other`` is a sub-box of this one, else -1.

        ``other`` must have as many dimensions and differ in exactly one of
        them, where its range lies inside this box's.  As in the reference,
        the dimensions are scanned in order and the first one whose range
        contains the other's settles the answer unless a later dimension
        also differs; so -1 is also returned for equal boxes.
        """
        if not isinstance(other, ParamRange):
            raise AssertionError("is_contain needs a ParamRange")
        if other.dims != self.dims:
            return -1
        differing = [d for d in range(self.dims) if self._box[d] != other._box[d]]
        inside = [d for d in differing if self._box[d].is_contain(other._box[d])]
        if not inside or inside[0] != differing[-1]:
            return -1
        return inside[0]

    def get_sub_range_slices(self, sub_range: "ParamRange") -> Tuple[slice, ...]:
        """Index tuple selecting ``sub_range`` out of a tensor holding this
        normalized box: whole slices except along the one differing dimension."""
        if not self.is_normalized or not isinstance(sub_range, ParamRange):
            raise AssertionError("slices are taken from a normalized ParamRange by a ParamRange")
        index = [slice(None)] * self.dims
        if sub_range == self:
            return tuple(index)
        d = self.is_contain(sub_range)
        if d < 0:
            raise AssertionError(f"{sub_range} is not a sub-box of {self} along one dimension")
        index[d] = slice(sub_range._box[d].start, sub_range._box[d].end)
        return tuple(index)

    def __eq__(self, other) -> bool:
        if not isinstance(other, ParamRange):
            return NotImplemented
        return self._box == other._box

    def __hash__(self) -> int:
        return hash((len(self._box), self._box))

    def __str__(self) -> str:
        return "ParamRange(" + " x ".join(str(r) for r in self._box) + ")"

    __repr__ = __str__
