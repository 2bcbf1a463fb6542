"""On-device verification of a reshard, per parameter and tensor kind.

The reference checks a reshard offline: it saves checkpoints before and
after, converts the first to the new layout with Megatron's converter on the
CPU, and diffs the resharded checkpoint (A) against the converted one (B) per
tensor with max |A - B|, max |A - B| / (|B| + 1e-12), RMS and RMS relative
to B's, against a threshold (tools/ckpt/compare_ckpt.py:17-76,
tools/ckpt/convert_and_compare.sh:53-69).  Here A is the destination state
and B what the plan says it must hold.  Differences are computed in fp32
(bf16 values are widened first); the reference subtracts in the tensors' own
dtype.

The plan itself says which source element every destination element must
equal, so the check runs on the device right after the switch, needs no
conversion and no copy, and adds an exact bit comparison: a reshard is
correct when every mismatch count is 0.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, List, NamedTuple, Optional, Tuple

import numpy as np

KIND_NAMES = ("param", "main", "exp_avg", "exp_avg_sq")


class TensorDiff(NamedTuple):
    """One (parameter, kind)'s comparison, with compare_ckpt.py's figures (compare_ckpt.py:52-66).

    An immutable tuple: a report holds one per (parameter, kind), hundreds per switch, and a tuple
    is built about three times faster than a frozen dataclass."""

    elements: int
    mismatches: int
    nonfinite: int
    sum_sq_diff: float
    sum_sq_expected: float
    max_abs: float
    max_rel: float

    @property
    def rms(self) -> float:
        return math.sqrt(self.sum_sq_diff / self.elements) if self.elements else 0.0

    @property
    def rel_rms(self) -> float:
        if not self.elements:
            return 0.0
        return self.rms / (math.sqrt(self.sum_sq_expected / self.elements) + 1e-12)


@dataclass
class VerifyReport:
    """Per (parameter name, kind): how the destination differs from the source it was resharded from."""

    tensors: Dict[Tuple[str, str], TensorDiff]

    @property
    def elements(self) -> int:
        return sum(t.elements for t in self.tensors.values())

    @property
    def mismatches(self) -> int:
        return sum(t.mismatches for t in self.tensors.values())

    @property
    def bit_exact(self) -> bool:
        return self.mismatches == 0

    def mismatched(self, rel_rms_thresh: Optional[float] = None) -> List[Tuple[str, str]]:
        """Keys that differ: any bit, or (with a threshold) relative RMS above it, as compare_ckpt judges."""
        if rel_rms_thresh is None:
            return [k for k, t in self.tensors.items() if t.mismatches]
        return [k for k, t in self.tensors.items() if t.nonfinite or t.rel_rms > rel_rms_thresh]

    def lines(self, rel_rms_thresh: Optional[float] = None) -> List[str]:
        """compare_ckpt.py's mismatch lines (compare_ckpt.py:68-72), with the bit count added."""
        out = []
        for k in self.mismatched(rel_rms_thresh):
            t = self.tensors[k]
            out.append(f"Value mismatch for {k[0]} [{k[1]}]: max_abs={t.max_abs:.3e}, max_rel={t.max_rel:.3e}, "
                       f"rms={t.rms:.3e}, rel_rms={t.rel_rms:.3e}, bits differ in {t.mismatches} of {t.elements}"
                       + (f" ({t.nonfinite} non-finite)" if t.nonfinite else ""))
        return out


def merge_stats(a: Optional[np.ndarray], b: np.ndarray) -> np.ndarray:
    """emrs_plan_compare records of two disjoint parts of one destination, combined: counts and sums
    add, maxima take the larger."""
    if a is None:
        return b.copy()
    out = a.copy()
    for f in ("elements", "mismatches", "nonfinite", "sum_sq_diff", "sum_sq_expected"):
        out[f] = a[f] + b[f]
    for f in ("max_abs_diff", "max_rel_diff"):
        out[f] = np.maximum(a[f], b[f])
    return out


def report_from_stats(stats: np.ndarray, names: List[str]) -> VerifyReport:
    """Build the report from emrs_plan_compare records indexed by ``4 * parameter index + kind``."""
    # Whole columns to Python numbers at once: reading the fields record by record costs
    # milliseconds per report on a few hundred parameters.
    cols = [stats[f].tolist() for f in ("elements", "mismatches", "nonfinite", "sum_sq_diff", "sum_sq_expected",
                                        "max_abs_diff", "max_rel_diff")]
    tensors = {}
    for g, rec in enumerate(zip(*cols)):
        if rec[0]:
            tensors[(names[g // 4], KIND_NAMES[g % 4])] = TensorDiff(*rec)
    return VerifyReport(tensors)
