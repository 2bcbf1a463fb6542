"""Megatron-core distributed-data-parallel buffer layout, restated.

The reference does not compute shard boundaries itself: it instantiates
Megatron-core's ``_ParamAndGradBuffer`` with mocked collectives and reads its
``param_index_map`` and ``bucket_indices``
(elastic_megatron/resharding/resharding_dp.py:155-257).  Megatron-core
(core_r0.11.0, megatron/core/distributed/param_and_grad_buffer.py) is not
vendored with the reference, so its layout rules are restated here:

1. Parameters are placed in reverse of the given order (backprop order).
2. With the distributed optimizer every parameter start is padded up to a
   multiple of 64 elements.
3. A bucket closes after the parameter whose end reaches ``bucket_size``
   elements past the bucket start (``bucket_size`` None: one bucket).  A
   parameter flagged ``shared_embedding`` gets a bucket of its own.
4. With the distributed optimizer each bucket end is padded up to a multiple
   of ``lcm(dp, 128)``; the next bucket starts there.
5. Bucket b is split into ``dp`` equal shards; DP rank r owns
   ``[start_b + r*s_b, start_b + (r+1)*s_b)`` with ``s_b = numel_b / dp``.

The rules cannot be checked against Megatron-core here; they are covered by
the invariants in the tests (shards tile buckets, every element has exactly
one owner, paddings and alignments as stated).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple


@dataclass
class Bucket:
    start: int
    end: int
    params: List[int]            # indices into the given parameter order, in placement order
    numel_unpadded: int

    @property
    def numel(self) -> int:
        return self.end - self.start


@dataclass
class BufferLayout:
    dp_size: int
    numel: int
    param_index_map: Dict[int, Tuple[int, int, int]]   # param -> (start, end, bucket id)
    buckets: List[Bucket]
    shard_prefix: List[int] = field(default_factory=list)  # per bucket: offset of its shard in a rank's flat shard

    def shard_size(self, bucket_id: int) -> int:
        return self.buckets[bucket_id].numel // self.dp_size

    @property
    def rank_shard_numel(self) -> int:
        """Elements of one DP rank's shard, over all buckets."""
        return self.numel // self.dp_size


def _pad(n: int, d: int) -> int:
    return -(-n // d) * d


def build_buffer_layout(numels: Sequence[int], dp_size: int, bucket_size: Optional[int],
                        shared_embedding: Optional[Sequence[bool]] = None,
                        use_distributed_optimizer: bool = True) -> BufferLayout:
    n = len(numels)
    shared = list(shared_embedding) if shared_embedding is not None else [False] * n
    end_div = math.lcm(dp_size, 128)

    def pad_end(i: int) -> int:
        return _pad(i, end_div) if use_distributed_optimizer else i

    def pad_start(i: int) -> int:
        return _pad(i, 64) if use_distributed_optimizer else i

    index_map: Dict[int, Tuple[int, int, int]] = {}
    buckets: List[Bucket] = []
    bucket_start = 0
    bucket_params: List[int] = []
    param_start = 0
    param_end = 0

    def close(end_unpadded: int) -> int:
        nonlocal bucket_start, bucket_params
        end = pad_end(end_unpadded)
        buckets.append(Bucket(bucket_start, end, bucket_params, end_unpadded - bucket_start))
        bucket_start = end
        bucket_params = []
        return end

    for i in reversed(range(n)):
        param_start = pad_start(param_start)
        own_bucket = shared[i] and use_distributed_optimizer
        if own_bucket:
            if param_start % dp_size != 0:
                param_start = pad_end(param_start)
            if bucket_params:
                close(param_start)
        param_end = param_start + int(numels[i])
        index_map[i] = (param_start, param_end, len(buckets))
        bucket_params.append(i)
        if (bucket_size is not None and param_end - bucket_start >= bucket_size) or own_bucket:
            param_start = close(param_end)
        else:
            param_start = param_end
    if bucket_params:
        close(param_end)

    numel = buckets[-1].end if buckets else 0
    if use_distributed_optimizer:
        assert numel % dp_size == 0
    layout = BufferLayout(dp_size=dp_size, numel=numel, param_index_map=index_map, buckets=buckets)
    acc = 0
    for b in range(len(buckets)):
        layout.shard_prefix.append(acc)
        acc += layout.shard_size(b)
    return layout


def dp_distribution(layout: BufferLayout) -> Dict[int, Dict[int, Tuple[int, int]]]:
    """param -> {dp_rank: (lo, hi) in param-local flat coordinates}, dp ranks ascending.

    Follows resharding_dp.py:262-315 and :389-409 (every DP rank must own at
    least one piece of the buffer).
    """
    dp = layout.dp_size
    per_param: Dict[int, Dict[int, Tuple[int, int]]] = {p: {} for p in layout.param_index_map}
    owns = [False] * dp
    for bid, b in enumerate(layout.buckets):
        s = layout.shard_size(bid)
        for p in b.params:
            ps, pe, _ = layout.param_index_map[p]
            if ps < b.start:
                # A shared-embedding parameter placed in the padding its predecessor bucket claimed
                # (its start is 64-aligned but the closed bucket's end was padded past it): its first
                # elements would belong to no shard.  The reference stops here too, when it makes the
                # parameter's range relative to its bucket (resharding_dp.py:276-278, Range.normalize).
                raise AssertionError(f"parameter {p} starts at {ps}, before its bucket at {b.start}")
            for r in range(dp):
                lo = max(ps, b.start + r * s)
                hi = min(pe, b.start + (r + 1) * s)
                if lo < hi:
                    per_param[p][r] = (lo - ps, hi - ps)
                    owns[r] = True
    if layout.param_index_map and not all(owns):
        raise AssertionError("a data-parallel rank owns no parameter piece (resharding_dp.py:397)")
    return {p: dict(sorted(d.items())) for p, d in per_param.items()}


def piece_offset_in_rank_shard(layout: BufferLayout, param: int, dp_rank: int, lo: int) -> int:
    """Offset, in a DP rank's flat shard of this buffer, of param-local element ``lo``."""
    ps, _, bid = layout.param_index_map[param]
    b = layout.buckets[bid]
    s = layout.shard_size(bid)
    pos = ps + lo - (b.start + dp_rank * s)
    assert 0 <= pos < s, "element is not in this rank's shard"
    return layout.shard_prefix[bid] + pos
