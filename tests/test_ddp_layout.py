"""Megatron DDP buffer layout (restated; the reference reads it from a mocked
Megatron-core _ParamAndGradBuffer, resharding_dp.py:155-315).

Megatron-core is not available, so parity with it is unpinned; these tests
pin the restated rules: hand-derived layouts, invariants on random inputs,
and the product and oracle restatements against each other.
"""

import math

import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from elasticmegatron_amd.resharding.ddp_layout import build_buffer_layout, dp_distribution
from oracle import megatron_buffer


def test_hand_derived_single_bucket():
    # Placed last-to-first: p2 [0,70), p1 at pad64(70)=128 -> [128,178), p0 at 192 -> [192,292);
    # bucket end pad(292, lcm(2,128)=128) = 384; shards of 192 elements.
    lay = build_buffer_layout([100, 50, 70], dp_size=2, bucket_size=None)
    assert lay.param_index_map == {2: (0, 70, 0), 1: (128, 178, 0), 0: (192, 292, 0)}
    assert [(b.start, b.end, b.params) for b in lay.buckets] == [(0, 384, [2, 1, 0])]
    assert dp_distribution(lay) == {0: {1: (0, 100)}, 1: {0: (0, 50)}, 2: {0: (0, 70)}}


def test_hand_derived_two_buckets():
    # bucket_size 100: p2 [0,70) stays open, p1 [128,178) closes bucket 0 at pad(178,128)=256,
    # p0 [256,356) closes bucket 1 at 384.  Shards: 128 and 64 elements.
    lay = build_buffer_layout([100, 50, 70], dp_size=2, bucket_size=100)
    assert [(b.start, b.end, b.params) for b in lay.buckets] == [(0, 256, [2, 1]), (256, 384, [0])]
    assert dp_distribution(lay) == {2: {0: (0, 70)}, 1: {1: (0, 50)}, 0: {0: (0, 64), 1: (64, 100)}}
    assert lay.shard_prefix == [0, 128] and lay.rank_shard_numel == 192


def test_dp6_pads_to_lcm_384():
    lay = build_buffer_layout([1000], dp_size=6, bucket_size=None)
    assert lay.numel == 1152 and lay.numel % math.lcm(6, 128) == 0
    d = dp_distribution(lay)[0]
    assert d == {0: (0, 192), 1: (192, 384), 2: (384, 576), 3: (576, 768), 4: (768, 960), 5: (960, 1000)}


def test_rank_without_piece_is_rejected():
    lay = build_buffer_layout([10], dp_size=8, bucket_size=None)  # 128 elements, 16 per rank
    with pytest.raises(AssertionError):
        dp_distribution(lay)


@given(st.lists(st.integers(1, 5000), min_size=1, max_size=30),
       st.sampled_from([1, 2, 4, 6, 8, 12]), st.sampled_from([None, 100, 1000, 7777]))
@settings(max_examples=150, deadline=None)
def test_invariants_and_restatements_agree(numels, dp, bucket):
    lay = build_buffer_layout(numels, dp, bucket)
    q = math.lcm(dp, 128)
    # Product and oracle restatements agree.
    ranges, buckets = megatron_buffer.layout(numels, dp, bucket)
    assert {i: (s, e) for i, (s, e, _) in lay.param_index_map.items()} == ranges
    assert [(b.start, b.end, b.params) for b in lay.buckets] == buckets
    # Reverse placement, 64-element starts, contiguous lcm-padded buckets.
    starts = [lay.param_index_map[i][0] for i in reversed(range(len(numels)))]
    assert starts == sorted(starts) and all(s % 64 == 0 for s in starts)
    prev = 0
    for bi, b in enumerate(lay.buckets):
        assert b.start == prev and b.end % q == 0 and b.end > b.start
        prev = b.end
        last = b.params[-1]
        if bucket is not None and bi < len(lay.buckets) - 1:
            assert lay.param_index_map[last][1] - b.start >= bucket
        for i in b.params:
            s, e, bid = lay.param_index_map[i]
            assert bid == bi and b.start <= s and e <= b.end
    # Every element has exactly one owner (unless a rank would own nothing).
    try:
        dist = dp_distribution(lay)
    except AssertionError:
        return
    assert dist == megatron_buffer.distribution(numels, dp, bucket)
    for i, n in enumerate(numels):
        pieces = sorted(dist[i].values())
        assert pieces[0][0] == 0 and pieces[-1][1] == n
        assert all(a[1] == b[0] for a, b in zip(pieces, pieces[1:]))
