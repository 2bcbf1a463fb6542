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


# Known answers for the branches above, each derived by hand from Megatron-core's published
# placement loop (param_and_grad_buffer.py, core_r0.11.0): reverse order, starts padded to 64,
# a bucket closes once param_end - bucket_start >= bucket_size, a shared-embedding parameter
# first pads its start to lcm(dp, 128) when it is not a multiple of dp, closes the open bucket
# at that start, and takes a bucket of its own; bucket ends padded to lcm(dp, 128).

def test_hand_derived_shared_embedding_padded_to_dp():
    # dp 6, lcm 384.  p1 (50) at [0, 50).  p0 (1000, shared): start pad64(50) = 64, and 64 % 6 != 0,
    # so it moves to 384; bucket 0 closes at 384.  p0 takes [384, 1384) and closes bucket 1 at
    # pad(1384, 384) = 1536.  Shards: bucket 0 of 64 elements, bucket 1 of 192.
    lay = build_buffer_layout([1000, 50], dp_size=6, bucket_size=None, shared_embedding=[True, False])
    assert lay.param_index_map == {1: (0, 50, 0), 0: (384, 1384, 1)}
    assert [(b.start, b.end, b.params) for b in lay.buckets] == [(0, 384, [1]), (384, 1536, [0])]
    assert dp_distribution(lay) == {
        1: {0: (0, 50)},
        0: {0: (0, 192), 1: (192, 384), 2: (384, 576), 3: (576, 768), 4: (768, 960), 5: (960, 1000)}}
    assert lay.shard_prefix == [0, 64] and lay.rank_shard_numel == 256
    ranges, buckets = megatron_buffer.layout([1000, 50], 6, None, shared=[True, False])
    assert ranges == {1: (0, 50), 0: (384, 1384)} and buckets == [(0, 384, [1]), (384, 1536, [0])]


def test_hand_derived_shared_embedding_placed_first():
    # The last parameter of the list (a tied output layer on the last stage) is placed first:
    # no open bucket to close.  p1 (1000, shared) [0, 1000) closes bucket 0 at 1024; p0 (50) at
    # [1024, 1074) is the last bucket, closed at 1152.  Shards of 512 and 64.
    lay = build_buffer_layout([50, 1000], dp_size=2, bucket_size=None, shared_embedding=[False, True])
    assert lay.param_index_map == {1: (0, 1000, 0), 0: (1024, 1074, 1)}
    assert [(b.start, b.end, b.params) for b in lay.buckets] == [(0, 1024, [1]), (1024, 1152, [0])]
    assert dp_distribution(lay) == {1: {0: (0, 512), 1: (512, 1000)}, 0: {0: (0, 50)}}


def test_shared_embedding_straddling_a_padded_bucket_end_is_refused():
    # p1 (150) at [0, 150); p0 (300, shared) starts at pad64(150) = 192, a multiple of dp 2, so it
    # stays there while the bucket it closes ends at pad(192, 128) = 256.  p0's first 64 elements
    # lie before its own bucket: the reference's Range.normalize assertion stops it, so must we.
    lay = build_buffer_layout([300, 150], dp_size=2, bucket_size=None, shared_embedding=[True, False])
    assert lay.param_index_map == {1: (0, 150, 0), 0: (192, 492, 1)}
    assert [(b.start, b.end) for b in lay.buckets] == [(0, 256), (256, 512)]
    with pytest.raises(AssertionError, match="before its bucket"):
        dp_distribution(lay)
    with pytest.raises(AssertionError):
        megatron_buffer.distribution([300, 150], 2, None, shared=[True, False])


def test_hand_derived_bucket_closes_at_exactly_bucket_size():
    # bucket_size 128: p2 (64) [0, 64) stays open; p1 (64) [64, 128) ends exactly 128 past the
    # bucket start, which closes it (>=); p0 (100) [128, 228) closes the last bucket at 256.
    # With a strict > the first bucket would have taken p0 as well.
    lay = build_buffer_layout([100, 64, 64], dp_size=2, bucket_size=128)
    assert lay.param_index_map == {2: (0, 64, 0), 1: (64, 128, 0), 0: (128, 228, 1)}
    assert [(b.start, b.end, b.params) for b in lay.buckets] == [(0, 128, [2, 1]), (128, 256, [0])]
    assert dp_distribution(lay) == {2: {0: (0, 64)}, 1: {1: (0, 64)}, 0: {0: (0, 64), 1: (64, 100)}}


def test_hand_derived_expert_buffer_at_edp2():
    """resharding_dp.py:354-375: the expert buffer is laid out for EP rank 0's experts over the
    expert-DP group and reused, in order, by every other EP rank."""
    from elasticmegatron_amd import ParallelStrategy as PS
    from elasticmegatron_amd.resharding import model_spec as ms
    from elasticmegatron_amd.resharding.virtual_param import build_virtual_model

    spec = ms.ModelSpec(name="tiny-moe", num_layers=1, hidden_size=64, num_attention_heads=2, ffn_hidden_size=128,
                        padded_vocab_size=256, num_experts=4, moe_ffn_hidden_size=96, ddp_bucket_size=10000,
                        overlap_grad_reduce=True)
    lay = build_virtual_model(spec).layout(PS(4, 1, 1, expert_model_parallel_size=2))
    assert lay.strategy.expert_data_parallel_size == 2
    # EP rank 0 holds experts 0 and 1: [fc1.w0, fc1.w1, fc2.w0, fc2.w1] with 2*96*64 = 12288 and
    # 64*96 = 6144 elements.  Reversed: fc2.w1 [0, 6144) leaves the bucket open (6144 < 10000);
    # fc2.w0 [6144, 12288) closes it at 12288 (a multiple of lcm(2, 128)); fc1.w1 [12288, 24576)
    # and fc1.w0 [24576, 36864) each close one.  Every bucket splits into shards of half its size.
    el = lay.stage_expert[0]
    assert el.param_index_map == {3: (0, 6144, 0), 2: (6144, 12288, 0), 1: (12288, 24576, 1),
                                  0: (24576, 36864, 2)}
    assert [(b.start, b.end, b.params) for b in el.buckets] == [(0, 12288, [3, 2]), (12288, 24576, [1]),
                                                                   (24576, 36864, [0])]
    want = {"fc2.weight1": {0: (0, 6144)}, "fc2.weight0": {1: (0, 6144)},
            "fc1.weight1": {0: (0, 6144), 1: (6144, 12288)}, "fc1.weight0": {0: (0, 6144), 1: (6144, 12288)}}
    space = lay.space
    for vp in space.all_virtual_params:
        if not vp.is_expert:
            continue
        local = vp.expert_id % 2        # EP rank 1's experts 2, 3 take the places of 0, 1
        short = vp.name.split("linear_")[1][:-1] + str(local)
        assert lay.dp_distribution(vp) == want[short], vp.name
        assert lay.place[vp.global_index].expert_ep == vp.expert_id // 2


def test_parameter_counts_of_the_workloads():
    """The four model shapes' parameter counts, from the product's model and the oracle's inventory."""
    from elasticmegatron_amd.resharding import model_spec as ms
    from oracle import model

    counts = {ms.tiny_llama2: 39_094_784, ms.llama2_7b: 6_738_415_616, ms.llama3_8b: 8_030_261_248,
              ms.mixtral_8x7b_slice: 6_067_228_672}
    for factory, n in counts.items():
        spec = factory()
        assert spec.num_params() == n, spec.name
        assert sum(model.numel(p["shape"]) for p in model.inventory(spec)) == n, spec.name
