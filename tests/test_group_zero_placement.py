"""Known answers for where a Group-ZeRO switch puts each optimizer shard, written out by hand.

Megatron builds the distributed-optimizer instances from the data-parallel
(with context) rank list of a model-parallel position: an instance is a
contiguous block of that list, and the inter-instance group of partial-DP
rank j is every part-th entry starting at j.  The reference's scale-up
(elastic_megatron/transfer/transfer.py:343-388) lets the first rank of each
inter-instance group migrate its own old state (training_state.py:40-60) and
broadcast it to the others; a scale-down keeps the state of the ranks that
remain.  With one pipeline stage the tables below follow from that alone.

The product is checked on arenas whose every element holds a distinct value,
so the rank and the offset inside the rank's shard that each destination
element came from can be read back; the oracle is checked with every source
rank's tensors holding their rank id.
"""

import numpy as np
import pytest
import torch

from elasticmegatron_amd import ParallelStrategy as PS
from elasticmegatron_amd.resharding.lowering import lower_redundant_backup
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from oracle import model
from oracle import transfer as oracle1
from tests.helpers import execute_numpy, small_llama2, strat

# {destination global rank: source global rank whose shard it holds}
W6_TO_W12_G2 = {0: 0, 1: 1, 2: 2, 3: 3, 4: 4, 5: 5,          # instance 0: the masters keep their own
                6: 0, 7: 1, 8: 2, 9: 3, 10: 4, 11: 5}        # instance 1: broadcast from rank j
# TP 2: the DP list of TP rank t is [t, 2+t, ..., 10+t]; instances of 2 partial-DP ranks each,
# so global ranks 2j+t, 2j+t+4 and 2j+t+8 form one inter-instance group whose master 2j+t was
# (dp j, tp t) of the old world as well.
W4TP2_TO_W12TP2_G3 = {0: 0, 1: 1, 2: 2, 3: 3,
                      4: 0, 5: 1, 6: 2, 7: 3,
                      8: 0, 9: 1, 10: 2, 11: 3}
# Scale-down: ranks 0-5 keep their own instance-0 state; ranks 6-11 leave.
W12_G2_TO_W6 = {g: g for g in range(6)}

CASES = [
    ("w6_w12_g2", PS(6, 1, 1), PS(12, 1, 1, num_distributed_optimizer_instances=2), True, W6_TO_W12_G2),
    ("w4tp2_w12tp2_g3", PS(4, 2, 1), PS(12, 2, 1, num_distributed_optimizer_instances=3), True,
     W4TP2_TO_W12TP2_G3),
    ("w12_g2_w6", PS(12, 1, 1, num_distributed_optimizer_instances=2), PS(6, 1, 1), False, W12_G2_TO_W6),
]

# An extension past the reference: with PP 2 the first rank of a stage-1 inter-instance group
# (global rank 4 or 5 of W8) did not exist in the W4 world, so the reference's master has no state
# to migrate.  The planner reads the shard of the same stage and partial-DP rank instead:
# stage s, dp d of W8 (rank 4s+d) holds stage s, dp d mod 2 of W4 (rank 2s + d mod 2).
PP2_EXTENSION = ("w4pp2_w8pp2_g2_extension", PS(4, 1, 2), PS(8, 1, 2, num_distributed_optimizer_instances=2),
                 True, {0: 0, 1: 1, 2: 0, 3: 1, 4: 2, 5: 3, 6: 2, 7: 3})

TAG = 28  # arena k's elements hold (k << TAG) | element index


def _tagged_arenas(layout):
    n = layout.fp32_numel
    assert n < (1 << TAG)
    idx = np.arange(n, dtype=np.uint32)
    return [idx | np.uint32(k << TAG) for k in range(3)] + [np.zeros(layout.bf16_numel, np.uint16)]


@pytest.mark.parametrize("name,src,dst,up,table", CASES + [PP2_EXTENSION], ids=[c[0] for c in CASES + [PP2_EXTENSION]])
def test_product_places_each_shard(name, src, dst, up, table):
    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(src), space.layout(dst)
    assert sorted(table) == list(range(dst.world_size))
    a = _tagged_arenas(ls)
    b = [np.full(ld.fp32_numel, 0xFFFFFFFF, np.uint32) for _ in range(3)] + [np.zeros(ld.bf16_numel, np.uint16)]
    execute_numpy(lower_redundant_backup(ls, ld, up), a, b)
    covered = np.zeros(dst.world_size, dtype=np.int64)
    for gi in sorted(ld.place):
        for h in ld.fp32_holders(space.all_virtual_params[gi]):
            g, n = h.rank, h.hi - h.lo
            s = table[g]
            at = h.offset - ld.rank_base[g]            # offset inside destination rank g's shard
            want = np.arange(ls.rank_base[s] + at, ls.rank_base[s] + at + n, dtype=np.uint32)
            for k in range(3):
                assert np.array_equal(b[k][h.offset:h.offset + n], want | np.uint32(k << TAG)), (name, g, gi, k)
            covered[g] += n
    # Every destination rank holds a whole shard: as many stored elements as its source rank.
    stored = np.zeros(src.world_size, dtype=np.int64)
    for gi in sorted(ls.place):
        for h in ls.fp32_holders(space.all_virtual_params[gi]):
            stored[h.rank] += h.hi - h.lo
    assert covered.tolist() == [int(stored[table[g]]) for g in range(dst.world_size)]


@pytest.mark.parametrize("name,src,dst,up,table", CASES + [PP2_EXTENSION], ids=[c[0] for c in CASES + [PP2_EXTENSION]])
def test_oracle_places_each_shard(name, src, dst, up, table):
    spec = small_llama2()
    inv = model.inventory(spec)
    S, D = strat(src), strat(dst)
    world = oracle1.build_src_world(inv, spec, S, 1234)
    for infos in world.values():
        for g, info in infos.items():
            info.tensors = [torch.full_like(t, float(g * 10 + k)) for k, t in enumerate(info.tensors)]
    out = oracle1.redundant_backup(inv, spec, S, D, world, up)
    seen = set()
    for infos in out.values():
        for g, info in infos.items():
            seen.add(g)
            for k, t in enumerate(info.tensors):
                assert torch.all(t == float(table[g] * 10 + k)), (name, g, k)
    assert seen == set(table)
