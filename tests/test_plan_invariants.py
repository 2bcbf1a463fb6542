"""Plan invariants at full size (host-only: no GPU needed).

Every workload's plan covers each destination element exactly once, stays in
bounds, takes the 16-byte path throughout, and moves exactly the algorithmic
bytes: 12 read + 14 written per parameter (+ the per-TP-rank copies of the
parameters that are not TP-split).
"""

import pytest

from elasticmegatron_amd import _native
from elasticmegatron_amd import ParallelStrategy as PS
from elasticmegatron_amd.resharding import model_spec as ms
from elasticmegatron_amd.resharding.layout import SEG_DUP
from elasticmegatron_amd.resharding.lowering import lower_redundant_backup, lower_transfer, payload_bytes, read_bytes
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model

CASES = [
    (ms.llama2_7b, PS(8, 1, 1), PS(8, 4, 1)),
    (ms.llama3_8b, PS(8, 2, 2), PS(8, 4, 1)),
    (ms.mixtral_8x7b_slice, PS(8, 1, 1, expert_model_parallel_size=4), PS(8, 1, 1, expert_model_parallel_size=8)),
    (ms.llama2_7b, PS(8, 1, 1), PS(6, 1, 1)),
    (ms.tiny_llama2, PS(8, 2, 1), PS(8, 1, 1)),
    (ms.tiny_llama2, PS(8, 1, 1), PS(8, 4, 1)),
]


def _replicated_extra(space, src, dst):
    """Elements of non-TP-split params written once more per extra destination TP rank."""
    extra = 0
    for vp in space.all_virtual_params:
        if not vp.tensor_parallel_attr.tensor_model_parallel:
            extra += vp.numel() * (vp.tp_size_at(dst) - 1)
    return extra


@pytest.mark.parametrize("factory,src,dst", CASES, ids=lambda x: getattr(x, "__name__", None))
def test_full_size_plan_invariants(factory, src, dst):
    spec = factory()
    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    table = lower_transfer(ls, ld)
    n = spec.num_params() + _replicated_extra(space, src, dst)
    assert read_bytes(table) == 12 * n
    assert payload_bytes(table) == 14 * n
    plan = _native.Plan(table, [ls.fp32_numel * 4] * 3 + [ls.bf16_numel * 2],
                        [ld.fp32_numel * 4] * 3 + [ld.bf16_numel * 2], check_disjoint=True)
    st = plan.stats()
    assert st.scalar_bytes == 0 and st.vector_bytes == 12 * n
    assert st.payload_bytes == 14 * n and st.read_bytes == 12 * n


def test_group_zero_plan_invariants():
    spec = ms.llama2_7b()
    space = build_virtual_model(spec)
    a, b = PS(6, 1, 1), PS(12, 1, 1, num_distributed_optimizer_instances=2)
    up = lower_redundant_backup(space.layout(a), space.layout(b), True)
    down = lower_redundant_backup(space.layout(b), space.layout(a), False)
    n = spec.num_params()
    # Scale-up: every shard is read once and written to both instances by one duplicating segment.
    assert (up["flags"] == SEG_DUP).all()
    assert read_bytes(up) == 12 * n and payload_bytes(up) == 24 * n
    assert read_bytes(down) == payload_bytes(down) == 12 * n
    assert (down["flags"] == 0).all()
    for t, (x, y) in ((up, (a, b)), (down, (b, a))):
        lx, ly = space.layout(x), space.layout(y)
        st = _native.Plan(t, [lx.fp32_numel * 4] * 3 + [lx.bf16_numel * 2],
                          [ly.fp32_numel * 4] * 3 + [ly.bf16_numel * 2], check_disjoint=True).stats()
        assert st.scalar_bytes == 0
        assert st.read_bytes == read_bytes(t) and st.payload_bytes == payload_bytes(t)


@pytest.mark.parametrize("bf16_source", ["cast", "copy"])
def test_switch_to_the_same_strategy_is_the_identity(bf16_source):
    """reshard(S -> S) reproduces every stored element.  (It is the identity on values, not on offsets:
    parameters that are not TP-split are read from TP rank 0 for every TP rank, and a tied output layer
    from the word embedding, as the reference reads them.)"""
    import numpy as np

    from tests.helpers import SEED, SMALL_CASES, compare, execute_numpy, extract, new_arenas, piece_fill_numpy

    for _, factory, seq in SMALL_CASES:
        space = build_virtual_model(factory())
        for s in seq:
            lay = space.layout(s)
            t = lower_transfer(lay, lay, bf16_source=bf16_source)
            assert ((t["flags"] & 2) == 0).all()
            assert np.array_equal(t["src_buf"], t["dst_buf"])
            a = new_arenas(lay)
            piece_fill_numpy(lay.pieces(), a, SEED)
            b = new_arenas(lay, fill=0)
            execute_numpy(t, a, b)
            assert compare(*extract(lay, b), *extract(lay, a)) == []
