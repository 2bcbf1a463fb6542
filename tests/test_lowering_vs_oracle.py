"""The product's copy plan, executed on the CPU, against the oracles.

Oracle-1 restates the reference's three-pass executor
(elastic_megatron/transfer/transfer.py:36-341); Oracle-2 regenerates each
destination piece from its full-tensor indices.  Both must agree with each
other and with the product's lowering, bit for bit.
"""

import pytest

from elasticmegatron_amd.resharding.lowering import lower_transfer
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from oracle import canonical, model
from oracle import transfer as oracle1
from tests.helpers import SEED, SMALL_CASES, compare, execute_numpy, extract, new_arenas, piece_fill_numpy, strat


def _switches():
    for name, factory, seq in SMALL_CASES:
        for a, b in zip(seq, seq[1:]):
            yield pytest.param(factory, a, b, id=f"{name}-{a.tensor_model_parallel_size}x{a.pipeline_model_parallel_size}x{a.world_size}"
                               f"-{b.tensor_model_parallel_size}x{b.pipeline_model_parallel_size}x{b.world_size}")


@pytest.mark.parametrize("factory,src,dst", list(_switches()))
@pytest.mark.parametrize("bf16_source", ["cast", "copy"])
def test_plan_matches_oracles(factory, src, dst, bf16_source):
    spec = factory()
    inv = model.inventory(spec)
    S, D = strat(src), strat(dst)
    world = oracle1.build_src_world(inv, spec, S, SEED)
    dw, dbf, _ = oracle1.transfer(inv, spec, S, D, world)
    o1_32 = oracle1.flatten(dw)
    o2_32, o2_bf = canonical.world(inv, spec, D, SEED)
    assert compare(o1_32, dbf, o2_32, o2_bf) == []

    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    table = lower_transfer(ls, ld, bf16_source=bf16_source)
    a_src, a_dst = new_arenas(ls), new_arenas(ld)
    piece_fill_numpy(ls.pieces(), a_src, SEED)
    execute_numpy(table, a_src, a_dst)
    got32, gotbf = extract(ld, a_dst)
    assert compare(got32, gotbf, o1_32, dbf) == []
