"""The reference-style communication figure equals Oracle-1's message count."""

import pytest

from elasticmegatron_amd.resharding.comm_stats import reference_comm_bytes
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from oracle import model
from oracle import transfer as oracle1
from tests.helpers import SEED, SMALL_CASES, strat


@pytest.mark.parametrize("name,factory,seq", [c for c in SMALL_CASES if c[0] != "tiny_tp2dp4_tp1dp8_tp4dp2"])
def test_reference_comm_bytes_match_oracle(name, factory, seq):
    spec = factory()
    inv = model.inventory(spec)
    for a, b in zip(seq, seq[1:]):
        S, D = strat(a), strat(b)
        world = oracle1.build_src_world(inv, spec, S, SEED)
        _, _, mb = oracle1.transfer(inv, spec, S, D, world)
        got = reference_comm_bytes(build_virtual_model(spec), a, b)
        want = {g: v for g, v in mb.cross_rank_bytes.items() if v}
        assert {g: v for g, v in got.items() if v} == want
