"""Group-ZeRO switches on the device against Oracle-1.

Oracle-1 restates the reference's redundant backup
(elastic_megatron/transfer/transfer.py:343-388; param_migrate,
elastic_megatron/megatron_manager/training_state.py:40-60): on a scale-up every
new optimizer instance receives instance 0's shard of the same partial-DP rank;
on a scale-down each kept rank keeps its own instance's shard.  The seeded
generator gives every instance the same values, which would hide a wrong
instance -> rank mapping, so each source rank's shard is first made distinct
(its low mantissa bits XORed with a rank-dependent tag), on the device and in
the oracle's world alike.  The destination's padding must keep its canary.
"""

import pytest
import torch

from elasticmegatron_amd.megatron_manager.training_state import TrainingState
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.transfer import TransferManager
from oracle import model
from oracle import transfer as oracle1
from tests.helpers import (CANARY16, SEED, compare, extract, fill_canaries, padding_damage, perturb_per_rank, small_llama2,
                           strat)
from tests.test_group_zero import CASES

pytestmark = pytest.mark.gpu


def _host_arenas(state):
    return [t.view(torch.int32).cpu().numpy().view("uint32") for t in (state.main, state.exp_avg, state.exp_avg_sq)] \
        + [state.param.view(torch.int16).cpu().numpy().view("uint16")]


@pytest.mark.parametrize("scale_up", [True, False], ids=["scale_up", "scale_down"])
@pytest.mark.parametrize("name,small,big", CASES, ids=[c[0] for c in CASES])
def test_redundant_backup_matches_oracle1(gpu_device, name, small, big, scale_up):
    src, dst = (small, big) if scale_up else (big, small)
    print(f"group-zero {name} {'up' if scale_up else 'down'}: {src} -> {dst}", flush=True)
    spec = small_llama2()
    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    a = TrainingState.allocate(ls, gpu_device)
    a.fill_synthetic(SEED)
    perturb_per_rank(a)
    b = TrainingState.allocate(ld, gpu_device)
    fill_canaries(b)
    tm = TransferManager()
    tm.redundant_backup(scale_up, a, b)
    torch.cuda.synchronize()

    inv = model.inventory(spec)
    world = oracle1.build_src_world(inv, spec, strat(src), SEED)
    perturb_per_rank(world)
    want = oracle1.flatten(oracle1.redundant_backup(inv, spec, strat(src), strat(dst), world, scale_up))
    got, _ = extract(ld, _host_arenas(b))
    assert compare(got, {}, want, {}) == []
    # The model-parallel shards do not change under Group ZeRO: the bf16 arena is not written at all.
    assert bool((b.param.view(torch.int16) == CANARY16).all())
    assert padding_damage(b) == 0


@pytest.mark.parametrize("group_src", [0, 1])
def test_scale_up_from_a_chosen_source_instance(gpu_device, group_src):
    """TransferManager.redundant_backup(is_scale_up, src, dst, group_src), the reference's broadcast
    root (transfer.py:343-371): from two instances to four, every new instance holds instance
    ``group_src``'s shard; each source rank's shard distinct, against Oracle-1."""
    from elasticmegatron_amd import ParallelStrategy as PS

    src, dst = PS(8, 1, 1, num_distributed_optimizer_instances=2), PS(16, 1, 1, num_distributed_optimizer_instances=4)
    print(f"group-zero scale-up from instance {group_src}: {src} -> {dst}", flush=True)
    spec = small_llama2()
    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    a = TrainingState.allocate(ls, gpu_device)
    a.fill_synthetic(SEED)
    perturb_per_rank(a)
    b = TrainingState.allocate(ld, gpu_device)
    fill_canaries(b)
    TransferManager().redundant_backup(True, a, b, group_src)
    torch.cuda.synchronize()
    inv = model.inventory(spec)
    world = oracle1.build_src_world(inv, spec, strat(src), SEED)
    perturb_per_rank(world)
    want = oracle1.flatten(oracle1.redundant_backup(inv, spec, strat(src), strat(dst), world, True,
                                                    group_src=group_src))
    got, _ = extract(ld, _host_arenas(b))
    assert compare(got, {}, want, {}) == []
    assert padding_damage(b) == 0
