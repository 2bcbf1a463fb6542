"""GPU: seeded random medium-size switches run on Megatron-shaped flat buffers.

Per model shard the flat bf16 ``param_data`` of each (stage, dense or expert)
DDP buffer, per rank the flat fp32 DP shards, padding in place and filled
with canaries; the per-tensor plan runs on the views :class:`MegatronBuffers`
hands out (thousands a side, through the pointer table).  Every destination
element must hold the generator's value, and no padding element of either
side may lose its canary.
"""

import numpy as np
import pytest
import torch

from elasticmegatron_amd.megatron_manager.training_state import TrainingState
from elasticmegatron_amd.resharding.megatron_buffers import MegatronBuffers
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.transfer import TransferManager
from tests.helpers import SEED
from tests.test_gpu_megatron_buffers import _canary, _gap_damage
from tests.test_gpu_random_medium import _medium_spec
from tests.test_random_switches import _random_strategy

pytestmark = pytest.mark.gpu


def _cases(n=8):
    out = []
    for k in range(6000, 6000 + n):
        rng = np.random.default_rng(k)
        spec = _medium_spec(rng, k)
        a, b = _random_strategy(rng, spec), _random_strategy(rng, spec)
        out.append(pytest.param(spec, a, b, id=f"{k}-{'moe' if spec.num_experts else 'dense'}-"
                                f"tp{a.tensor_model_parallel_size}pp{a.pipeline_model_parallel_size}w{a.world_size}-"
                                f"tp{b.tensor_model_parallel_size}pp{b.pipeline_model_parallel_size}w{b.world_size}"))
    return out


@pytest.mark.parametrize("spec,src,dst", _cases())
def test_random_switch_on_megatron_flat_buffers(gpu_device, spec, src, dst):
    space = build_virtual_model(spec)
    space.register_reshard(src, dst)
    ls, ld = space.layout(src), space.layout(dst)
    tm = TransferManager(check_disjoint=True)
    plan = tm.compile_tensors(ls, ld)
    print(f"case {spec.name} {spec.num_params()} params: {src} -> {dst}, {len(plan.src)} + {len(plan.dst)} tensors",
          flush=True)
    ms_, md = MegatronBuffers(ls), MegatronBuffers(ld)
    sbuf, dbuf = ms_.allocate(gpu_device), md.allocate(gpu_device)
    _canary(sbuf)
    _canary(dbuf)
    src_views, dst_views = ms_.tensor_views(plan.src, sbuf), md.tensor_views(plan.dst, dbuf)
    a = TrainingState.allocate(ls, gpu_device)
    a.fill_synthetic(SEED)
    for v, w in zip(src_views, plan.src.views(a)):
        v.copy_(w)
    del a
    tm.execute_tensors(plan, src_views, dst_views)
    torch.cuda.synchronize()
    skeys = [ms_.locate(ar, o, n)[0] for ar, o, n in zip(plan.src.arena, plan.src.offset, plan.src.numel)]
    dkeys = [md.locate(ar, o, n)[0] for ar, o, n in zip(plan.dst.arena, plan.dst.offset, plan.dst.numel)]
    assert _gap_damage(dbuf, dst_views, dkeys) == 0
    assert _gap_damage(sbuf, src_views, skeys) == 0
    b = TrainingState.allocate(ld, gpu_device)
    for v, w in zip(dst_views, plan.dst.views(b)):
        w.copy_(v)
    bad, first = b.verify_synthetic(SEED)
    assert bad == 0, first


@pytest.mark.parametrize("spec,src,dst", _cases(12)[8:])
def test_random_rank_shares_into_their_own_buffers(gpu_device, spec, src, dst):
    """Every destination rank's share of a random switch, run with views of that rank's own flat
    buffers as its only destination tensors: its fp32 buffers, padding included, equal the whole
    switch's, and every bf16 element it writes equals the whole switch's."""
    from tests.helpers import CANARY16

    space = build_virtual_model(spec)
    space.register_reshard(src, dst)
    ls, ld = space.layout(src), space.layout(dst)
    tm = TransferManager(check_disjoint=True)
    ms_, md = MegatronBuffers(ls), MegatronBuffers(ld)
    sbuf, whole = ms_.allocate(gpu_device), md.allocate(gpu_device)
    _canary(sbuf)
    _canary(whole)
    full = tm.compile_tensors(ls, ld)
    a = TrainingState.allocate(ls, gpu_device)
    a.fill_synthetic(SEED)
    for v, w in zip(ms_.tensor_views(full.src, sbuf), full.src.views(a)):
        v.copy_(w)
    del a
    tm.execute_tensors(full, ms_.tensor_views(full.src, sbuf), md.tensor_views(full.dst, whole))
    print(f"case {spec.name} {spec.num_params()} params: every rank's share, {src} -> {dst}", flush=True)
    for g in range(dst.world_size):
        plan = tm.compile_share_tensors(ls, ld, g)
        own = {k: torch.empty_like(whole[k]) for k in md.rank_keys(g)}
        _canary(own)
        dst_views = md.tensor_views(plan.dst, own, partial=True)
        tm.execute_tensors(plan, ms_.tensor_views(plan.src, sbuf), dst_views)
        torch.cuda.synchronize()
        for k, t in own.items():
            if k[0] == "param":
                bits, want = t.view(torch.int16), whole[k].view(torch.int16)
                written = bits != CANARY16
                assert torch.equal(bits[written], want[written]), (g, k)
            else:
                assert torch.equal(t.view(torch.int32), whole[k].view(torch.int32)), (g, k)
