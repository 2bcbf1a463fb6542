"""A switch run directly on Megatron-shaped flat buffers (the buffer adapter).

The caller holds, per model-parallel shard, the flat bf16 ``param_data`` of
each (stage, dense or expert) DDP buffer with Megatron's padding in place,
and per rank the flat fp32 DP shards of main / exp_avg / exp_avg_sq
(elastic_megatron/resharding/resharding_dp.py:224-315 computes the same
bucket and shard views over a real buffer).  :class:`MegatronBuffers` hands
out the per-parameter views of those buffers that a per-tensor plan reads
and writes.  The result must equal Oracle-1 bit for bit, and every padding
element of the source and destination buffers must keep its canary.
"""

import numpy as np
import pytest
import torch

from elasticmegatron_amd import ParallelStrategy as PS
from elasticmegatron_amd.megatron_manager.training_state import TrainingState
from elasticmegatron_amd.resharding.megatron_buffers import MegatronBuffers
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.transfer import TransferManager
from oracle import model
from oracle import transfer as oracle1
from tests.helpers import (CANARY16, CANARY32, SEED, compare, small_llama2, small_llama3, small_mixtral,
                           small_ragged, strat)

pytestmark = pytest.mark.gpu

CASES = [
    pytest.param(small_llama2, PS(8, 1, 1), PS(8, 4, 1), id="llama2-tp1dp8-tp4dp2"),
    pytest.param(small_llama3, PS(8, 2, 2), PS(8, 4, 1), id="llama3-tp2pp2dp2-tp4pp1dp2"),
    pytest.param(small_mixtral, PS(8, 1, 1, expert_model_parallel_size=4),
                 PS(8, 1, 1, expert_model_parallel_size=8), id="mixtral-ep4-ep8"),
    pytest.param(small_ragged, PS(8, 2, 1), PS(6, 1, 1), id="ragged-tp2dp4-dp6"),
]


def _canary(buffers):
    for t in buffers.values():
        (t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)).fill_(
            CANARY16 if t.dtype == torch.bfloat16 else CANARY32)


def _padding_damage(buffers, views, keys_of_views):
    """Elements of the flat buffers outside every view that lost their canary."""
    covered = {k: torch.zeros(t.numel(), dtype=torch.bool, device=t.device) for k, t in buffers.items()}
    for v, k in zip(views, keys_of_views):
        off = v.storage_offset() - buffers[k].storage_offset()
        covered[k][off:off + v.numel()] = True
    bad = 0
    for k, t in buffers.items():
        bits = t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)
        canary = CANARY16 if t.dtype == torch.bfloat16 else CANARY32
        bad += int(torch.count_nonzero(~covered[k] & (bits != canary)))
    return bad


@pytest.mark.parametrize("factory,src,dst", CASES)
def test_switch_on_megatron_flat_buffers(gpu_device, factory, src, dst):
    spec = factory()
    print(f"case megatron buffers {spec.name}: {src} -> {dst}", flush=True)
    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    tm = TransferManager(check_disjoint=True)
    plan = tm.compile_tensors(ls, ld)
    ms_, md = MegatronBuffers(ls), MegatronBuffers(ld)
    sbuf, dbuf = ms_.allocate(gpu_device), md.allocate(gpu_device)
    _canary(sbuf)
    _canary(dbuf)
    src_views = ms_.tensor_views(plan.src, sbuf)
    dst_views = md.tensor_views(plan.dst, dbuf)
    # The job's state: the seeded values, written into the source buffers' pieces.
    a = TrainingState.allocate(ls, gpu_device)
    a.fill_synthetic(SEED)
    for v, w in zip(src_views, plan.src.views(a)):
        v.copy_(w)
    del a
    tm.execute_tensors(plan, src_views, dst_views)
    torch.cuda.synchronize()

    skeys = [ms_.locate(ar, o, n)[0] for ar, o, n in zip(plan.src.arena, plan.src.offset, plan.src.numel)]
    dkeys = [md.locate(ar, o, n)[0] for ar, o, n in zip(plan.dst.arena, plan.dst.offset, plan.dst.numel)]
    assert _padding_damage(dbuf, dst_views, dkeys) == 0
    assert _padding_damage(sbuf, src_views, skeys) == 0

    pid = {vp.name: vp.global_index for vp in space.all_virtual_params}
    got32, gotbf = {}, {}
    for key, v in zip(plan.dst.keys, dst_views):
        if key[0] == "param":
            gotbf[(key[1], pid[key[2]])] = v.view(torch.int16).cpu().numpy().view(np.uint16)
        else:
            got32.setdefault((key[1], pid[key[2]]), {})[key[0]] = v.cpu().numpy()
    inv = model.inventory(spec)
    world = oracle1.build_src_world(inv, spec, strat(src), SEED)
    dw, dbf, _ = oracle1.transfer(inv, spec, strat(src), strat(dst), world)
    assert compare(got32, gotbf, oracle1.flatten(dw), dbf) == []


def _gap_damage(buffers, views, keys_of_views):
    """Padding elements (outside every view) that lost their canary, read gap by gap."""
    runs = {}
    for v, k in zip(views, keys_of_views):
        off = v.storage_offset() - buffers[k].storage_offset()
        runs.setdefault(k, []).append((off, off + v.numel()))
    bad = 0
    for k, t in buffers.items():
        bits = t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)
        canary = CANARY16 if t.dtype == torch.bfloat16 else CANARY32
        at = 0
        for a, b in sorted(runs.get(k, [])) + [(t.numel(), t.numel())]:
            if a > at:
                bad += int(torch.count_nonzero(bits[at:a] != canary))
            at = max(at, b)
    return bad


@pytest.mark.parametrize("src,dst", [pytest.param(PS(8, 1, 1), PS(8, 4, 1), id="llama2-7b-tp1dp8-tp4dp2"),
                                     pytest.param(PS(8, 1, 1), PS(6, 1, 1), id="llama2-7b-dp8-dp6")])
def test_full_size_switch_on_megatron_buffers(gpu_device, src, dst):
    """Llama-2-7B switched directly on Megatron-shaped buffers: each buffer its own allocation, the
    source filled with the seeded values through the remapped pieces, every stored destination
    element checked against the generator on the device, every padding element's canary kept."""
    from elasticmegatron_amd import _native
    from elasticmegatron_amd.resharding import model_spec as ms

    print(f"case megatron buffers full size {src} -> {dst}", flush=True)
    space = build_virtual_model(ms.llama2_7b())
    ls, ld = space.layout(src), space.layout(dst)
    tm = TransferManager()
    plan = tm.compile_tensors(ls, ld)
    ms_, md = MegatronBuffers(ls), MegatronBuffers(ld)
    try:
        sbuf, dbuf = ms_.allocate(gpu_device), md.allocate(gpu_device)
        _canary(dbuf)
        st = torch.cuda.current_stream().cuda_stream
        _native.synth_fill(ms_.remap_pieces(ls.pieces()), [sbuf[k].data_ptr() for k in ms_.keys()],
                           ms_.byte_sizes(), SEED, st)
        src_views, dst_views = ms_.tensor_views(plan.src, sbuf), md.tensor_views(plan.dst, dbuf)
        tm.execute_tensors(plan, src_views, dst_views)
        bad, first = _native.synth_verify(md.remap_pieces(ld.pieces()), [dbuf[k].data_ptr() for k in md.keys()],
                                          md.byte_sizes(), SEED, st)
        assert bad == 0, first
        dkeys = [md.locate(ar, o, n)[0] for ar, o, n in zip(plan.dst.arena, plan.dst.offset, plan.dst.numel)]
        assert _gap_damage(dbuf, dst_views, dkeys) == 0
    finally:
        sbuf = dbuf = src_views = dst_views = None  # noqa: F841
        torch.cuda.empty_cache()


@pytest.mark.parametrize("factory,src,dst", CASES[:3])
def test_each_rank_writes_its_share_into_its_own_buffers(gpu_device, factory, src, dst):
    """With one rank per GPU each rank holds only its own flat buffers (MegatronBuffers.rank_keys: its
    fp32 DP shards and its model shard's param_data).  Each destination rank's share
    (compile_share_tensors) runs with views of those buffers as its only destination tensors, the
    job's source buffers as sources.  Rank g's fp32 buffers then equal the whole switch's, padding
    included (the canary), and every bf16 element it writes equals the whole switch's."""
    spec = factory()
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
    for g in range(dst.world_size):
        print(f"case rank {g}'s share into its own buffers, {spec.name}: {src} -> {dst}", flush=True)
        plan = tm.compile_share_tensors(ls, ld, g)
        own = {k: torch.empty_like(whole[k]) for k in md.rank_keys(g)}
        _canary(own)
        dst_views = md.tensor_views(plan.dst, own, partial=True)
        assert all(dst_views[i] is not None for i in plan.dst_refs)
        tm.execute_tensors(plan, ms_.tensor_views(plan.src, sbuf), dst_views)
        torch.cuda.synchronize()
        for k, t in own.items():
            if k[0] == "param":
                bits, want = t.view(torch.int16), whole[k].view(torch.int16)
                written = bits != CANARY16
                assert bool(written.any()) and torch.equal(bits[written], want[written])
            else:
                assert torch.equal(t.view(torch.int32), whole[k].view(torch.int32)), k
