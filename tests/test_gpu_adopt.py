"""GPU: Group-ZeRO switches whose new state takes over the old one's leading granules.

Between shared states (arenas held in granules) that this process owns, a
Group-ZeRO switch leaves instance 0 where it is: the new state holds the old
state's leading granules of every fp32 arena, the plan writes only the rest,
and the old state hands those granules over before it is released.  After the
old state is gone, and its freed memory has been handed out again and filled
with NaN, the new state must hold the generator's values: a granule freed
while still held, or one left unwritten, breaks that.  The plan's
verification, which reads the taken-over memory from both sides, must find no
difference.
"""

import numpy as np
import pytest
import torch

from elasticmegatron_amd import ElasticMegatronManager, ParallelStrategy as PS
from elasticmegatron_amd.resharding.granules import GranuleBuffers
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.ipc_manager import SharedTrainingState
from elasticmegatron_amd.transfer.transfer import TransferManager, adoptable_granules, backup_kind
from tests.helpers import SEED, small_llama2
from tests.test_gpu_random_medium import _medium_spec
from tests.test_random_switches import _random_strategy

pytestmark = pytest.mark.gpu


def _heads(state, n):
    ptrs = state.buffer_ptrs()
    return [ptrs[b] for a in range(3) for b in state.buffers.granules_of(a)[:n]]


def _reuse_freed(sizes, device):
    """Hand the caching allocator's freed granules out again, filled with NaN."""
    return [torch.full((n,), float("nan"), dtype=torch.float32, device=device) for n in sizes]


def test_manager_chain_takes_over_instance_0(gpu_device):
    g = 1 << 16
    seq = [PS(4, 1, 1), PS(8, 1, 1, num_distributed_optimizer_instances=2), PS(4, 1, 1),
           PS(12, 1, 1, num_distributed_optimizer_instances=3), PS(4, 1, 1), PS(4, 1, 2),
           PS(8, 1, 2, num_distributed_optimizer_instances=2), PS(4, 1, 2),
           PS(8, 2, 1, context_parallel_size=2),
           PS(16, 2, 1, context_parallel_size=2, num_distributed_optimizer_instances=2),
           PS(8, 2, 1, context_parallel_size=2), PS(8, 1, 1)]
    mgr = ElasticMegatronManager(seq, small_llama2(), device=gpu_device, share_granule_bytes=g)
    mgr.training_state.fill_synthetic(SEED)
    for s in seq[1:]:
        old = mgr.training_state
        backup = PS.is_redundant_backup(old.parallel_strategy, s)
        n = 0 if backup is None else adoptable_granules(old.layout, mgr.space_for(s).layout(s), g,
                                                        backup_kind(backup))
        print(f"case adopting chain -> {s}: {n} granules a fp32 arena taken over", flush=True)
        heads = _heads(old, n)
        freed = [old.buffers.numel[b] for a in range(3) for b in old.buffers.granules_of(a)[n:]]
        mgr.reshard(s, is_meta_device=True)
        new = mgr.reshard(s, verify=True)
        junk = _reuse_freed(freed, gpu_device)
        torch.cuda.synchronize()
        assert mgr.last_verification.bit_exact
        assert backup is None or n > 0
        assert _heads(new, n) == heads
        bad, first = new.verify_synthetic(SEED)
        assert bad == 0, first
        del junk


def _cases(n=10, seed0=5000):
    out = []
    for s in range(seed0, seed0 + 400):
        rng = np.random.default_rng(s)
        spec = _medium_spec(rng, s)
        if spec.num_experts:
            continue
        base = _random_strategy(rng, spec)
        k, cp, up = int(rng.choice([2, 3])), int(rng.choice([1, 2])), bool(rng.random() < 0.5)
        tp, pp = base.tensor_model_parallel_size, base.pipeline_model_parallel_size
        try:
            small = PS(base.world_size * cp, tp, pp, context_parallel_size=cp)
            big = PS(base.world_size * cp * k, tp, pp, context_parallel_size=cp,
                     num_distributed_optimizer_instances=k)
            for st in (small, big):
                st.validate_for(spec.num_layers, spec.num_experts)
        except (ValueError, AssertionError, RuntimeError):
            continue
        m = int(rng.integers(2, 60))
        out.append(pytest.param(spec, small, big, up, m, id=f"{s}-tp{tp}pp{pp}cp{cp}-{small.world_size}x1"
                                f"{'->' if up else '<-'}{big.world_size}x{k}-m{m}"))
        if len(out) == n:
            break
    return out


@pytest.mark.parametrize("spec,small,big,up,m", _cases())
def test_random_adopting_switch(gpu_device, spec, small, big, up, m):
    src, dst = (small, big) if up else (big, small)
    kind = backup_kind(up)
    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    # Granules that cut the smaller arena into about m, so the head ends inside a run.
    g = max(256, -(-min(ls.fp32_numel, ld.fp32_numel) * 4 // m // 256) * 256)
    n = adoptable_granules(ls, ld, g, kind)
    print(f"case {spec.name} {spec.num_params()} params: {src} -> {dst} ({kind}), granule {g} B, "
          f"{n} taken over", flush=True)
    assert n >= 1
    tm = TransferManager(check_disjoint=True)
    plan = tm.compile_granules(ls, ld, g, g, kind, adopt_granules=n)
    a = SharedTrainingState.allocate(ls, gpu_device, g)
    a.fill_synthetic(SEED)
    b = SharedTrainingState.allocate(ld, gpu_device, g, param_granules=[a.tensors[x] for x in a.buffers.granules_of(3)],
                                     adopted=a.leading_fp32_granules(n))
    for k in range(3):
        for x in b.buffers.granules_of(k)[n:]:
            b.tensors[x].fill_(float("nan"))
    tm.execute_states(plan, a, b)
    assert tm.verify(a, b, kind).bit_exact
    freed = [a.buffers.numel[x] for k in range(3) for x in a.buffers.granules_of(k)[n:]]
    a.hand_over(n)
    a.release_optimizer()
    del a
    junk = _reuse_freed(freed, gpu_device)
    torch.cuda.synchronize()
    bad, first = b.verify_synthetic(SEED)
    assert bad == 0, first
    del junk


def test_hand_off_of_a_state_holding_taken_over_granules(gpu_device):
    """The old process reached its strategy by a Group-ZeRO scale-up that took over instance 0, so
    the state it exports holds granules adopted from the state before.  Mapped in this process and
    switched back down (the bf16 params copied, since the exporter frees its memory), every element
    holds the generator's value."""
    from tests.test_gpu_ipc import _hand_off

    src, dst = PS(8, 1, 1, num_distributed_optimizer_instances=2), PS(4, 1, 1)
    print(f"case hand-off of a taken-over state: child {dst} -> {src}, then here -> {dst}", flush=True)
    mgr, new, n_granules, n_mapped = _hand_off(gpu_device, small_llama2(), src, dst, (1 << 20) + 256 * 3, 240,
                                               start_from=dst)
    print(f"  {n_granules} granules in {n_mapped} allocations", flush=True)
    bad, first = new.verify_synthetic(SEED)
    assert bad == 0, first


def test_failed_switch_leaves_the_old_state_whole(gpu_device, monkeypatch):
    """A switch whose verification fails raises, and the old state stays the live state with every
    granule it lent to the new one: nothing is handed over before the check passes.  The new
    state's own memory, freed with it, is handed out again and filled with NaN first; then the
    same switch runs clean."""
    import gc

    g = 1 << 16
    small, big = PS(4, 1, 1), PS(8, 1, 1, num_distributed_optimizer_instances=2)
    mgr = ElasticMegatronManager([small, big], small_llama2(), device=gpu_device, share_granule_bytes=g)
    old = mgr.training_state
    old.fill_synthetic(SEED)
    ld = mgr.space_for(big).layout(big)
    vp = next(v for v in ld.space.all_virtual_params if ld.has_param(v))
    h = next(x for x in ld.fp32_holders(vp) if x.instance == 1)
    real = mgr.transfer_manager.execute_states

    def corrupting(plan, src, dst, stream=None):
        real(plan, src, dst, stream)
        b, off = dst.buffers.locate(1, h.offset)     # an exp_avg element of instance 1: written, not taken over
        dst.tensors[b].view(torch.int32)[off] ^= 1

    monkeypatch.setattr(mgr.transfer_manager, "execute_states", corrupting)
    print("case failed switch with instance 0 lent to the new state", flush=True)
    with pytest.raises(RuntimeError, match="verification failed"):
        mgr.reshard(big, verify=True)
    assert mgr.training_state is old
    gc.collect()
    n, gb = adoptable_granules(old.layout, ld, g, "backup_up"), GranuleBuffers(ld, g)
    junk = _reuse_freed([gb.numel[b] for a in range(3) for b in gb.granules_of(a)[n:]], gpu_device)
    torch.cuda.synchronize()
    bad, first = old.verify_synthetic(SEED)
    assert bad == 0, first
    del junk
    monkeypatch.undo()
    new = mgr.reshard(big, verify=True)
    torch.cuda.synchronize()
    assert mgr.last_verification.bit_exact and new.verify_synthetic(SEED)[0] == 0
