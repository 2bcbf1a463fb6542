"""GPU: staged switches (ElasticMegatronManager(low_memory=True)).

Each optimizer kind moves in its own launch; its destination arena is
allocated just before and its source arena released right after, as the
reference releases every optimizer tensor once it is sent
(transfer.py:182-228, resharding_metadata.py:58-65).  The result must equal
the seeded generator's values everywhere, each stage is verified on the
device before its source goes, and a Llama-2-13B switch (182 GB per state,
364 GB for both) must run within one GPU's HBM.
"""

import gc

import pytest
import torch

from elasticmegatron_amd import ElasticMegatronManager
from elasticmegatron_amd import ParallelStrategy as PS
from elasticmegatron_amd.resharding import model_spec as ms
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from tests.helpers import SEED, small_llama2, small_llama3

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("factory,seq", [
    (small_llama2, [PS(8, 1, 1), PS(8, 4, 1), PS(8, 2, 2)]),
    (small_llama3, [PS(8, 2, 2), PS(8, 4, 1)]),
    (small_llama2, [PS(6, 1, 1), PS(12, 1, 1, num_distributed_optimizer_instances=2)]),
], ids=["llama2-tp1-tp4-tp2pp2", "llama3-tp2pp2-tp4", "groupzero-1-2"])
def test_staged_switch_matches_the_generator(gpu_device, factory, seq):
    mgr = ElasticMegatronManager(seq, factory(), device=gpu_device, low_memory=True)
    mgr.training_state.fill_synthetic(SEED)
    for s in seq[1:]:
        print(f"case staged {factory.__name__} -> {s}", flush=True)
        old = mgr.training_state
        new = mgr.reshard(s, verify=True)
        assert mgr.last_verification.bit_exact and mgr.last_verification.elements > 0
        assert all(t.numel() == 0 for t in (old.main, old.exp_avg, old.exp_avg_sq))   # released
        torch.cuda.synchronize()
        bad, first = new.verify_synthetic(SEED)
        assert bad == 0, first


def test_llama2_13b_switch_fits_in_one_gpu(gpu_device):
    """Llama-2-13B TP1DP8 -> TP4DP2: both whole states would need 364 GB; staged, the peak is the
    source state plus the destination's bf16 params and one fp32 arena (260 GB)."""
    gc.collect()                      # what earlier tests left behind
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    base = torch.cuda.memory_allocated(gpu_device)
    total = torch.cuda.get_device_properties(gpu_device).total_memory
    spec = ms.llama2_13b()
    src, dst = PS(8, 1, 1), PS(8, 4, 1)
    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    state = 3 * ls.fp32_numel * 4 + ls.bf16_numel * 2
    # Source state, destination bf16 params and one destination fp32 arena; each of the four fp32
    # arenas alive at once is rounded up to a 1 GiB granule.
    peak_bound = state + ld.bf16_numel * 2 + ld.fp32_numel * 4 + 4 * (1 << 30)
    both = state + 3 * ld.fp32_numel * 4 + ld.bf16_numel * 2
    print(f"case staged llama2-13b: state {state / 1e9:.1f} GB, bound {peak_bound / 1e9:.1f} GB, "
          f"device {total / 1e9:.1f} GB", flush=True)
    if peak_bound > 0.95 * total:
        pytest.skip("the device is too small even for the staged switch")
    del space, ls, ld
    mgr = ElasticMegatronManager([src, dst], spec, device=gpu_device, low_memory=True)
    assert both > total   # the unstaged switch cannot fit
    try:
        mgr.training_state.fill_synthetic(SEED)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(gpu_device)
        new = mgr.reshard(dst, verify=True)
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated(gpu_device) - base
        print(f"staged llama2-13b: executor {mgr.last_transfer_ms:.2f} ms over 3 stages "
              f"({mgr.last_stage_ms}), peak allocated {peak / 1e9:.1f} GB", flush=True)
        assert mgr.last_verification.bit_exact
        assert peak <= peak_bound
        bad, first = new.verify_synthetic(SEED)
        assert bad == 0, first
    finally:
        mgr = new = None  # noqa: F841
        gc.collect()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()


def _random_chains(n=6):
    import numpy as np

    from tests.test_gpu_random_medium import _medium_spec
    from tests.test_random_switches import _random_strategy

    out = []
    for k in range(7000, 7000 + n):
        rng = np.random.default_rng(k)
        spec = _medium_spec(rng, k)
        seq = [_random_strategy(rng, spec) for _ in range(3)]
        out.append(pytest.param(spec, seq, id=f"{k}-{'moe' if spec.num_experts else 'dense'}-" + "-".join(
            f"tp{s.tensor_model_parallel_size}pp{s.pipeline_model_parallel_size}w{s.world_size}" for s in seq)))
    return out


@pytest.mark.parametrize("spec,seq", _random_chains())
def test_random_staged_chain(gpu_device, spec, seq):
    """Seeded medium models (dense and MoE) through a chain of three random strategies, every switch
    staged and verified on the device stage by stage, each source arena released after its stage;
    the last state holds the generator's values."""
    mgr = ElasticMegatronManager(seq, spec, device=gpu_device, low_memory=True)
    mgr.training_state.fill_synthetic(SEED)
    for s in seq[1:]:
        print(f"case staged {spec.name} {spec.num_params()} params -> {s}", flush=True)
        mgr.reshard(s, verify=True)
        assert mgr.last_verification.bit_exact
    torch.cuda.synchronize()
    bad, first = mgr.training_state.verify_synthetic(SEED)
    assert bad == 0, first


@pytest.mark.parametrize("factory,seq", [
    (small_llama2, [PS(8, 1, 1), PS(8, 4, 1), PS(8, 2, 2)]),
    (small_llama2, [PS(6, 1, 1), PS(12, 1, 1, num_distributed_optimizer_instances=2), PS(6, 1, 1)]),
], ids=["llama2-tp1-tp4-tp2pp2", "groupzero-1-2-1"])
def test_staged_switch_between_shared_states(gpu_device, factory, seq):
    """low_memory with share_granule_bytes: each destination arena's granules are allocated just
    before its stage and each source arena's released right after it, so no more than one
    destination fp32 arena (and the destination's bf16 params when they are new) sits beside the
    source at any time; every switch verified, the last state against the generator."""
    from elasticmegatron_amd.transfer.ipc_manager import SharedTrainingState

    g = 1 << 20
    mgr = ElasticMegatronManager(seq, factory(), device=gpu_device, low_memory=True, share_granule_bytes=g)
    mgr.training_state.fill_synthetic(SEED)
    for s in seq[1:]:
        old = mgr.training_state
        print(f"case staged shared {factory.__name__} -> {s}", flush=True)
        torch.cuda.synchronize()
        gc.collect()
        base = torch.cuda.memory_allocated(gpu_device)
        torch.cuda.reset_peak_memory_stats(gpu_device)
        new = mgr.reshard(s, verify=True)
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated(gpu_device)
        assert isinstance(new, SharedTrainingState) and mgr.last_verification.bit_exact
        assert all(old.buffer_bytes()[b] == 0 for a in range(3) for b in old.buffers.granules_of(a))
        shared = new.tensors[new.buffers.granules_of(3)[0]] is old.tensors[old.buffers.granules_of(3)[0]]
        bound = new.layout.fp32_numel * 4 + (0 if shared else new.layout.bf16_numel * 2) + (64 << 20)
        assert peak - base <= bound, (peak - base, bound)
    bad, first = mgr.training_state.verify_synthetic(SEED)
    assert bad == 0, first


def test_failed_stage_stops_before_its_source_is_released(gpu_device, monkeypatch):
    """A mismatch found in stage 1 (exp_avg) raises before that stage's source arena is released:
    the old state keeps exp_avg and exp_avg_sq, having released main after stage 0 passed."""
    spec = small_llama2()
    src, dst = PS(8, 1, 1), PS(8, 4, 1)
    mgr = ElasticMegatronManager([src, dst], spec, device=gpu_device, low_memory=True)
    old = mgr.training_state
    old.fill_synthetic(SEED)
    real, calls = mgr.transfer_manager.execute_states, []

    def corrupting(plan, s, d, stream=None):
        real(plan, s, d, stream)
        calls.append(plan)
        if len(calls) == 2:                      # stage 1 writes exp_avg
            d.exp_avg.view(torch.int32)[d.layout.rank_fp32_slice(0)[0]] ^= 1

    monkeypatch.setattr(mgr.transfer_manager, "execute_states", corrupting)
    print("case staged switch with a planted mismatch in stage 1", flush=True)
    with pytest.raises(RuntimeError, match="stage 1"):
        mgr.reshard(dst, verify=True)
    assert mgr.training_state is old
    assert old.main.numel() == 0 and old.exp_avg.numel() > 0 and old.exp_avg_sq.numel() > 0
    bad, first = old.verify_synthetic(SEED, params=None, bf16=True, fp32=False)
    assert bad == 0, first
