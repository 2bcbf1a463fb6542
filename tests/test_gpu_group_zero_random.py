"""GPU: seeded random medium-size Group-ZeRO switches (optimizer instances 1 <-> 2 or 3, TP 1-4, CP 1-2).

Every fp32 element of the new state is checked against the generator's closed
form (its value depends only on parameter, kind and full-tensor index, so an
instance placed on the wrong rank reads wrong), and the plan's own
verification must find no difference.  PP 1 only: with PP > 1 the instance rule
is an extension past the reference, pinned elsewhere.
"""

import numpy as np
import pytest
import torch

from elasticmegatron_amd import ParallelStrategy as PS
from elasticmegatron_amd.megatron_manager.training_state import TrainingState
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.transfer import TransferManager
from tests.helpers import SEED
from tests.test_gpu_random_medium import _medium_spec
from tests.test_random_switches import _random_strategy

pytestmark = pytest.mark.gpu


def _cases(n=12, seed0=3000):
    out = []
    for s in range(seed0, seed0 + 200):
        rng = np.random.default_rng(s)
        spec = _medium_spec(rng, s)
        if spec.num_experts:
            continue
        base = _random_strategy(rng, spec)
        k, cp = int(rng.choice([2, 3])), int(rng.choice([1, 2]))
        if base.pipeline_model_parallel_size > 1:
            continue
        small = PS(base.world_size * cp, base.tensor_model_parallel_size, 1, context_parallel_size=cp)
        big = PS(base.world_size * cp * k, base.tensor_model_parallel_size, 1, context_parallel_size=cp,
                 num_distributed_optimizer_instances=k)
        up = bool(rng.random() < 0.5)
        out.append(pytest.param(spec, small, big, up, id=f"{s}-tp{small.tensor_model_parallel_size}-cp{cp}-"
                                f"{small.world_size}x1{'->' if up else '<-'}{big.world_size}x{k}"))
        if len(out) == n:
            break
    return out


@pytest.mark.parametrize("spec,small,big,up", _cases())
def test_random_group_zero_switch(gpu_device, spec, small, big, up):
    src, dst = (small, big) if up else (big, small)
    kind = "backup_up" if up else "backup_down"
    print(f"case {spec.name} {spec.num_params()} params: {src} -> {dst} ({kind})", flush=True)
    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    tm = TransferManager(check_disjoint=True)
    plan = tm.compile(ls, ld, kind)
    a = TrainingState.allocate(ls, gpu_device)
    a.fill_synthetic(SEED)
    b = TrainingState.allocate(ld, gpu_device, param=a.param)   # the model shards are unchanged
    for t in (b.main, b.exp_avg, b.exp_avg_sq):
        t.fill_(float("nan"))
    tm.execute(plan, a, b)
    torch.cuda.synchronize()
    bad, first = b.verify_synthetic(SEED, bf16=False)
    assert bad == 0, first
    assert tm.verify(a, b, kind).bit_exact
