"""GPU: seeded random medium-size switches between states held in granules of random sizes.

A state handed between processes is held in granules (separate allocations of
less than 2 GiB); the arena plan is re-based onto them.  Here the granules are
small (2 to 200 per fp32 arena, sizes not powers of two) so that plans carry
hundreds of buffers a side and cut segments anywhere; one side of some cases is
a whole-arena state.  Every destination element is checked against the
generator's closed form, and the plan's own verification must find no
difference.
"""

import numpy as np
import pytest
import torch

from elasticmegatron_amd.megatron_manager.training_state import TrainingState
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.ipc_manager import SharedTrainingState
from elasticmegatron_amd.transfer.transfer import TransferManager
from tests.helpers import SEED
from tests.test_gpu_random_medium import _medium_spec
from tests.test_random_switches import _random_strategy

pytestmark = pytest.mark.gpu
SEEDS = range(2000, 2016)


def _granule_bytes(rng, layout):
    """None (whole arenas) a quarter of the time, else a 256-byte multiple cutting the fp32 arenas
    into 2 to 200 granules."""
    k = int(rng.integers(2, 200))
    if rng.random() < 0.25:
        return None
    return max(256, -(-layout.fp32_numel * 4 // k // 256) * 256)


def _case(seed):
    rng = np.random.default_rng(seed)
    spec = _medium_spec(rng, seed)
    a, b = _random_strategy(rng, spec), _random_strategy(rng, spec)
    space = build_virtual_model(spec)
    la, lb = space.layout(a), space.layout(b)
    gs, gd = _granule_bytes(rng, la), _granule_bytes(rng, lb)
    if gs is None and gd is None:
        gs = 1 << 24
    return spec, la, lb, gs, gd


def _state(layout, granule_bytes, device):
    if granule_bytes is None:
        return TrainingState.allocate(layout, device)
    return SharedTrainingState.allocate(layout, device, granule_bytes)


@pytest.mark.parametrize("seed", SEEDS)
def test_random_granule_switch(gpu_device, seed):
    spec, la, lb, gs, gd = _case(seed)
    tm = TransferManager(check_disjoint=True)
    plan = tm.compile_granules(la, lb, gs, gd)
    print(f"case {seed}: {spec.num_params()} params, {la.strategy} -> {lb.strategy}, granules {gs} -> {gd}, "
          f"{len(plan.src)} + {len(plan.dst)} buffers, {plan.segments.shape[0]} segments", flush=True)
    src, dst = _state(la, gs, gpu_device), _state(lb, gd, gpu_device)
    src.fill_synthetic(SEED)
    tm.execute_states(plan, src, dst)
    torch.cuda.synchronize()
    bad, first = dst.verify_synthetic(SEED)
    assert bad == 0, first
    assert tm.verify(src, dst).bit_exact
