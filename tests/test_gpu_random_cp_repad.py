"""GPU: seeded random medium-size switches with context parallelism, and with the vocabulary re-padded.

Context parallelism: the distributed optimizer shards over DP x CP ranks, so a
CP change moves every shard boundary.  Re-padding: each side is laid out at
Megatron's padded vocabulary for its own TP size (an extension; the reference
keeps the padded vocabulary fixed).  Every destination element is checked
against the generator's closed form (new padding rows must be zero), the
plan's own verification must find no difference, and the CP switches must
round-trip.
"""

from dataclasses import replace

import numpy as np
import pytest
import torch

from elasticmegatron_amd.megatron_manager.training_state import TrainingState
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.transfer import TransferManager
from tests.helpers import SEED, repad_spaces
from tests.test_gpu_random_medium import _medium_spec
from tests.test_random_switches import _random_strategy, _with_cp

pytestmark = pytest.mark.gpu


def _cp_cases(n=10):
    rng, cp_rng = np.random.default_rng(9001), np.random.default_rng(9002)
    out = []
    for k in range(400):
        spec = _medium_spec(rng, k)
        a, b = _random_strategy(rng, spec), _random_strategy(rng, spec)
        a, b = _with_cp(cp_rng, a, spec), _with_cp(cp_rng, b, spec)
        if max(a.context_parallel_size, b.context_parallel_size) == 1:
            continue
        out.append(pytest.param(spec, a, b, id=f"{k}-{'moe' if spec.num_experts else 'dense'}-"
                                f"tp{a.tensor_model_parallel_size}cp{a.context_parallel_size}w{a.world_size}-"
                                f"tp{b.tensor_model_parallel_size}cp{b.context_parallel_size}w{b.world_size}"))
        if len(out) == n:
            break
    return out


def _repad_cases(n=8):
    rng = np.random.default_rng(9003)
    out = []
    for k in range(400):
        spec = _medium_spec(rng, k)
        if spec.num_experts:
            continue
        spec = replace(spec, vocab_size=int(rng.integers(30_000, 33_000)))
        a, b = _random_strategy(rng, spec), _random_strategy(rng, spec)
        pa, pb = (spec.padded_vocab_for_tp(s.tensor_model_parallel_size) for s in (a, b))
        if pa == pb:
            continue
        out.append(pytest.param(spec, a, b, id=f"{k}-vocab{spec.vocab_size}-tp{a.tensor_model_parallel_size}"
                                f"w{a.world_size}-{pa}-tp{b.tensor_model_parallel_size}w{b.world_size}-{pb}"))
        if len(out) == n:
            break
    return out


def _fresh(layout, device):
    st = TrainingState.allocate(layout, device)
    for t in st.arenas():
        t.fill_(0) if t.dtype != torch.float32 else t.fill_(float("nan"))
    return st


@pytest.mark.parametrize("spec,src,dst", _cp_cases())
def test_random_context_parallel_switch(gpu_device, spec, src, dst):
    print(f"case {spec.name} {spec.num_params()} params: {src} -> {dst}", flush=True)
    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    tm = TransferManager(check_disjoint=True)
    a = TrainingState.allocate(ls, gpu_device)
    a.fill_synthetic(SEED)
    b = _fresh(ld, gpu_device)
    tm.transfer_optimizer_tensors(None, src=a, dst=b)
    bad, first = b.verify_synthetic(SEED)
    assert bad == 0, first
    assert tm.verify(a, b).bit_exact
    back = _fresh(ls, gpu_device)
    tm.transfer_optimizer_tensors(None, src=b, dst=back)
    bad, first = back.verify_synthetic(SEED)
    assert bad == 0, first


@pytest.mark.parametrize("spec,src,dst", _repad_cases())
def test_random_repadded_switch(gpu_device, spec, src, dst):
    sa, sb = repad_spaces(spec, (src.tensor_model_parallel_size, dst.tensor_model_parallel_size))
    print(f"case {spec.name} vocab {spec.vocab_size}: {sa.spec.padded_vocab_size} -> {sb.spec.padded_vocab_size}, "
          f"{src} -> {dst}", flush=True)
    ls, ld = sa.layout(src), sb.layout(dst)
    tm = TransferManager(check_disjoint=True)
    a = TrainingState.allocate(ls, gpu_device)
    a.fill_synthetic(SEED)
    b = _fresh(ld, gpu_device)
    tm.transfer_optimizer_tensors(None, src=a, dst=b)
    bad, first = b.verify_synthetic(SEED, vocab_rows=sa.spec.padded_vocab_size)
    assert bad == 0, first
    assert tm.verify(a, b).bit_exact
