"""GPU: seeded random medium-size models and switches, checked on the device.

Larger than the CPU oracles can run quickly (hidden 1024-2048, up to 8
layers, vocabularies to 32k, MoE), so every destination element is checked
against the generator's closed form (its value is a function of parameter,
kind and full-tensor index only), the plan's own verification must find no
difference, and the switch back must reproduce the source.
"""

import numpy as np
import pytest
import torch

from elasticmegatron_amd.megatron_manager.training_state import TrainingState
from elasticmegatron_amd.resharding import model_spec as ms
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.transfer import TransferManager
from tests.helpers import SEED
from tests.test_random_switches import _random_strategy

pytestmark = pytest.mark.gpu
N_CASES = 40


def _medium_spec(rng, k):
    heads = int(rng.choice([8, 16]))
    groups = int(rng.choice([0] + [g for g in (2, 4, 8) if heads % g == 0]))
    moe = rng.random() < 0.3
    hidden = int(rng.choice([1024, 2048]))
    return ms.ModelSpec(
        name=f"medium{k}", num_layers=int(rng.choice([4, 8])), hidden_size=hidden, num_attention_heads=heads,
        num_query_groups=groups or None, ffn_hidden_size=int(rng.choice([2816, 5632])),
        padded_vocab_size=int(rng.choice([8192, 32000])), num_experts=int(rng.choice([4, 8])) if moe else None,
        moe_ffn_hidden_size=1408 if moe else None, moe_grouped_gemm=bool(rng.random() < 0.5),
        untie_embeddings_and_output_weights=bool(moe or rng.random() < 0.7),
        ddp_bucket_size=int(rng.choice([1_000_000, 4_000_000, 40_000_000])), overlap_grad_reduce=bool(rng.random() < 0.7))


def _cases():
    rng = np.random.default_rng(7)
    out = []
    for k in range(N_CASES):
        spec = _medium_spec(rng, k)
        a, b = _random_strategy(rng, spec), _random_strategy(rng, spec)
        out.append(pytest.param(spec, a, b, id=f"{k}-{'moe' if spec.num_experts else 'dense'}-h{spec.hidden_size}"
                                f"-tp{a.tensor_model_parallel_size}pp{a.pipeline_model_parallel_size}w{a.world_size}"
                                f"ep{a.expert_model_parallel_size}-tp{b.tensor_model_parallel_size}"
                                f"pp{b.pipeline_model_parallel_size}w{b.world_size}ep{b.expert_model_parallel_size}"))
    return out


@pytest.mark.parametrize("spec,src,dst", _cases())
def test_medium_random_switch(gpu_device, spec, src, dst):
    print(f"case {spec.name} {spec.num_params()} params: {src} -> {dst}", flush=True)
    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    tm = TransferManager(check_disjoint=True)
    a = TrainingState.allocate(ls, gpu_device)
    b = TrainingState.allocate(ld, gpu_device)
    a.fill_synthetic(SEED)
    for t in b.arenas():
        t.fill_(0) if t.dtype != torch.float32 else t.fill_(float("nan"))
    tm.transfer_optimizer_tensors(None, src=a, dst=b)
    bad, first = b.verify_synthetic(SEED)
    assert bad == 0, first
    assert tm.verify(a, b).bit_exact
    back = TrainingState.allocate(ls, gpu_device)
    for t in back.arenas():
        t.fill_(0) if t.dtype != torch.float32 else t.fill_(float("nan"))
    tm.transfer_optimizer_tensors(None, src=b, dst=back)
    bad, first = back.verify_synthetic(SEED)  # the round trip reproduces every source element
    assert bad == 0, first
