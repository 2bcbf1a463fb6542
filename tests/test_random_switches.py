"""Randomised switches: the product's plan against both oracles, bit for bit.

Seeded random small models -- MHA or GQA, dense or MoE, tied or untied
embeddings, with or without DDP buckets -- and random valid pairs of
parallel strategies (TP, PP, DP, EP and world size changing together).  For
each, the plan executed by the numpy model of the kernel must equal
Oracle-1 (the reference's three-pass executor restated) and Oracle-2 (the
canonical full-tensor reslice), in both bf16 modes.
"""

import numpy as np
import pytest

from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy as PS
from elasticmegatron_amd.resharding import model_spec as ms
from elasticmegatron_amd.resharding.lowering import lower_transfer
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from oracle import canonical, model
from oracle import transfer as oracle1
from tests.helpers import SEED, compare, execute_numpy, extract, new_arenas, piece_fill_numpy, strat

N_CASES = 24


def _random_spec(rng, k):
    heads = int(rng.choice([4, 8]))
    choices = [0] + [g for g in (2, 4) if heads % g == 0]
    groups = int(rng.choice(choices))
    moe = rng.random() < 0.3
    return ms.ModelSpec(
        name=f"rand{k}", num_layers=int(rng.choice([2, 4])), hidden_size=int(rng.choice([128, 256])),
        num_attention_heads=heads, num_query_groups=groups or None, kv_channels=int(rng.choice([16, 32])),
        ffn_hidden_size=int(rng.choice([256, 384, 512])), padded_vocab_size=int(rng.choice([512, 1024])),
        num_experts=int(rng.choice([4, 8])) if moe else None, moe_ffn_hidden_size=256 if moe else None,
        moe_grouped_gemm=bool(rng.random() < 0.5),
        untie_embeddings_and_output_weights=bool(moe or rng.random() < 0.7),
        ddp_bucket_size=int(rng.choice([20_000, 60_000, 200_000])), overlap_grad_reduce=bool(rng.random() < 0.7))


def _with_cp(rng, s, spec):
    """``s`` with context parallelism 2 (half the DP ranks), when that is valid and the draw says so."""
    if rng.random() >= 0.35:
        return s
    try:
        c = PS(s.world_size, s.tensor_model_parallel_size, s.pipeline_model_parallel_size, context_parallel_size=2,
               expert_model_parallel_size=s.expert_model_parallel_size,
               expert_tensor_parallel_size=s.expert_tensor_parallel_size if spec.num_experts else None)
        c.validate_for(spec.num_layers, spec.num_experts)
    except (ValueError, AssertionError, RuntimeError):
        return s
    return c


def _random_strategy(rng, spec):
    for _ in range(200):
        world = int(rng.choice([2, 4, 6, 8]))
        tp = int(rng.choice([t for t in (1, 2, 4) if world % t == 0]))
        pp = int(rng.choice([p for p in (1, 2) if (world // tp) % p == 0]))
        ep = 1
        if spec.num_experts:
            ep = int(rng.choice([e for e in (1, 2, 4) if spec.num_experts % e == 0 and (world // pp) % e == 0]))
        groups = spec.num_query_groups or spec.num_attention_heads
        if groups % tp or spec.num_attention_heads % tp or spec.ffn_hidden_size % tp:
            continue
        if spec.num_layers % pp:
            continue
        try:
            s = PS(world, tp, pp, expert_model_parallel_size=ep,
                   expert_tensor_parallel_size=1 if spec.num_experts else None)
            s.validate_for(spec.num_layers, spec.num_experts)
        except (ValueError, AssertionError, RuntimeError):
            continue
        return s
    raise RuntimeError("no valid strategy")


def _cases():
    rng = np.random.default_rng(20261201)
    cp_rng = np.random.default_rng(20261202)  # separate, so the other draws stay as they were
    out = []
    for k in range(N_CASES):
        spec = _random_spec(rng, k)
        a, b = _random_strategy(rng, spec), _random_strategy(rng, spec)
        a, b = _with_cp(cp_rng, a, spec), _with_cp(cp_rng, b, spec)
        mode = "cast" if k % 2 == 0 else "copy"
        out.append(pytest.param(spec, a, b, mode, id=f"{k}-{'moe' if spec.num_experts else 'dense'}"
                                f"-tp{a.tensor_model_parallel_size}pp{a.pipeline_model_parallel_size}"
                                f"w{a.world_size}ep{a.expert_model_parallel_size}cp{a.context_parallel_size}"
                                f"-tp{b.tensor_model_parallel_size}pp{b.pipeline_model_parallel_size}"
                                f"w{b.world_size}ep{b.expert_model_parallel_size}cp{b.context_parallel_size}-{mode}"))
    return out


@pytest.mark.parametrize("spec,src,dst,bf16_source", _cases())
def test_random_switch_matches_oracles(spec, src, dst, bf16_source):
    inv = model.inventory(spec)
    S, D = strat(src), strat(dst)
    world = oracle1.build_src_world(inv, spec, S, SEED)
    dw, dbf, _ = oracle1.transfer(inv, spec, S, D, world)
    o1_32 = oracle1.flatten(dw)
    o2_32, o2_bf = canonical.world(inv, spec, D, SEED)
    assert compare(o1_32, dbf, o2_32, o2_bf) == []

    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    table = lower_transfer(ls, ld, bf16_source=bf16_source)
    a, b = new_arenas(ls), new_arenas(ld)
    piece_fill_numpy(ls.pieces(), a, SEED)
    execute_numpy(table, a, b)
    got32, gotbf = extract(ld, b)
    assert compare(got32, gotbf, o1_32, dbf) == []
