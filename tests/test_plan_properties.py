"""Properties of the copy plan over hypothesis-drawn models and strategy pairs (CPU).

For every drawn switch A -> B:

- the plan writes every stored destination element exactly once: its
  destination ranges are disjoint (emrs_plan_create's own check) and its
  payload equals the bytes the destination layout stores;
- A -> B -> A restores every stored value of A (run through a numpy model of
  the kernel), and A -> A reproduces A.

The values are the seeded generator's, which depend only on (parameter,
kind, full-tensor index), so replicas agree and a round trip must be exact.
"""

from hypothesis import HealthCheck, assume, given, settings
from hypothesis import strategies as st

from elasticmegatron_amd import _native
from elasticmegatron_amd import ParallelStrategy as PS
from elasticmegatron_amd.resharding import model_spec as ms
from elasticmegatron_amd.resharding.lowering import lower_transfer
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from tests.helpers import SEED, compare, execute_numpy, extract, new_arenas, piece_fill_numpy


@st.composite
def switches(draw):
    heads = draw(st.sampled_from([4, 8]))
    groups = draw(st.sampled_from([None] + [g for g in (2, 4) if heads % g == 0]))
    moe = draw(st.booleans())
    spec = ms.ModelSpec(
        name="prop", num_layers=draw(st.sampled_from([2, 4])), hidden_size=draw(st.sampled_from([128, 256])),
        num_attention_heads=heads, num_query_groups=groups, kv_channels=32,
        ffn_hidden_size=draw(st.sampled_from([256, 384])), padded_vocab_size=draw(st.sampled_from([512, 1024])),
        num_experts=4 if moe else None, moe_ffn_hidden_size=256 if moe else None,
        untie_embeddings_and_output_weights=moe or draw(st.booleans()),
        ddp_bucket_size=draw(st.sampled_from([20_000, 200_000])), overlap_grad_reduce=draw(st.booleans()))

    def strategy():
        world = draw(st.sampled_from([2, 4, 8]))
        tp = draw(st.sampled_from([t for t in (1, 2, 4) if world % t == 0]))
        pp = draw(st.sampled_from([p for p in (1, 2) if (world // tp) % p == 0]))
        ep = draw(st.sampled_from([e for e in (1, 2, 4) if (world // pp) % e == 0])) if moe else 1
        return PS(world, tp, pp, expert_model_parallel_size=ep, expert_tensor_parallel_size=1 if moe else None)

    a, b = strategy(), strategy()
    for s in (a, b):
        q = groups or heads
        assume(q % s.tensor_model_parallel_size == 0 and heads % s.tensor_model_parallel_size == 0)
        assume(spec.num_layers % s.pipeline_model_parallel_size == 0)
        try:
            s.validate_for(spec.num_layers, spec.num_experts)
        except (AssertionError, ValueError):
            assume(False)
    return spec, a, b


def _stored_bytes(layout):
    space = layout.space
    held = [vp for vp in space.all_virtual_params if layout.has_param(vp)]
    return (12 * sum(h.hi - h.lo for vp in held for h in layout.fp32_holders(vp))
            + 2 * sum(h.hi - h.lo for vp in held for h in layout.bf16_holders(vp)))


def _lowered(space, a, b):
    try:
        space.register_reshard(a, b)
        la, lb = space.layout(a), space.layout(b)
    except (AssertionError, RuntimeError, ValueError):
        assume(False)   # a layout the reference refuses too (e.g. a DP rank with no piece)
    return la, lb, lower_transfer(la, lb)


@settings(max_examples=20, deadline=None, suppress_health_check=[HealthCheck.filter_too_much, HealthCheck.too_slow])
@given(switches())
def test_plan_is_a_bijection_and_round_trips(sw):
    spec, a, b = sw
    space = build_virtual_model(spec)
    la, lb, ab = _lowered(space, a, b)
    _, _, ba = _lowered(space, b, a)
    # Exactly once: disjoint destinations (checked natively) and as many bytes as the destination stores.
    for t, src, dst in ((ab, la, lb), (ba, lb, la)):
        plan = _native.Plan(t, [src.fp32_numel * 4] * 3 + [src.bf16_numel * 2],
                            [dst.fp32_numel * 4] * 3 + [dst.bf16_numel * 2], check_disjoint=True)
        assert plan.stats().payload_bytes == _stored_bytes(dst)
    # A -> B -> A restores A.
    arena_a = new_arenas(la)
    piece_fill_numpy(la.pieces(), arena_a, SEED)
    arena_b = new_arenas(lb)
    execute_numpy(ab, arena_a, arena_b)
    back = new_arenas(la)
    execute_numpy(ba, arena_b, back)
    got32, gotbf = extract(la, back)
    want32, wantbf = extract(la, arena_a)
    assert compare(got32, gotbf, want32, wantbf) == []


@settings(max_examples=10, deadline=None, suppress_health_check=[HealthCheck.filter_too_much, HealthCheck.too_slow])
@given(switches())
def test_switch_to_the_same_strategy_reproduces_the_state(sw):
    spec, a, _ = sw
    space = build_virtual_model(spec)
    la, _, aa = _lowered(space, a, a)
    arena = new_arenas(la)
    piece_fill_numpy(la.pieces(), arena, SEED)
    out = new_arenas(la)
    execute_numpy(aa, arena, out)
    got32, gotbf = extract(la, out)
    want32, wantbf = extract(la, arena)
    assert compare(got32, gotbf, want32, wantbf) == []


@settings(max_examples=15, deadline=None, suppress_health_check=[HealthCheck.filter_too_much, HealthCheck.too_slow])
@given(switches())
def test_megatron_buffer_views_tile_the_stored_elements(sw):
    """Over drawn layouts, the views MegatronBuffers hands out are disjoint, lie inside their
    buffers, cover exactly the layout's stored elements, and the remapped generator pieces land
    in the same views as the arena pieces."""
    import numpy as np
    import torch

    from elasticmegatron_amd.resharding.megatron_buffers import MegatronBuffers
    from elasticmegatron_amd.resharding.tensors import TensorBuffers

    spec, a, _ = sw
    space = build_virtual_model(spec)
    try:
        lay = space.layout(a)
    except (AssertionError, RuntimeError, ValueError):
        assume(False)
    mb, tb = MegatronBuffers(lay), TensorBuffers(lay)
    flat = [np.zeros(n, dtype=np.uint16 if d == "bf16" else np.uint32) for _, d, n in mb.specs]
    piece_fill_numpy(mb.remap_pieces(lay.pieces()), flat, SEED)
    hits = [np.zeros(x.size, dtype=np.int32) for x in flat]
    bufs = {k: torch.from_numpy(x.view(np.int16) if x.dtype == np.uint16 else x.view(np.int32))
            for k, x in zip(mb.keys(), flat)}
    index = {k: i for i, k in enumerate(mb.keys())}
    arenas = new_arenas(lay, fill=0)
    piece_fill_numpy(lay.pieces(), arenas, SEED)
    for ar, off, n, v in zip(tb.arena, tb.offset, tb.numel, mb.tensor_views(tb, bufs)):
        key, local = mb.locate(ar, off, n)
        hits[index[key]][local:local + n] += 1
        assert np.array_equal(v.numpy().view(arenas[ar].dtype), arenas[ar][off:off + n])
    assert all(int(h.max(initial=0)) <= 1 for h in hits)
    covered = sum(int(h.sum()) for h in hits)
    assert covered == sum(tb.numel)
    fp32 = sum(n for ar, n in zip(tb.arena, tb.numel) if ar != 3)   # three kinds
    bf16 = sum(n for ar, n in zip(tb.arena, tb.numel) if ar == 3)
    assert 4 * fp32 + 2 * bf16 == _stored_bytes(lay)
