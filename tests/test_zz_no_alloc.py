"""emrs_plan_compare_static, the comparison that allocates nothing, against emrs_plan_compare.

Both run through the C ABI on the same plans and states, with mismatches
planted in the destination (flipped bits, NaN, infinities), on consecutive
calls whose second input is smaller than the first: the static array keeps
the previous call's contents, so stale accumulators would show.  Counts and
maxima must be equal, sums equal to 1e-12 relative (atomic accumulation
order varies).  A plan over more than 128 buffers per side stages its
pointer table in the array too.
"""

import numpy as np
import pytest
import torch

from elasticmegatron_amd import ParallelStrategy as PS
from elasticmegatron_amd import _native
from elasticmegatron_amd.megatron_manager.training_state import TrainingState
from elasticmegatron_amd.resharding.lowering import lower_transfer
from elasticmegatron_amd.resharding.model_spec import tiny_llama2
from elasticmegatron_amd.resharding.layout import SEGMENT_DTYPE
from elasticmegatron_amd.resharding.tensors import TensorBuffers, rebase_on_tensors
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.transfer import TransferManager
from tests.helpers import SEED, small_llama2, small_llama3


def _same(a, b):
    for f in ("elements", "mismatches", "nonfinite", "max_abs_diff", "max_rel_diff"):
        assert np.array_equal(a[f], b[f]), f
    for f in ("sum_sq_diff", "sum_sq_expected"):
        assert np.allclose(a[f], b[f], rtol=1e-12, atol=0), f


def _switched(factory, src, dst, dev, plant):
    space = build_virtual_model(factory())
    ls, ld = space.layout(src), space.layout(dst)
    a, b = TrainingState.allocate(ls, dev), TrainingState.allocate(ld, dev)
    a.fill_synthetic(SEED)
    tm = TransferManager()
    tm.execute(tm.compile(ls, ld), a, b)
    # Planted mismatches: bit flips, NaN and infinities in the fp32 arenas, a flip in the bf16 one.
    g = torch.Generator().manual_seed(plant)
    for t in (b.main, b.exp_avg, b.exp_avg_sq):
        idx = torch.randint(0, t.numel(), (7,), generator=g).to(dev)
        t.view(torch.int32)[idx] ^= 1 << plant % 23
        t[idx[:2]] = torch.tensor([float("nan"), float("inf")], device=dev)
    pi = torch.randint(0, b.param.numel(), (5,), generator=g).to(dev)
    b.param.view(torch.int16)[pi] ^= 3
    torch.cuda.synchronize()
    table, groups, aux_groups = lower_transfer(ls, ld, with_groups=True)
    return space, ls, ld, a, b, table, groups, aux_groups


def _both(plan, sp, dp, groups, aux_groups, n):
    st = torch.cuda.current_stream().cuda_stream
    want = plan.compare(sp, dp, groups, aux_groups, n, st)
    got = plan.compare(sp, dp, groups, aux_groups, n, st, no_alloc=True)
    return got, want


@pytest.mark.gpu
def test_static_compare_equals_compare_on_consecutive_calls(gpu_device):
    # Call 1: a larger switch, every group of its model.
    print("case no-alloc 1: small-llama3 TP2PP2 -> TP4PP1", flush=True)
    space, ls, ld, a, b, table, groups, aux_groups = _switched(small_llama3, PS(8, 2, 2), PS(8, 4, 1),
                                                               gpu_device, 5)
    n1 = 4 * len(space.all_virtual_params)
    plan = _native.Plan(table, [ls.fp32_numel * 4] * 3 + [ls.bf16_numel * 2],
                        [ld.fp32_numel * 4] * 3 + [ld.bf16_numel * 2])
    got, want = _both(plan, a.arena_ptrs(), b.arena_ptrs(), groups, aux_groups, n1)
    _same(got, want)
    assert int(want["mismatches"].sum()) >= 20 and int(want["nonfinite"].sum()) >= 6
    # Call 2: a smaller switch with fewer groups and segments (the array still holds call 1's sums).
    print("case no-alloc 2: tiny-llama2 TP2DP4 -> TP1DP8", flush=True)
    space2, ls2, ld2, a2, b2, table2, g2, ag2 = _switched(tiny_llama2, PS(8, 2, 1), PS(8, 1, 1), gpu_device, 9)
    n2 = 4 * len(space2.all_virtual_params)
    assert n2 < n1 and len(table2) < len(table)
    plan2 = _native.Plan(table2, [ls2.fp32_numel * 4] * 3 + [ls2.bf16_numel * 2],
                         [ld2.fp32_numel * 4] * 3 + [ld2.bf16_numel * 2])
    got2, want2 = _both(plan2, a2.arena_ptrs(), b2.arena_ptrs(), g2, ag2, n2)
    _same(got2, want2)
    assert int(want2["mismatches"].sum()) >= 20
    # Call 3, smaller again: one group over the whole plan.
    got3 = plan2.compare(a2.arena_ptrs(), b2.arena_ptrs(), None, None, 1, 0, no_alloc=True)
    want3 = plan2.compare(a2.arena_ptrs(), b2.arena_ptrs(), None, None, 1, 0)
    _same(got3, want3)
    assert got3["mismatches"][0] == want2["mismatches"].sum()


@pytest.mark.gpu
def test_static_compare_with_a_pointer_table(gpu_device):
    """A per-tensor plan (more than 128 buffers a side): its pointer table is staged in the array."""
    print("case no-alloc 3: per-tensor small-llama2 TP1DP8 -> TP4DP2", flush=True)
    space, ls, ld, a, b, table, groups, aux_groups = _switched(small_llama2, PS(8, 1, 1), PS(8, 4, 1),
                                                               gpu_device, 13)
    sb, db = TensorBuffers(ls), TensorBuffers(ld)
    assert len(sb) > 128 and len(db) > 128
    t = rebase_on_tensors(table, sb, db)
    plan = _native.Plan(t, sb.nbytes(), db.nbytes())
    sv, dv = sb.views(a), db.views(b)
    sp, dp = [x.data_ptr() for x in sv], [x.data_ptr() for x in dv]
    for call in range(2):   # a second call with the same pointers, the array already filled
        got = plan.compare(sp, dp, None, None, 1, 0, no_alloc=True)
        want = plan.compare(sp, dp, None, None, 1, 0)
        _same(got, want)
        assert int(want["mismatches"][0]) >= 20


def test_static_compare_refuses_more_than_its_scratch():
    """A comparison beyond the array is refused before any device work (no GPU needed)."""
    n = 80_000   # 80,000 device segments of 64 bytes need more than 4 MiB
    t = np.zeros(n, dtype=SEGMENT_DTYPE)
    t["elem_bytes"] = 4
    t["rows"] = 1
    t["len"] = 4
    t["src_off"] = np.arange(n) * 4
    t["dst_off"] = np.arange(n) * 4
    plan = _native.Plan(t, [n * 16], [n * 16])
    with pytest.raises(_native.EmrsError) as e:
        plan.compare([1 << 20], [1 << 30], None, None, 1, 0, no_alloc=True)
    assert e.value.code == -10 and "scratch" in str(e.value)


@pytest.mark.gpu
def test_static_compare_allocates_nothing(gpu_device):
    """The defining property: on a fresh plan, arena or per-tensor, the static comparison leaves the
    device's free memory unchanged and uploads none of the plan's tables (its first execution is
    still refused under graph capture, as an execution that would upload is), and only then is
    it compared with the allocating path."""
    print("case no-alloc 4: allocates nothing on fresh plans", flush=True)
    # The library meets the device first: kernel code, device properties, the array's address.
    wspace, wls, wld, wa, wb, wt, wg, wag = _switched(tiny_llama2, PS(8, 2, 1), PS(8, 4, 1), gpu_device, 3)
    warm = _native.Plan(wt, [wls.fp32_numel * 4] * 3 + [wls.bf16_numel * 2],
                        [wld.fp32_numel * 4] * 3 + [wld.bf16_numel * 2])
    _both(warm, wa.arena_ptrs(), wb.arena_ptrs(), wg, wag, 4 * len(wspace.all_virtual_params))
    space, ls, ld, a, b, table, groups, aux_groups = _switched(small_llama2, PS(8, 1, 1), PS(8, 4, 1),
                                                               gpu_device, 17)
    n = 4 * len(space.all_virtual_params)
    sb, db = TensorBuffers(ls), TensorBuffers(ld)
    tt = rebase_on_tensors(table, sb, db)
    cases = [
        ("arena", _native.Plan(table, [ls.fp32_numel * 4] * 3 + [ls.bf16_numel * 2],
                               [ld.fp32_numel * 4] * 3 + [ld.bf16_numel * 2]),
         a.arena_ptrs(), b.arena_ptrs(), groups, aux_groups, n),
        ("per-tensor", _native.Plan(tt, sb.nbytes(), db.nbytes()),
         [x.data_ptr() for x in sb.views(a)], [x.data_ptr() for x in db.views(b)], None, None, 1),
    ]
    assert len(sb) > 128
    st = torch.cuda.current_stream()
    marker = torch.zeros(1, device=gpu_device)
    for name, plan, sp, dp, g, ag, ng in cases:
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info(gpu_device)[0]
        got = plan.compare(sp, dp, g, ag, ng, st.cuda_stream, no_alloc=True)
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info(gpu_device)[0] == free0, name
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            marker.fill_(1.0)
            with pytest.raises(_native.EmrsError) as e:
                plan.execute(sp, dp, torch.cuda.current_stream().cuda_stream)
        assert e.value.code == -9, name   # the plan's tables are still to be uploaded
        want = plan.compare(sp, dp, g, ag, ng, st.cuda_stream)
        _same(got, want)
        assert int(want["mismatches"].sum()) >= 20, name
