"""GPU: the switch over one separately allocated tensor per stored tensor.

The reference's storage format at the transfer boundary -- one tensor per
(rank, parameter, kind) plus the bf16 parameter of each model shard.  The
plan passes their base pointers through kernel arguments (up to 128 per
side) or a device table (more); either way the result must equal the arena
path's, checked element by element against the seeded generator.
"""

import pytest
import torch

from elasticmegatron_amd import ParallelStrategy as PS
from elasticmegatron_amd.megatron_manager.training_state import TrainingState
from elasticmegatron_amd.resharding import model_spec as ms
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.transfer import TransferManager
from tests.helpers import SEED, small_llama2, small_llama3, small_mixtral

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("factory,src,dst", [
    (ms.tiny_llama2, PS(8, 2, 1), PS(8, 1, 1)),
    (small_llama3, PS(8, 2, 2), PS(8, 4, 1)),
    (small_mixtral, PS(8, 1, 1, expert_model_parallel_size=4), PS(8, 1, 1, expert_model_parallel_size=8)),
    (small_llama2, PS(8, 1, 1), PS(6, 2, 1)),
])
def test_separate_tensors_match_arena_path(gpu_device, factory, src, dst):
    space = build_virtual_model(factory())
    ls, ld = space.layout(src), space.layout(dst)
    tm = TransferManager(check_disjoint=True)
    tp = tm.compile_tensors(ls, ld)
    print(f"case {factory.__name__} {src} -> {dst}: {len(tp.src)} / {len(tp.dst)} tensors", flush=True)
    a = TrainingState.allocate(ls, gpu_device)
    a.fill_synthetic(SEED)
    # One allocation per tensor, filled from the generator's arena state.
    src_t = [torch.empty(n, dtype=v.dtype, device=gpu_device) for n, v in zip(tp.src.numel, tp.src.views(a))]
    for t, v in zip(src_t, tp.src.views(a)):
        t.copy_(v)
    dst_t = [torch.full((n,), float("nan"), dtype=torch.float32 if k[0] != "param" else torch.bfloat16,
                        device=gpu_device) for n, k in zip(tp.dst.numel, tp.dst.keys)]
    tm.execute_tensors(tp, src_t, dst_t)
    b = TrainingState.allocate(ld, gpu_device)
    for t, v in zip(dst_t, tp.dst.views(b)):
        v.copy_(t)
    bad, first = b.verify_synthetic(SEED)
    assert bad == 0, first


@pytest.mark.parametrize("n_inst", [2, 3])
def test_group_zero_scale_up_over_separate_tensors(gpu_device, n_inst):
    """Group-ZeRO 1 -> n instances with one allocation per tensor: duplicating segments whose second
    copy lands in another tensor.  The bf16 model shards do not change and are carried over."""
    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(4, 2, 1)), space.layout(PS(4 * n_inst, 2, 1, num_distributed_optimizer_instances=n_inst))
    tm = TransferManager(check_disjoint=True)
    tp = tm.compile_tensors(ls, ld, kind="backup_up")
    assert (tp.segments["flags"] & 4).any()
    print(f"case group zero 1 -> {n_inst}: {len(tp.src)} / {len(tp.dst)} tensors", flush=True)
    a = TrainingState.allocate(ls, gpu_device)
    a.fill_synthetic(SEED)
    src_t = [v.clone() for v in tp.src.views(a)]
    dst_t = [torch.full((n,), float("nan"), dtype=torch.float32 if k[0] != "param" else torch.bfloat16,
                        device=gpu_device) for n, k in zip(tp.dst.numel, tp.dst.keys)]
    tm.execute_tensors(tp, src_t, dst_t)
    b = TrainingState.allocate(ld, gpu_device)
    for t, v, k in zip(dst_t, tp.dst.views(b), tp.dst.keys):
        if k[0] != "param":
            v.copy_(t)
    b.arenas()[3].copy_(a.arenas()[3])
    bad, first = b.verify_synthetic(SEED)
    assert bad == 0, first


@pytest.mark.parametrize("factory,src,dst", [
    (ms.llama2_7b, PS(8, 1, 1), PS(8, 4, 1)),
    (ms.llama3_8b, PS(8, 2, 2), PS(8, 4, 1)),
    (ms.mixtral_8x7b_slice, PS(8, 1, 1, expert_model_parallel_size=4), PS(8, 1, 1, expert_model_parallel_size=8)),
    (ms.llama2_7b, PS(8, 1, 1), PS(6, 1, 1)),
], ids=["llama2-7b-tp1dp8-tp4dp2", "llama3-8b-tp2pp2dp2-tp4pp1dp2", "mixtral-4l-ep4-ep8", "llama2-7b-dp8-dp6"])
def test_full_size_tensor_views(gpu_device, factory, src, dst):
    """Full-size switches over one tensor view per stored tensor (thousands per side): the device-table
    path, checked against the generator and by the plan's own verification."""
    spec = factory()
    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    tm = TransferManager()
    tp = tm.compile_tensors(ls, ld)
    print(f"case full size tensors {spec.name} {src} -> {dst}: {len(tp.src)} / {len(tp.dst)} tensors", flush=True)
    a = b = None
    try:
        a = TrainingState.allocate(ls, gpu_device)
        b = TrainingState.allocate(ld, gpu_device)
        a.fill_synthetic(SEED)
        tm.execute_tensors(tp, tp.src.views(a), tp.dst.views(b))
        bad, first = b.verify_synthetic(SEED)
        assert bad == 0, first
        assert tm.verify(a, b).bit_exact
    finally:
        a = b = None  # noqa: F841
        torch.cuda.synchronize()
        torch.cuda.empty_cache()


def test_compare_through_pointer_table(gpu_device):
    """emrs_plan_compare over a per-tensor plan with more than 128 buffers per side."""
    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(8, 1, 1)), space.layout(PS(6, 2, 1))
    tm = TransferManager()
    tp = tm.compile_tensors(ls, ld)
    assert len(tp.src) > 128 and len(tp.dst) > 128
    a = TrainingState.allocate(ls, gpu_device)
    b = TrainingState.allocate(ld, gpu_device)
    a.fill_synthetic(SEED)
    sv, dv = tp.src.views(a), tp.dst.views(b)
    tm.execute_tensors(tp, sv, dv)
    stream = torch.cuda.current_stream().cuda_stream
    ps, pd = [t.data_ptr() for t in sv], [t.data_ptr() for t in dv]
    stats = tp.native.compare(ps, pd, stream=stream)
    total = int((tp.segments["len"] * tp.segments["rows"]).sum()) + \
        int((tp.segments["len"] * tp.segments["rows"])[(tp.segments["flags"] & 1) != 0].sum())
    assert int(stats["elements"][0]) == total and int(stats["mismatches"][0]) == 0
    # One element changed on the host, uploaded back: exactly one mismatch.
    host = b.main.cpu()
    host[7] = host[7] + 1.0
    b.main.copy_(host)
    torch.cuda.synchronize()
    stats = tp.native.compare(ps, pd, stream=stream)
    assert int(stats["mismatches"][0]) == (1 if 7 in _covered(tp, ld) else 0)


def test_repeated_tensor_lists_skip_the_layout_check(gpu_device):
    """The same tensors again skip the layout check; a tensor at another address is checked again."""
    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(8, 1, 1)), space.layout(PS(8, 4, 1))
    tm = TransferManager()
    tp = tm.compile_tensors(ls, ld)
    a, b = TrainingState.allocate(ls, gpu_device), TrainingState.allocate(ld, gpu_device)
    a.fill_synthetic(SEED)
    src_v, dst_v = tp.src.views(a), tp.dst.views(b)
    print("case repeated tensor lists", flush=True)
    for _ in range(3):
        b.main.zero_()
        tm.execute_tensors(tp, src_v, dst_v)
        torch.cuda.synchronize()
        assert b.verify_synthetic(SEED)[0] == 0
    assert tm._checked_tensors[id(tp)][1] == [t.data_ptr() for t in list(src_v) + list(dst_v)]
    strided = torch.empty(2 * dst_v[0].numel(), dtype=dst_v[0].dtype, device=gpu_device)[::2]
    assert strided.nbytes == dst_v[0].nbytes and not strided.is_contiguous()
    with pytest.raises(ValueError):
        tm.execute_tensors(tp, src_v, [strided] + list(dst_v[1:]))
    b.main.zero_()
    tm.execute_tensors(tp, src_v, dst_v)
    torch.cuda.synchronize()
    assert b.verify_synthetic(SEED)[0] == 0


def _covered(tp, ld):
    """Element indices of the main arena that some fp32 tensor holds (the checked ones)."""
    out = set()
    for a, o, n in zip(tp.dst.arena, tp.dst.offset, tp.dst.numel):
        if a == 0 and o <= 7 < o + n:
            out.add(7)
    return out
