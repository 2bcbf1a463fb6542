"""GPU: emrs_plan_compare against its numpy model, and reshard verification end to end.

Differences are planted in host copies of the destination (on the CPU) and
uploaded; the kernel must report exactly the counts and maxima the numpy
model (tests.helpers.compare_numpy, itself pinned against compare_ckpt.py's
formulas in tests/test_verify.py) reports, and the same sums to 1e-9.
"""

import numpy as np
import pytest
import torch

from elasticmegatron_amd import _native
from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy as PS
from elasticmegatron_amd.megatron_manager.training_state import TrainingState
from elasticmegatron_amd.resharding.layout import SEGMENT_DTYPE
from elasticmegatron_amd.resharding.lowering import lower_transfer
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.transfer import TransferManager
from tests.helpers import SEED, compare_numpy, small_llama2, small_llama3
from tests.test_gpu_parity import _host_arenas, _random_table
from tests.test_verify import _plant

pytestmark = pytest.mark.gpu


def _assert_stats_equal(got, want):
    for f in ("elements", "mismatches", "nonfinite", "max_abs_diff", "max_rel_diff"):
        assert np.array_equal(got[f], want[f]), f
    for f in ("sum_sq_diff", "sum_sq_expected"):
        np.testing.assert_allclose(got[f], want[f], rtol=1e-9, atol=0)


def _upload(state, host):
    for t, h in zip(state.arenas(), host):
        src = torch.from_numpy(h.view(np.int32) if h.dtype == np.uint32 else h.view(np.int16))
        t.view(torch.int32 if t.dtype == torch.float32 else torch.int16).copy_(src)
    torch.cuda.synchronize()


@pytest.mark.parametrize("factory,src,dst,bf16_source", [
    (small_llama3, PS(8, 2, 2), PS(8, 4, 1), "cast"),
    (small_llama2, PS(8, 1, 1), PS(8, 4, 1), "copy"),
    (small_llama2, PS(8, 1, 4), PS(6, 2, 1), "cast"),
])
def test_compare_kernel_matches_numpy(gpu_device, factory, src, dst, bf16_source):
    print(f"case {factory.__name__} {src} -> {dst} {bf16_source}", flush=True)
    space = build_virtual_model(factory())
    ls, ld = space.layout(src), space.layout(dst)
    a = TrainingState.allocate(ls, gpu_device)
    b = TrainingState.allocate(ld, gpu_device)
    a.fill_synthetic(SEED)
    tm = TransferManager(bf16_source=bf16_source)
    tm.transfer_optimizer_tensors(None, src=a, dst=b)
    rep = tm.verify(a, b)
    assert rep.bit_exact
    held = [vp for vp in space.all_virtual_params if ld.has_param(vp)]
    assert rep.elements == sum(3 * (h.hi - h.lo) for vp in held for h in ld.fp32_holders(vp)) + \
        sum(h.hi - h.lo for vp in held for h in ld.bf16_holders(vp))

    host_src = _host_arenas(a)
    host_dst = _host_arenas(b)
    _plant(host_dst, np.random.default_rng(1), 100)
    _upload(b, host_dst)
    table, groups, aux_groups = lower_transfer(ls, ld, bf16_source=bf16_source, with_groups=True)
    n_groups = 4 * len(space.all_virtual_params)
    want = compare_numpy(table, groups, aux_groups, n_groups, host_src, host_dst)
    plan = _native.Plan(table, [ls.fp32_numel * 4] * 3 + [ls.bf16_numel * 2],
                        [ld.fp32_numel * 4] * 3 + [ld.bf16_numel * 2])
    got = plan.compare(a.arena_ptrs(), b.arena_ptrs(), groups, aux_groups, n_groups,
                       torch.cuda.current_stream().cuda_stream)
    _assert_stats_equal(got, want)
    rep = tm.verify(a, b)
    assert rep.mismatches == int(want["mismatches"].sum()) > 0


@pytest.mark.parametrize("seed", [0, 1])
def test_compare_random_tables(gpu_device, seed):
    """Every element width and path, zero fills, casts and duplicates, random groups."""
    rng = np.random.default_rng(seed)
    nbytes = 1 << 20
    table = _random_table(rng, 120, (nbytes, nbytes))
    # Keep segments whose destination bytes (and bf16 images) do not overlap earlier ones.
    used = np.zeros(2 * nbytes, dtype=bool)
    keep = []
    for s in table:
        eb = int(s["elem_bytes"])
        spans = [(int(s["dst_off"]) * eb + r * int(s["dst_stride"]) * eb, int(s["len"]) * eb)
                 for r in range(int(s["rows"]))]
        if int(s["flags"]) & 5:
            w = 2 if int(s["flags"]) & 1 else eb
            spans += [(nbytes + (int(s["aux_off"]) + r * int(s["aux_stride"])) * w, int(s["len"]) * w)
                      for r in range(int(s["rows"]))]
        if any(used[o:o + n].any() for o, n in spans):
            continue
        for o, n in spans:
            used[o:o + n] = True
        keep.append(s)
    t = np.array(keep, dtype=SEGMENT_DTYPE)
    print(f"case seed {seed}: {len(t)} segments", flush=True)
    groups = rng.integers(0, 5, len(t)).astype(np.uint32)
    aux_groups = rng.integers(0, 5, len(t)).astype(np.uint32)
    src_h = rng.integers(0, 256, nbytes, dtype=np.uint8)
    src = torch.from_numpy(src_h).to(gpu_device)
    dst = torch.zeros(nbytes, dtype=torch.uint8, device=gpu_device)
    aux = torch.zeros(nbytes, dtype=torch.uint8, device=gpu_device)
    plan = _native.Plan(t, [nbytes], [nbytes, nbytes], check_disjoint=True)
    stream = torch.cuda.current_stream().cuda_stream
    plan.execute([src.data_ptr()], [dst.data_ptr(), aux.data_ptr()], stream)
    torch.cuda.synchronize()
    d_h, a_h = dst.cpu().numpy(), aux.cpu().numpy()
    got = plan.compare([src.data_ptr()], [dst.data_ptr(), aux.data_ptr()], groups, aux_groups, 5, stream)
    assert int(got["mismatches"].sum()) == 0
    want = compare_numpy(t, groups, aux_groups, 5, [src_h], [d_h, a_h])
    _assert_stats_equal(got, want)
    # Plant differences in the host copies and compare again.
    idx = rng.choice(nbytes, 2000, replace=False)
    d_h[idx] ^= np.uint8(0x5A)
    a_h[idx[:500]] ^= np.uint8(0x01)
    dst.copy_(torch.from_numpy(d_h))
    aux.copy_(torch.from_numpy(a_h))
    got = plan.compare([src.data_ptr()], [dst.data_ptr(), aux.data_ptr()], groups, aux_groups, 5, stream)
    want = compare_numpy(t, groups, aux_groups, 5, [src_h], [d_h, a_h])
    _assert_stats_equal(got, want)
    assert int(got["mismatches"].sum()) > 0


def test_manager_reshard_with_verification(gpu_device):
    """reshard(verify=True) through TP, PP, DP, Group-ZeRO and re-padding switches."""
    from dataclasses import replace
    from elasticmegatron_amd import ElasticMegatronManager

    spec = replace(small_llama3(), vocab_size=2300)
    seq = [dict(world_size=8, tensor_model_parallel_size=2, pipeline_model_parallel_size=2),
           dict(world_size=8, tensor_model_parallel_size=4, pipeline_model_parallel_size=1),
           dict(world_size=6, tensor_model_parallel_size=2, pipeline_model_parallel_size=1),
           dict(world_size=12, tensor_model_parallel_size=2, pipeline_model_parallel_size=1,
                num_distributed_optimizer_instances=2)]
    for repad in (False, True):
        mgr = ElasticMegatronManager(seq, spec, device=gpu_device, repad_vocab=repad)
        mgr.training_state.fill_synthetic(SEED)
        for s in seq[1:] + seq[2:3] + seq[:1]:
            print(f"case repad {repad} -> {s}", flush=True)
            mgr.reshard(new_parallel_strategy=s, verify=True)
            rep = mgr.last_verification
            assert rep.bit_exact and rep.elements > 0
        assert mgr.training_state.verify_synthetic(SEED)[0] == 0


@pytest.mark.parametrize("granule", [None, 1 << 16], ids=["arenas", "granules"])
@pytest.mark.parametrize("no_alloc", [False, True], ids=["compare", "compare_static"])
def test_compare_reads_a_state_against_itself(gpu_device, granule, no_alloc):
    """A comparison only reads, so its source and destination may be the same memory (a state that
    took over part of its source's).  The identity switch S -> S, compared between a state and
    itself, finds every element equal: in arenas, and in granules of 64 KiB (hundreds of buffers
    a side, the pointer-table path), with either entry point."""
    from elasticmegatron_amd.resharding.granules import GranuleBuffers
    from elasticmegatron_amd.resharding.tensors import rebase_on_tensors
    from elasticmegatron_amd.transfer.ipc_manager import SharedTrainingState

    space = build_virtual_model(small_llama2())
    s = PS(8, 2, 1)
    space.register_reshard(s, s)
    lay = space.layout(s)
    table, groups, aux_groups = lower_transfer(lay, lay, with_groups=True)
    if granule is None:
        st = TrainingState.allocate(lay, gpu_device)
        sizes = [lay.fp32_numel * 4] * 3 + [lay.bf16_numel * 2]
        ptrs = st.arena_ptrs()
    else:
        gb = GranuleBuffers(lay, granule)
        table, origin = rebase_on_tensors(table, gb, gb, return_origin=True)
        groups, aux_groups = groups[origin], aux_groups[origin]
        st = SharedTrainingState.allocate(lay, gpu_device, granule)
        sizes, ptrs = gb.nbytes(), st.buffer_ptrs()
        assert len(ptrs) > 128
    st.fill_synthetic(SEED)
    plan = _native.Plan(table, sizes, sizes)
    n_groups = 4 * len(space.all_virtual_params)
    print(f"case self-compare granule={granule} no_alloc={no_alloc}: {len(ptrs)} buffers a side", flush=True)
    stats = plan.compare(ptrs, ptrs, groups, aux_groups, n_groups, torch.cuda.current_stream(gpu_device).cuda_stream,
                         no_alloc=no_alloc)
    assert int(stats["elements"].sum()) > 0
    assert int(stats["mismatches"].sum()) == 0
    with pytest.raises(_native.EmrsError) as e:       # an execution over the same memory is refused
        plan.execute(ptrs, ptrs, torch.cuda.current_stream(gpu_device).cuda_stream)
    assert e.value.code == -8
