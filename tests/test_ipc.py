"""Inter-process hand-off: host-side checks that need no GPU.

The reference exports one CUDA-IPC handle per optimizer tensor storage and
rebuilds the tensors in the new process (elastic_megatron/transfer/ipc_manager.py:23-155).
Here a state is exported as granules of less than 2 GiB.  These tests cover
the payload's encoding, the checks made before any handle reaches the driver,
and planning a switch from a received state on the meta device; the hand-off
itself runs on the GPU (tests/test_gpu_ipc.py).
"""

import ctypes
import dataclasses
import json

import numpy as np
import pytest
import torch

from elasticmegatron_amd import ElasticMegatronManager, ParallelStrategy as PS, _native
from elasticmegatron_amd.resharding.granules import GranuleBuffers
from elasticmegatron_amd.resharding.model_spec import ModelSpec, llama2_7b, tiny_llama2
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer import ipc_manager as ipc
from elasticmegatron_amd.transfer.transfer import (CompiledTensorPlan, TransferManager, adoptable_granules,
                                                   held_granules, shares_params)
from tests.helpers import small_llama2


def _record(**kw):
    rec = np.zeros(1, dtype=_native.IPC_BUFFER_DTYPE)
    rec["handle"] = np.arange(64, dtype=np.uint8)
    for k, v in kw.items():
        rec[k] = v
    return rec[0]


def test_record_layout_matches_the_header():
    lib = _native.load()
    assert _native.IPC_BUFFER_DTYPE.itemsize == 96
    assert [n for n in _native.IPC_BUFFER_DTYPE.names] == ["handle", "offset", "bytes", "allocation_bytes",
                                                          "device", "reserved"]
    assert lib.emrs_ipc_open_count() == 0


def test_record_round_trips_through_text():
    rec = _record(offset=4096, bytes=1 << 20, allocation_bytes=1 << 30, device=3)
    back = ipc._record_of(ipc._record_hex(rec))
    assert back.tobytes() == np.asarray(rec).tobytes()
    with pytest.raises(ValueError):
        ipc._record_of("00" * 95)


@pytest.mark.parametrize("alloc", [2 << 30, (2 << 30) + 4096, 0])
def test_open_refuses_allocations_of_2gib_or_more_before_the_driver(alloc):
    with pytest.raises(_native.EmrsError) as e:
        _native.ipc_open(_record(offset=0, bytes=256, allocation_bytes=alloc))
    assert e.value.code == -10   # EMRS_ERR_TOO_LARGE
    assert _native.ipc_open_count() == 0


def test_open_checks_the_record():
    with pytest.raises(_native.EmrsError) as e:
        _native.ipc_open(_record(offset=0, bytes=256, allocation_bytes=4096, reserved=1))
    assert e.value.code == -1
    with pytest.raises(_native.EmrsError) as e:
        _native.ipc_open(_record(offset=4000, bytes=256, allocation_bytes=4096))
    assert e.value.code == -2    # runs past its allocation
    with pytest.raises(_native.EmrsError) as e:
        _native.ipc_open(_record(offset=8, bytes=256, allocation_bytes=4096))
    assert e.value.code == -3    # not 16-byte aligned


def test_close_and_export_refuse_unknown_pointers():
    with pytest.raises(_native.EmrsError) as e:
        _native.ipc_close(0x1000)
    assert e.value.code == -1
    lib = _native.load()
    rec = np.zeros(1, dtype=_native.IPC_BUFFER_DTYPE)
    assert lib.emrs_ipc_export(None, 256, rec.ctypes.data) == -1
    assert lib.emrs_ipc_export(ctypes.c_void_p(0x1008), 256, rec.ctypes.data) == -3


def test_strategy_and_model_round_trip():
    for s in (PS(8, 2, 1), PS(8, 1, 2, context_parallel_size=2), PS(12, 1, 1, num_distributed_optimizer_instances=2),
              PS(8, 1, 1, expert_model_parallel_size=4)):
        d = json.loads(json.dumps(ipc.strategy_to_dict(s)))
        back = PS(**d)
        assert back == s and back.sequence_parallel == s.sequence_parallel
    spec = llama2_7b()
    assert ModelSpec(**json.loads(json.dumps(dataclasses.asdict(spec)))) == spec


def _payload(spec, strategy, granule):
    layout = build_virtual_model(spec).layout(strategy)
    bufs = GranuleBuffers(layout, granule)
    return {"format": ipc.PAYLOAD_FORMAT, "model_spec": dataclasses.asdict(spec),
            "strategy": ipc.strategy_to_dict(strategy), "granule_bytes": granule,
            "buffers": [{"key": list(k), "record": ipc._record_hex(_record(offset=0, bytes=n, allocation_bytes=n))}
                        for k, n in zip(bufs.keys, bufs.nbytes())], "misc": {"iteration": 7}}


def test_receive_validates_before_mapping():
    spec = small_llama2()
    p = _payload(spec, PS(8, 2, 1), 1 << 16)
    bad = dict(p, format="something-else")
    with pytest.raises(ValueError):
        ipc.receive_training_state(bad, device="cpu")
    short = dict(p, buffers=p["buffers"][:-1])
    with pytest.raises(ValueError):
        ipc.receive_training_state(short, device="cpu")
    other = dict(p, granule_bytes=1 << 15)
    with pytest.raises(ValueError):
        ipc.receive_training_state(other, device="cpu")
    with pytest.raises(ValueError):
        ipc.receive_training_state(p, device="cpu", space=build_virtual_model(tiny_llama2()))
    with pytest.raises(EOFError):
        ipc.receive_training_state(__import__("io").StringIO(""), device="cpu")
    assert _native.ipc_open_count() == 0


def test_release_notice_round_trip():
    import io

    buf = io.StringIO()
    ipc.notify_release(buf)
    assert ipc.wait_for_release(io.StringIO("noise\n" + buf.getvalue())) is True
    assert ipc.wait_for_release(io.StringIO("")) is False


def _fake_shared(layout, granule):
    """A received state's description without mappings (host-side planning only)."""
    bufs = GranuleBuffers(layout, granule)
    return ipc.SharedTrainingState(layout, bufs, [0x10000 * (i + 1) for i in range(len(bufs))], torch.device("cpu"))


def test_meta_manager_plans_then_attaches_a_received_state():
    """The reference's new process: build on meta, pre-build the switch, swap the received state in
    (tools/agent/env_utils.py:326-456).  Planning runs on the host; the launch needs a GPU."""
    spec = small_llama2()
    src, dst = PS(8, 2, 1), PS(8, 4, 1)
    mgr = ElasticMegatronManager([src, dst], spec, device="meta")
    assert mgr.training_state.device.type == "meta"
    assert mgr.reshard(dst, is_meta_device=True) is None
    state = _fake_shared(mgr.virtual_param_space.layout(src), 1 << 16)
    with pytest.raises(ValueError):
        mgr.attach_training_state(_fake_shared(mgr.virtual_param_space.layout(dst), 1 << 16))
    mgr.attach_training_state(state)
    assert mgr.training_state is state
    assert mgr.reshard(dst, is_meta_device=True) is None   # plans the granule switch
    plans = [p for k, p in mgr.transfer_manager._plans.items() if k[0] == "granules"]
    assert len(plans) == 1 and isinstance(plans[0], CompiledTensorPlan)
    assert len(plans[0].src) == len(state.buffers)


def test_meta_manager_refuses_a_real_switch_before_attach():
    mgr = ElasticMegatronManager([PS(8, 1, 1), PS(8, 2, 1)], small_llama2(), device="meta")
    with pytest.raises(RuntimeError):
        mgr.reshard(PS(8, 2, 1))


def test_attach_adopts_a_separately_built_model():
    spec = small_llama2()
    src, dst = PS(8, 1, 1), PS(6, 1, 1)
    mgr = ElasticMegatronManager([src, dst], spec, device="meta")
    other_space = build_virtual_model(spec)
    state = _fake_shared(other_space.layout(src), 1 << 18)
    mgr.attach_training_state(state)
    assert mgr.virtual_param_space is other_space
    assert mgr.reshard(dst, is_meta_device=True) is None


def test_group_zero_from_a_received_state_copies_the_params():
    """The exporter frees a received state's memory, bf16 params included, so a Group-ZeRO switch from
    it cannot leave them in place: its plan copies them into the new state's own granules."""
    spec = small_llama2()
    src, dst = PS(4, 1, 1), PS(8, 1, 1, num_distributed_optimizer_instances=2)
    mgr = ElasticMegatronManager([src, dst], spec, device="meta")
    state = _fake_shared(mgr.virtual_param_space.layout(src), 1 << 16)
    mgr.attach_training_state(state)
    assert mgr.reshard(dst, is_meta_device=True) is None
    plans = [(k, p) for k, p in mgr.transfer_manager._plans.items() if k[0] == "granules"]
    assert len(plans) == 1 and plans[0][0][5] == "backup_up_bf16"
    table = plans[0][1].segments
    param = set(state.buffers.granules_of(3))
    bf16 = table[np.isin(table["src_buf"], list(param))]
    assert len(bf16) and (bf16["elem_bytes"] == 2).all()
    stored = sum(h.hi - h.lo for vp in mgr.virtual_param_space.all_virtual_params
                 for h in state.layout.bf16_holders(vp))
    assert int((bf16["len"].astype(np.int64) * bf16["rows"]).sum()) == stored


def _owned_cpu(layout, granule, adopted=None, param=None):
    """An owned state's bookkeeping over host tensors (the ownership rules need no device)."""
    bufs = GranuleBuffers(layout, granule)
    held = {}
    for a, ts in enumerate(adopted or ()):
        held.update(zip(bufs.granules_of(a), ts))
    pg = list(bufs.granules_of(3))
    ts = [held[b] if b in held else param[b - pg[0]] if (param is not None and b in pg) else
          torch.zeros(n, dtype=torch.bfloat16 if a == 3 else torch.float32)
          for b, (a, n) in enumerate(zip(bufs.arena, bufs.numel))]
    return ipc.SharedTrainingState(layout, bufs, [t.data_ptr() for t in ts], torch.device("cpu"), ts)


def test_group_zero_new_state_takes_over_instance_0_granules():
    """A state built for a Group-ZeRO scale-up holds the old state's leading fp32 granules; once the
    old state hands them over, releasing it frees everything else and leaves them to the new one."""
    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(4, 1, 1)), space.layout(PS(8, 1, 1, num_distributed_optimizer_instances=2))
    g = 1 << 14
    n = adoptable_granules(ls, ld, g, "backup_up")
    assert n == ls.fp32_numel * 4 // g and n > 1
    assert adoptable_granules(ls, ld, g, "transfer") == 0
    old = _owned_cpu(ls, g)
    new = _owned_cpu(ld, g, old.leading_fp32_granules(n), [old.tensors[b] for b in old.buffers.granules_of(3)])
    assert held_granules(old, new) == n and shares_params(old, new)
    kept = [new.tensors[b] for a in range(3) for b in new.buffers.granules_of(a)[:n]]
    for i, t in enumerate(kept):
        t.fill_(float(i + 1))
    others = [old.tensors[b] for a in range(3) for b in old.buffers.granules_of(a)[n:]]
    old.hand_over(n)
    old.release_optimizer()
    assert all(t.untyped_storage().nbytes() == 0 for t in others)
    assert all(t.untyped_storage().nbytes() == t.numel() * 4 and bool((t == i + 1).all()) for i, t in enumerate(kept))
    ptrs, nbytes = old.buffer_ptrs(), old.buffer_bytes()
    assert all(ptrs[b] == 0 and nbytes[b] == 0 for a in range(3) for b in old.buffers.granules_of(a))
    with pytest.raises(ValueError):
        old.leading_fp32_granules(1)
    assert held_granules(old, new) == 0


def test_export_refuses_a_state_that_is_not_whole():
    """A released arena's granules are freed and handed-over ones belong to another state: exporting
    either would hand out memory this state no longer owns, so export refuses before any handle."""
    space = build_virtual_model(small_llama2())
    ls = space.layout(PS(4, 1, 1))
    for cut in ("release", "hand_over"):
        st = _owned_cpu(ls, 1 << 14)
        st.release_kind(1) if cut == "release" else st.hand_over(1)
        with pytest.raises(RuntimeError, match="only a whole state"):
            st.export()


def test_synthetic_fill_refuses_granules_the_state_no_longer_owns():
    """The synthetic fill and check address a state's granules through its own pointers and sizes:
    a released or handed-over granule has no bytes, so a piece there is refused on the host
    (OUT_OF_BOUNDS), where a whole state gets as far as looking for a device."""
    space = build_virtual_model(small_llama2())
    ls = space.layout(PS(4, 1, 1))
    for cut in (None, "release", "hand_over"):
        st = _owned_cpu(ls, 1 << 14)
        if cut == "release":
            st.release_kind(1)
        elif cut == "hand_over":
            st.hand_over(2)
        for a, pcs, ptrs, nb, _ in st._per_arena(ls.pieces()):
            if a != 1:
                continue
            with pytest.raises(_native.EmrsError) as e:
                _native.synth_fill(pcs, ptrs, nb, 1, 0)
            assert e.value.code == (-6 if cut is None else -2)
            break


def test_adoption_is_refused_where_it_cannot_hold():
    space = build_virtual_model(small_llama2())
    ls, ld = space.layout(PS(4, 1, 1)), space.layout(PS(8, 1, 1, num_distributed_optimizer_instances=2))
    tm = TransferManager()
    g = 1 << 14
    n = ls.fp32_numel * 4 // g
    with pytest.raises(ValueError):
        tm.compile_granules(ls, ld, g, g, "backup_up", adopt_granules=n + 1)   # past instance 0
    with pytest.raises(ValueError):
        tm.compile_granules(ls, ld, g, 2 * g, "backup_up", adopt_granules=1)   # two granule sizes
    with pytest.raises(ValueError):
        tm.compile_granules(ls, ld, g, g, "transfer", adopt_granules=1)       # not Group ZeRO
    with pytest.raises(RuntimeError):
        _fake_shared(ls, g).hand_over(1)                                        # not this process's memory
    plan = tm.compile_granules(ls, ld, g, g, "backup_up", adopt_granules=n)
    head = {b for a in range(3) for b in plan.dst.granules_of(a)[:n]}
    written = set(plan.dst_refs)
    assert not head & written and set(range(3 * len(plan.dst.granules_of(0)))) - head <= written


def test_manager_plans_the_adopting_switch_for_an_owned_shared_state():
    """Group ZeRO from a shared state this process owns and releases: the plan leaves the adoptable
    head in place.  Without release_source the old state must stay whole, so nothing is taken over."""
    spec = small_llama2()
    src, dst = PS(4, 1, 1), PS(8, 1, 1, num_distributed_optimizer_instances=2)
    g = 1 << 14
    for release, want in ((True, True), (False, False)):
        mgr = ElasticMegatronManager([src, dst], spec, device="meta", share_granule_bytes=g, release_source=release)
        state = _owned_cpu(mgr.virtual_param_space.layout(src), g)
        mgr.attach_training_state(state)
        assert mgr.reshard(dst, is_meta_device=True) is None
        keys = [k for k in mgr.transfer_manager._plans if k[0] == "granules"]
        assert len(keys) == 1 and keys[0][5] == "backup_up"
        assert (keys[0][-1] == state.layout.fp32_numel * 4 // g) is want and (keys[0][-1] == 0) is not want


def test_staged_manager_plans_between_shared_states():
    """low_memory with share_granule_bytes: the three staged plans are re-based onto granules of one
    size on both sides, and a released arena's granules are allocated again, one arena at a time."""
    spec = small_llama2()
    src, dst, g = PS(8, 2, 1), PS(8, 4, 1), 1 << 16
    mgr = ElasticMegatronManager([src, dst], spec, device="meta", low_memory=True, share_granule_bytes=g)
    state = _owned_cpu(mgr.virtual_param_space.layout(src), g)
    mgr.attach_training_state(state)
    assert mgr.reshard(dst, is_meta_device=True) is None
    staged = [(k, p) for k, p in mgr.transfer_manager._plans.items() if k[0] == "staged-granules"]
    assert len(staged) == 1 and staged[0][0][-2:] == (g, g) and len(staged[0][1]) == 3
    before = state.buffer_bytes()
    state.release_kind(1)
    assert all(state.buffer_bytes()[b] == 0 for b in state.buffers.granules_of(1))
    state.allocate_kind(1)
    assert state.buffer_bytes() == before and all(state.buffer_ptrs()[b] for b in state.buffers.granules_of(1))
    with pytest.raises(RuntimeError):
        _fake_shared(state.layout, g).allocate_kind(0)       # another process's memory


def test_arena_release_protocol():
    """A staged switch from a received state releases the source arena by arena: the importer's
    notice names the arena, the exporter frees it and answers, and the final notice ends the wait."""
    import io

    to_exporter, to_importer = io.StringIO(), io.StringIO()
    to_importer.write("noise\n")
    ipc.notify_freed(to_importer, "main")
    ipc.notify_freed(to_importer, "exp_avg")
    to_importer.seek(0)
    hook = ipc.release_hook(to_exporter, to_importer)
    hook(0)
    hook(1)
    with pytest.raises(RuntimeError):
        hook(2)                      # the exporter never answered: the channel ended
    ipc.notify_release(to_exporter)
    freed = []
    assert ipc.wait_for_release(io.StringIO(to_exporter.getvalue()), on_arena=freed.append) is True
    assert freed == ["main", "exp_avg", "exp_avg_sq"]
    # Only fp32 arenas are released one at a time.
    assert ipc.wait_for_release(io.StringIO("released param\nreleased\n"), on_arena=freed.append) is True
    assert freed == ["main", "exp_avg", "exp_avg_sq"]


def test_staged_manager_accepts_a_received_state():
    """low_memory with a received source: the staged plans are re-based onto its granules."""
    spec = small_llama2()
    src, dst = PS(8, 2, 1), PS(8, 4, 1)
    mgr = ElasticMegatronManager([src, dst], spec, device="meta", low_memory=True)
    state = _fake_shared(mgr.virtual_param_space.layout(src), 1 << 16)
    mgr.attach_training_state(state)
    assert mgr.reshard(dst, is_meta_device=True) is None
    staged = [p for k, p in mgr.transfer_manager._plans.items() if k[0] == "staged-granules"]
    assert len(staged) == 1 and len(staged[0]) == 3
    assert all(isinstance(p, CompiledTensorPlan) and len(p.src) == len(state.buffers) for p in staged[0])
