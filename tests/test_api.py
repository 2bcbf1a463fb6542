"""The public API mirrors the reference's (elastic_manager.py:30-265) and fails loudly without a GPU."""

import pytest
import torch

from elasticmegatron_amd import ElasticMegatronManager, ParallelStrategy, TrainingState, tiny_llama2
from elasticmegatron_amd import _native
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model

SEQ = [dict(world_size=8, tensor_model_parallel_size=2, pipeline_model_parallel_size=1),
       dict(world_size=8, tensor_model_parallel_size=1, pipeline_model_parallel_size=1),
       dict(world_size=8, tensor_model_parallel_size=4, pipeline_model_parallel_size=1)]


def test_meta_device_reshard_plans_without_touching_memory():
    mgr = ElasticMegatronManager(SEQ, tiny_llama2(), device="cpu")
    state = mgr.training_state
    assert mgr.reshard(SEQ[1], is_meta_device=True) is None
    assert mgr.training_state is state  # nothing switched
    # The plan is cached for the real switch.
    assert len(mgr.transfer_manager._plans) == 1
    plan = next(iter(mgr.transfer_manager._plans.values()))
    assert plan.payload_bytes == 14 * tiny_llama2().num_params()
    with pytest.raises(AssertionError):
        mgr.reshard(SEQ[1], is_meta_device=True, save_ckpt=True)
    with pytest.raises(NotImplementedError):
        mgr.reshard(SEQ[1], save_ckpt=True)


def test_clear_meta_state_drops_the_prebuilt_plans():
    """elastic_manager.py:180-187: a meta-device pre-build is forgotten; the live strategy is not a meta state."""
    mgr = ElasticMegatronManager(SEQ, tiny_llama2(), device="cpu")
    mgr.reshard(SEQ[1], is_meta_device=True)
    mgr.reshard(SEQ[2], is_meta_device=True)
    assert len(mgr.transfer_manager._plans) == 2
    assert mgr.clear_meta_state(SEQ[1]) == 1
    assert len(mgr.transfer_manager._plans) == 1   # the pre-build for SEQ[2] stays
    assert mgr.clear_meta_state(SEQ[1]) == 0
    with pytest.raises(AssertionError):
        mgr.clear_meta_state(SEQ[0])
    assert mgr.transfer_manager.evict() == 1 and not mgr.transfer_manager._plans


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the behaviour without a GPU")
def test_reshard_without_gpu_raises():
    mgr = ElasticMegatronManager(SEQ, tiny_llama2(), device="cpu")
    with pytest.raises(RuntimeError, match="no CPU path"):
        mgr.reshard(SEQ[1])
    # The C ABI itself refuses to run without a device.
    plan = next(iter(mgr.transfer_manager._plans.values()))
    src = mgr.training_state
    dst = TrainingState.allocate(mgr.virtual_param_space.layout(ParallelStrategy(**SEQ[1])), "cpu")
    with pytest.raises(_native.EmrsError) as e:
        plan.native.execute(src.arena_ptrs(), dst.arena_ptrs(), 0)
    assert e.value.code == -6  # EMRS_ERR_NO_DEVICE


def test_training_state_views():
    spec = tiny_llama2()
    space = build_virtual_model(spec)
    lay = space.layout(ParallelStrategy(8, 2, 1))
    st = TrainingState.allocate(lay, "cpu")
    vp = space.all_virtual_params[3]  # layer 0 linear_qkv.weight, TP dim 0
    shapes = []
    for g in range(8):
        info = st.optimizer_tensor_info(vp, g)
        if info is not None:
            assert info.main_weight.numel() == info.optimizer_tensor_range_in_model_param.size
            assert info.model_param_shape == (768, 512)
            shapes.append(info.main_weight.numel())
    assert sum(shapes) == 2 * 768 * 512  # two TP ranks, each split over its DP ranks
    assert st.model_param(vp, 1).shape == (768, 512)


def test_strategy_list_and_redundant_backup_dispatch():
    spec = tiny_llama2()
    mgr = ElasticMegatronManager([dict(world_size=6, tensor_model_parallel_size=1, pipeline_model_parallel_size=1)],
                                 spec, device="cpu")
    assert mgr.reshard(dict(world_size=12, tensor_model_parallel_size=1, pipeline_model_parallel_size=1,
                            num_distributed_optimizer_instances=2), is_meta_device=True) is None
    (key, plan), = mgr.transfer_manager._plans.items()
    assert "backup_up" in key and plan.payload_bytes == 24 * spec.num_params()
    with pytest.raises(ValueError):  # the reference rejects a reshard inside a Group-ZeRO layout
        ParallelStrategy.is_redundant_backup(ParallelStrategy(12, 1, 1, num_distributed_optimizer_instances=2),
                                             ParallelStrategy(12, 1, 1, num_distributed_optimizer_instances=2))


def test_manager_adopts_a_given_state():
    """A state laid out elsewhere for the same model is adopted with its virtual model; another model's is refused."""
    spec = tiny_llama2()
    lay = build_virtual_model(spec).layout(ParallelStrategy(**SEQ[0]))
    st = TrainingState.allocate(lay, "cpu")
    mgr = ElasticMegatronManager(SEQ, spec, training_state=st)
    assert mgr.virtual_param_space is lay.space
    assert mgr.space_for(ParallelStrategy(**SEQ[2])) is lay.space
    assert mgr.reshard(SEQ[1], is_meta_device=True) is None
    with pytest.raises(ValueError):
        ElasticMegatronManager(SEQ[1:], spec, training_state=st)   # not the first strategy
    other = TrainingState.allocate(build_virtual_model(spec.with_padded_vocab(32256)).layout(
        ParallelStrategy(**SEQ[0])), "cpu")
    with pytest.raises(ValueError):
        ElasticMegatronManager(SEQ, spec, training_state=other)


def test_reshard_releases_the_source_state(monkeypatch):
    """After a switch only the new state holds optimizer memory (training_state.py:313-315), with or without
    verification.  The device calls are stubbed: this checks the host-side ownership only."""
    import gc
    import weakref

    from elasticmegatron_amd.transfer.transfer import TransferManager
    from elasticmegatron_amd.transfer.verify import VerifyReport

    monkeypatch.setattr(TransferManager, "execute", lambda self, plan, src, dst, stream=None: None)
    monkeypatch.setattr(TransferManager, "verify", lambda self, src, dst, kind="transfer", include_bf16=True,
                        stream=None, **kw: VerifyReport({}))
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    mgr = ElasticMegatronManager(SEQ, tiny_llama2(), device="cpu")
    arenas = [weakref.ref(mgr.training_state.main)]
    for i, s in enumerate(SEQ[1:] + SEQ[:1] + SEQ[1:]):
        mgr.reshard(s, verify=bool(i % 2))
        arenas.append(weakref.ref(mgr.training_state.main))
        gc.collect()
        alive = [r for r in arenas if r() is not None and r().numel() > 0]
        assert len(alive) == 1 and alive[0]() is mgr.training_state.main
    keep = ElasticMegatronManager(SEQ, tiny_llama2(), device="cpu", release_source=False)
    first = keep.training_state
    keep.reshard(SEQ[1])
    assert first.main.numel() > 0


def test_reference_constructor_arguments_are_accepted():
    """TransferManager(send_fn, recv_fn, broadcast_fn) and the manager's transport arguments, as the
    reference takes them (transfer.py:23-34, elastic_manager.py:41-82)."""
    from elasticmegatron_amd.transfer.transfer import TransferManager

    calls = []
    send = lambda t, dst: calls.append(("send", dst))  # noqa: E731
    recv = lambda t, src: calls.append(("recv", src))  # noqa: E731
    tm = TransferManager(send, recv, None)
    assert tm.send_fn is send and tm.recv_fn is recv and tm.broadcast_fn is None
    mgr = ElasticMegatronManager(SEQ, tiny_llama2(), device="cpu", send_fn=send, recv_fn=recv,
                                 broadcast_fn=None, use_p2p_to_collective=False)
    assert mgr.transfer_manager.send_fn is send
    assert mgr.reshard(SEQ[1], is_meta_device=True) is None
    assert calls == []   # one device: every hop is a local copy inside the plan
    with pytest.raises(ValueError):
        TransferManager(bf16_source="fp8")


def test_execute_refuses_states_of_another_model(monkeypatch):
    """A plan runs only on arenas at least as large as those it was built for (no device access otherwise)."""
    from dataclasses import replace

    from elasticmegatron_amd.transfer.transfer import TransferManager
    from tests.helpers import small_llama3

    spec = replace(small_llama3(), vocab_size=2300)
    big = build_virtual_model(spec.with_padded_vocab(2560))
    small = build_virtual_model(spec.with_padded_vocab(2304))
    s, d = ParallelStrategy(8, 4, 1), ParallelStrategy(8, 2, 1)
    tm = TransferManager()
    plan = tm.compile(big.layout(s), big.layout(d))
    a = TrainingState.allocate(small.layout(s), "cpu")
    b = TrainingState.allocate(small.layout(d), "cpu")
    # Pretend the states are on a GPU: the size check comes before any device work.
    monkeypatch.setattr(TrainingState, "device", property(lambda self: torch.device("cuda", 0)))
    with pytest.raises(ValueError, match="another model"):
        tm.execute(plan, a, b)


def test_execute_tensors_checks_bytes():
    from elasticmegatron_amd.transfer.transfer import TransferManager

    space = build_virtual_model(tiny_llama2())
    tm = TransferManager()
    tp = tm.compile_tensors(space.layout(ParallelStrategy(**SEQ[0])), space.layout(ParallelStrategy(**SEQ[1])))
    src = [torch.empty(n, dtype=torch.float32 if k[0] != "param" else torch.bfloat16) for n, k in
           zip(tp.src.numel, tp.src.keys)]
    dst = [torch.empty(n, dtype=torch.int8) for n in tp.dst.numel]   # right numel, too few bytes
    with pytest.raises(ValueError, match="bytes"):
        tm.execute_tensors(tp, src, dst)


@pytest.mark.parametrize("repad,padded,vocab", [(False, 768, 700), (True, 512, 500)])
def test_non_power_of_two_tp_is_refused_on_every_path(repad, padded, vocab):
    """resharding_tp.py:98-99: TP sizes must be powers of two, also when the vocabulary is re-padded
    (500 pads to 512 at TP1 and 768 at TP3: a switch between two model spaces, which does not go
    through register_reshard)."""
    from elasticmegatron_amd.resharding.model_spec import ModelSpec

    spec = ModelSpec(name="tp3", num_layers=2, hidden_size=384, num_attention_heads=6, kv_channels=64,
                     ffn_hidden_size=768, padded_vocab_size=padded, vocab_size=vocab)
    mgr = ElasticMegatronManager([dict(world_size=6, tensor_model_parallel_size=1, pipeline_model_parallel_size=1),
                                  dict(world_size=6, tensor_model_parallel_size=3, pipeline_model_parallel_size=1)],
                                 spec, device="cpu", repad_vocab=repad)
    with pytest.raises(AssertionError, match="powers of two"):
        mgr.reshard(dict(world_size=6, tensor_model_parallel_size=3, pipeline_model_parallel_size=1),
                    is_meta_device=True)


@pytest.mark.gpu
def test_space_does_not_keep_states_alive(gpu_device):
    """The virtual model outlives a switch; it must not hold the states of the last transfer."""
    import weakref

    mgr = ElasticMegatronManager(SEQ, tiny_llama2(), device=gpu_device)
    old = weakref.ref(mgr.training_state)
    mgr.reshard(SEQ[1])
    space = mgr.virtual_param_space
    assert space.src_state is None and space.dst_state is None
    import gc

    gc.collect()
    assert old() is None


def test_dict_strategies_share_the_cached_plan():
    """A strategy passed as a dict, or with only sequence_parallel changed, is the same strategy
    (parallel_strategy.py:223-232): the plan a meta-device reshard built is the one reused."""
    listed = [ParallelStrategy(8, 2, 1, sequence_parallel=False), ParallelStrategy(8, 4, 1)]
    mgr = ElasticMegatronManager(listed, tiny_llama2(), device="cpu")
    assert mgr.reshard(dict(world_size=8, tensor_model_parallel_size=4, pipeline_model_parallel_size=1),
                       is_meta_device=True) is None
    assert len(mgr.transfer_manager._plans) == 1
    plan = next(iter(mgr.transfer_manager._plans.values()))
    mgr.reshard(ParallelStrategy(8, 4, 1, sequence_parallel=False), is_meta_device=True)
    mgr.reshard(listed[1], is_meta_device=True)
    assert len(mgr.transfer_manager._plans) == 1
    assert next(iter(mgr.transfer_manager._plans.values())) is plan
    # A state laid out for the dict form of the first strategy is adopted as its state.
    state = TrainingState.allocate(mgr.virtual_param_space.layout(ParallelStrategy(8, 2, 1)), "cpu")
    ElasticMegatronManager([dict(world_size=8, tensor_model_parallel_size=2, pipeline_model_parallel_size=1,
                                 sequence_parallel=False)], tiny_llama2(), training_state=state)


def test_block_and_print_keeps_the_reference_signature():
    """transfer_optimizer_tensors(space, use_block_and_print) as the reference declares it
    (transfer.py:291-293); the dump lists every registered parameter's global send and receive
    ranges, one line per (source rank, destination rank) pair of its plan."""
    import inspect

    from elasticmegatron_amd.resharding.model_spec import tiny_llama2
    from elasticmegatron_amd.transfer.transfer import TransferManager, plan_dump

    params = list(inspect.signature(TransferManager.transfer_optimizer_tensors).parameters)
    assert params[:3] == ["self", "virtual_param_space", "use_block_and_print"]
    space = build_virtual_model(tiny_llama2())
    src, dst = ParallelStrategy(8, 2, 1), ParallelStrategy(8, 4, 1)
    space.register_reshard(src, dst)
    text = plan_dump(space).splitlines()
    heads = [l for l in text if l.startswith("[reshard plan]")]
    assert len(heads) == len(space.all_virtual_params)
    sends = sum(len(d) for vp in space.all_virtual_params for d in vp.reshard_plan.global_send_info.values())
    recvs = sum(len(d) for vp in space.all_virtual_params for d in vp.reshard_plan.global_recv_info.values())
    assert sum(l.startswith("  send") for l in text) == sends > 0
    assert sum(l.startswith("  recv") for l in text) == recvs > 0


def test_fake_transfer_plans_without_moving_data():
    """set_fake_transfer(fake_transfer) under the reference's argument name (transfer.py:32-34):
    with it set a transfer plans, caches the plan and returns before touching either state, so it
    runs on CPU states too; cleared, the same call refuses them."""
    from elasticmegatron_amd.transfer.transfer import TransferManager

    space = build_virtual_model(tiny_llama2())
    s, d = ParallelStrategy(8, 1, 1), ParallelStrategy(8, 2, 1)
    src, dst = TrainingState.allocate(space.layout(s), "cpu"), TrainingState.allocate(space.layout(d), "cpu")
    src.main.fill_(1.0)
    dst.main.zero_()
    tm = TransferManager()
    tm.set_fake_transfer(fake_transfer=True)
    plan = tm.transfer_optimizer_tensors(space, src=src, dst=dst)
    assert plan.payload_bytes > 0 and tm.compile(src.layout, dst.layout) is plan
    assert int(dst.main.count_nonzero()) == 0
    tm.set_fake_transfer(False)
    with pytest.raises(RuntimeError, match="GPU memory"):
        tm.transfer_optimizer_tensors(space, src=src, dst=dst)


def test_manager_transfer_methods_keep_the_reference_argument_order():
    """transfer_params(src, dst, union_world_group, is_meta_device), redundant_backup(src, dst,
    is_scale_up, is_meta_device) and log_communication_info(transfer_time, union_world_group,
    logger) in the reference's order (elastic_manager.py:106-178).  With ``is_meta_device`` both
    transfers only plan, so CPU states pass through untouched and the fake flag is restored."""
    import logging

    mgr = ElasticMegatronManager(SEQ, tiny_llama2(), device="cpu")
    space = mgr.virtual_param_space
    src = mgr.training_state
    dst = TrainingState.allocate(space.layout(ParallelStrategy(**SEQ[1])), "cpu")
    src.main.fill_(1.0)
    dst.main.zero_()
    assert mgr.transfer_params(src, dst, None, True) >= 0.0
    assert int(dst.main.count_nonzero()) == 0 and mgr.transfer_manager.fake_transfer is False
    with pytest.raises(RuntimeError, match="GPU memory"):
        mgr.transfer_params(src, dst, None, False)
    assert mgr.transfer_manager.fake_transfer is False
    s, d = ParallelStrategy(8, 1, 1, num_distributed_optimizer_instances=2), ParallelStrategy(4, 1, 1)
    a, b = TrainingState.allocate(space.layout(s), "cpu"), TrainingState.allocate(space.layout(d), "cpu")
    assert mgr.redundant_backup(a, b, False, True) >= 0.0
    seen = []

    class Keep(logging.Handler):
        def emit(self, record):
            seen.append(record.getMessage())

    log = logging.getLogger("emrs-test-perf-line")
    log.addHandler(Keep())
    log.setLevel(logging.INFO)
    msg = mgr.log_communication_info(12.5, None, log)
    assert seen == [msg] and msg.startswith("[ElasticMegatron-Perf] : transfer time: 12.50 ms")


def test_prepare_needs_a_gpu_and_meta_reshard_on_cpu_skips_it():
    """TransferManager.prepare refuses a CPU device (no CPU path); a meta-device reshard of CPU
    states plans without preparing anything."""
    from elasticmegatron_amd.transfer.transfer import TransferManager

    space = build_virtual_model(tiny_llama2())
    ls, ld = space.layout(ParallelStrategy(8, 2, 1)), space.layout(ParallelStrategy(8, 1, 1))
    tm = TransferManager()
    with pytest.raises(RuntimeError, match="GPU"):
        tm.prepare(tm.compile(ls, ld), "cpu")
    mgr = ElasticMegatronManager(SEQ, tiny_llama2(), device="cpu", low_memory=True)
    assert mgr.reshard(SEQ[1], is_meta_device=True) is None
