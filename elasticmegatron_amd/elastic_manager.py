"""Public façade: ``ElasticMegatronManager.reshard(new_parallel_strategy=...)``.

Mirrors elastic_megatron/elastic_manager.py:30-265.  The reference's manager
wraps a live Megatron model, optimizer and process groups; this one wraps a
:class:`~.megatron_manager.training_state.TrainingState` holding every rank's
state on one device.  ``reshard`` keeps the reference's control flow:

1. pick the destination strategy (elastic_manager.py:189-258);
2. Group-ZeRO instance switches take the redundant-backup path, everything
   else plans and transfers (elastic_manager.py:106-141,
   parallel_strategy.py:234-263);
3. the transfer is timed with a device-synchronised timer around the executor
   only (elastic_manager.py:119-120);
4. the source optimizer state is released and the perf line is logged in the
   reference's format (elastic_manager.py:158-178).

Process-group rebuild, learning-rate broadcast and dataloader rebuild have no
counterpart on one device and are not performed.

The padded vocabulary stays fixed across switches, as in the reference
(virtual_param.py:480-481).  With ``repad_vocab=True`` it follows Megatron's
padding rule for each strategy's TP size instead: the true vocabulary rows
are carried over and new padding rows are zero in all four tensors.
"""

from __future__ import annotations

import logging
from typing import Callable, Dict, List, Optional, Union

import torch

from .megatron_manager.parallel_strategy import ParallelStrategy
from .megatron_manager.training_state import ARENA_GRANULE_BYTES, TrainingState
from .resharding.model_spec import ModelSpec
from .resharding.util import Timer
from .resharding.virtual_param import VirtualParamSpace, build_virtual_model
from .transfer.ipc_manager import SharedTrainingState
from .transfer.transfer import BACKUP_KINDS, TransferManager, _granule_of, backup_kind, held_granules, shares_params
from .transfer.verify import merge_stats, report_from_stats

StrategyLike = Union[ParallelStrategy, Dict[str, int]]


def _as_strategy(s: StrategyLike) -> ParallelStrategy:
    return s if isinstance(s, ParallelStrategy) else ParallelStrategy(**s)


class ElasticMegatronManager:
    def __init__(self, parallel_strategy_list: List[StrategyLike], model_spec: ModelSpec,
                 training_state: Optional[TrainingState] = None, device=None,
                 release_source: bool = True, repad_vocab: bool = False,
                 send_fn: Optional[Callable] = None, recv_fn: Optional[Callable] = None,
                 broadcast_fn: Optional[Callable] = None, use_p2p_to_collective: bool = True,
                 low_memory: bool = False, share_granule_bytes: Optional[int] = None):
        """``model_spec`` and ``training_state`` stand in for the reference's live Megatron
        ``model`` / ``optimizer`` (elastic_manager.py:41-82).  ``send_fn``, ``recv_fn``,
        ``broadcast_fn`` and ``use_p2p_to_collective`` are accepted as the reference accepts
        them and handed to the TransferManager; on one device no message is sent.

        ``low_memory=True`` runs each switch in three stages, one optimizer kind at a time: the
        destination arena of a kind is allocated just before its stage and, with
        ``release_source``, the source arena is released right after it, as the reference releases
        every optimizer tensor once it is sent.  The peak is the source state plus one fp32 arena
        and the bf16 params of the destination, instead of both whole states.  The fp32 arenas are
        then allocated in 1 GiB granules, so that the memory a released source arena leaves serves
        the next destination arena without a call to the driver (a state passed in
        ``training_state`` should be allocated with ``granule_bytes=ARENA_GRANULE_BYTES`` too).
        The source may be a state received from another process: each of its fp32 arenas is
        unmapped after its stage, and the state's ``on_release`` hook
        (:func:`~.transfer.ipc_manager.release_hook`) has the exporting process free that arena
        before the next stage allocates.

        ``share_granule_bytes``: the states this manager allocates are
        :class:`~.transfer.ipc_manager.SharedTrainingState` objects with granules of that size, so that the
        live state can be handed to another process at any time (``send_training_state``).  A
        ``training_state`` passed in may be one as well, for instance one just received from the
        process that held it (``receive_training_state``).  ``device="meta"`` allocates nothing: the
        manager plans (``reshard(..., is_meta_device=True)``) until :meth:`attach_training_state`
        hands it the real state, as the reference builds its new process on the meta device first.
        A Group-ZeRO switch from such a state that this process owns and releases
        (``release_source``) leaves instance 0 where it is: the new state takes over the old one's
        leading granules of every fp32 arena (all of instance 0 with PP = 1) instead of copying
        them, so a scale-up to two instances moves two thirds of the bytes, a scale-down almost
        none, and the peak memory drops by the granules taken over.  With ``low_memory`` too, each
        switch is staged between such states: a destination arena's granules are allocated just
        before its stage, from the source granules the previous stage released (nothing is taken
        over in a staged switch).
        """
        if not parallel_strategy_list:
            raise ValueError("parallel_strategy_list is empty")
        if repad_vocab and model_spec.vocab_size is None:
            raise ValueError("repad_vocab needs model_spec.vocab_size")
        self.parallel_strategy_list = [_as_strategy(s) for s in parallel_strategy_list]
        self.model_spec = model_spec
        self.repad_vocab = repad_vocab
        self._spaces: Dict[int, VirtualParamSpace] = {}
        cur = self.parallel_strategy_list[0]
        if training_state is not None:
            if training_state.parallel_strategy != cur:
                raise ValueError("training_state does not use the first strategy of the list")
            # Adopt the state's virtual model when it is the model this manager would build.
            spec = training_state.layout.space.spec
            if spec != self._spec_for(cur):
                raise ValueError("training_state was laid out for another model")
            self._spaces[spec.padded_vocab_size] = training_state.layout.space
        for s in self.parallel_strategy_list:
            self.space_for(s).build_model_virtual_params(s)
        self.transfer_manager = TransferManager(send_fn, recv_fn, broadcast_fn)
        self.use_p2p_to_collective = use_p2p_to_collective
        self.release_source = release_source
        self.low_memory = low_memory
        self.share_granule_bytes = share_granule_bytes
        self.last_stage_ms: List[Dict[str, float]] = []   # staged switches: per stage, allocate / execute ms
        self.last_transfer_ms = 0.0
        self.last_verification = None
        if training_state is None:
            training_state = self._allocate(self.space_for(cur).layout(cur), device)
        self.training_state = training_state

    def _allocate(self, layout, device, param=None, adopted=None):
        """A new state of ``layout`` of the kind this manager keeps (nothing on the meta device);
        ``adopted``: leading fp32 granules of the old state it takes over (shared states only)."""
        meta = device is not None and torch.device(device).type == "meta"
        if self.share_granule_bytes is not None and not meta:
            return SharedTrainingState.allocate(layout, device, self.share_granule_bytes, param_granules=param,
                                                adopted=adopted)
        if adopted is not None:
            raise AssertionError("only a shared state takes over granules")
        return TrainingState.allocate(layout, device, param=param,
                                      granule_bytes=ARENA_GRANULE_BYTES if self.low_memory else 0)

    def attach_training_state(self, state) -> None:
        """Make ``state`` the live state: the state a meta-device manager was planning for, now
        backed by memory, such as one received from the process that held it.  The reference swaps
        the tensors it received into the optimizer of its meta-built model the same way
        (tools/agent/env_utils.py:423-433).  It must use the current strategy and model."""
        if state.parallel_strategy != self.training_state.parallel_strategy:
            raise ValueError("the state does not use the manager's current strategy")
        spec = state.layout.space.spec
        if spec != self._spec_for(state.parallel_strategy):
            raise ValueError("the state was laid out for another model")
        space = state.layout.space
        if space is not self._spaces.get(spec.padded_vocab_size):
            # Adopt the state's virtual model, built for every strategy of the list it serves.
            self._spaces[spec.padded_vocab_size] = space
            for s in self.parallel_strategy_list:
                if self._spec_for(s).padded_vocab_size == spec.padded_vocab_size:
                    space.build_model_virtual_params(s)
        self.training_state = state

    def _spec_for(self, strategy: ParallelStrategy) -> ModelSpec:
        pv = (self.model_spec.padded_vocab_for_tp(strategy.tensor_model_parallel_size) if self.repad_vocab
              else self.model_spec.padded_vocab_size)
        return self.model_spec if pv == self.model_spec.padded_vocab_size else self.model_spec.with_padded_vocab(pv)

    def space_for(self, strategy: ParallelStrategy) -> VirtualParamSpace:
        """The virtual model a strategy's state is laid out in (one per padded vocabulary size)."""
        spec = self._spec_for(strategy)
        space = self._spaces.get(spec.padded_vocab_size)
        if space is None:
            space = self._spaces[spec.padded_vocab_size] = build_virtual_model(spec)
        return space

    @property
    def virtual_param_space(self) -> VirtualParamSpace:
        """The virtual model of the current state."""
        return self.training_state.layout.space

    @property
    def parallel_strategy(self) -> ParallelStrategy:
        return self.training_state.parallel_strategy

    def _prepare(self, plan, state) -> None:
        """The meta-device pass's upload of a plan's tables, on the state's GPU (none elsewhere)."""
        if state.device.type == "cuda":
            self.transfer_manager.prepare(plan, state.device)

    def transfer_params(self, src: TrainingState, dst: TrainingState, union_world_group=None,
                        is_meta_device: bool = False) -> float:
        """Plan (cached) and move the state; returns the executor's time in ms.

        The arguments keep the reference's order (elastic_manager.py:106-122).  One process holds
        every rank's state, so ``union_world_group`` is accepted and unused; ``is_meta_device``
        plans, caches and uploads the plan's tables to the state's GPU without moving data, as the
        reference's fake transfer builds its connections (elastic_manager.py:115-117, 282-285).
        """
        space = src.layout.space
        if space is dst.layout.space:
            space.register_reshard(src.parallel_strategy, dst.parallel_strategy)
        gs, gd = _granule_of(src), _granule_of(dst)
        if gs is not None or gd is not None:   # shared granules: the re-based plan
            plan = self.transfer_manager.compile_granules(src.layout, dst.layout, gs, gd)
            if is_meta_device:
                self._prepare(plan, src)
            with Timer() as t:
                if not is_meta_device:
                    self.transfer_manager.execute_states(plan, src, dst)
            return t.elapsed
        plan = self.transfer_manager.compile(src.layout, dst.layout)
        if is_meta_device:
            self._prepare(plan, src)
        # The states are the space's for the duration of the transfer only: the space outlives the
        # switch, and holding them would keep a released state's memory alive.
        space.src_state, space.dst_state = src, dst
        fake = self.transfer_manager.fake_transfer
        try:
            if is_meta_device:
                self.transfer_manager.set_fake_transfer(True)
            with Timer() as t:
                self.transfer_manager.transfer_optimizer_tensors(space)
        finally:
            space.src_state = space.dst_state = None
            self.transfer_manager.set_fake_transfer(fake)
        return t.elapsed

    def transfer_staged(self, src: TrainingState, dst: TrainingState, kind: str = "transfer",
                        verify: bool = False, *, lost_ranks=()):
        """The switch in three launches, one optimizer kind at a time (see ``low_memory``).

        ``dst`` may start without fp32 arenas; each is allocated just before its stage.  With
        ``release_source`` the source arena of each kind is released right after its stage, once
        it has been checked when ``verify`` is set.  ``src`` may be held in granules (a shared or
        received state).  Returns (ms of the stages' allocation, launch and release, summed;
        verification records or None); ``last_stage_ms`` has each stage's three times.
        ``lost_ranks``: as for :meth:`reshard`.
        """
        if kind == "transfer" and src.layout.space is dst.layout.space:
            src.layout.space.register_reshard(src.parallel_strategy, dst.parallel_strategy)
        stages = self.transfer_manager.staged_for_states(src.layout, dst.layout, _granule_of(src), _granule_of(dst),
                                                         kind, lost_ranks=lost_ranks)
        elapsed, stats, names = 0.0, None, None
        self.last_stage_ms = []
        for k, plan in enumerate(stages):
            with Timer() as ta:
                dst.allocate_kind(k)
            with Timer() as te:
                self.transfer_manager.execute_states(plan, src, dst)
            elapsed += ta.elapsed + te.elapsed
            self.last_stage_ms.append({"allocate": ta.elapsed, "execute": te.elapsed})
            if verify:
                part, names = self.transfer_manager.verify_stats(src, dst, kind, stage=k, lost_ranks=lost_ranks)
                stats = merge_stats(stats, part)
                if int(part["mismatches"].sum()):
                    # Stop before this stage's source is released; earlier stages were checked.
                    raise RuntimeError(f"reshard verification failed in stage {k} "
                                       f"({('main', 'exp_avg', 'exp_avg_sq')[k]}): "
                                       + "\n".join(report_from_stats(stats, names).lines()[:20]))
            with Timer() as tr:
                if self.release_source:
                    src.release_kind(k)
            elapsed += tr.elapsed
            self.last_stage_ms[-1]["release"] = tr.elapsed
        return elapsed, (stats, names) if verify else None

    def redundant_backup(self, src: TrainingState, dst: TrainingState, is_scale_up: bool,
                         is_meta_device: bool = False, *, lost_ranks=()) -> float:
        """Group-ZeRO switch in the reference's argument order (elastic_manager.py:124-142);
        ``is_meta_device`` plans, caches and uploads the plan's tables without moving data.  The
        bf16 params stay where they are when ``dst`` shares ``src``'s, and are copied otherwise;
        the leading fp32 granules that ``dst`` holds in ``src``'s memory are left in place.
        ``lost_ranks``: as for :meth:`reshard`.  Returns the executor's ms."""
        kind = backup_kind(is_scale_up, not shares_params(src, dst))
        plan = self.transfer_manager.plan_for_states(src.layout, dst.layout, _granule_of(src), _granule_of(dst), kind,
                                                     adopt_granules=held_granules(src, dst), lost_ranks=lost_ranks)
        if is_meta_device:
            self._prepare(plan, src)
        with Timer() as t:
            if not is_meta_device:
                self.transfer_manager.execute_states(plan, src, dst)
        return t.elapsed

    def _adoptable(self, src_state, dst_layout, kind: str, dst_granule_bytes, param, lost_ranks=()) -> int:
        """Leading fp32 granules that the new state of a Group-ZeRO switch takes over from the old
        one: only from a shared state this process owns and the switch releases, into granules of
        the same size, with the bf16 params shared too, in a whole (not staged) switch, and only
        granules that end before the first lost rank's state."""
        if kind not in BACKUP_KINDS or param is None or not self.release_source or self.low_memory:
            return 0
        if not isinstance(src_state, SharedTrainingState) or src_state.imported \
                or src_state.granule_bytes != dst_granule_bytes:
            return 0
        return self.transfer_manager.adoptable(src_state.layout, dst_layout, dst_granule_bytes, kind,
                                               lost_ranks=lost_ranks)

    @staticmethod
    def _carried_params(src_state, dst_granule_bytes):
        """The bf16 params a Group-ZeRO switch carries over unchanged: the source's own param arena
        (or granules), which the new state shares.  None when the new state cannot share them: the
        source was received from another process, which frees it, or the two states are held
        differently (arenas and granules, or granules of two sizes); the switch then copies them."""
        if isinstance(src_state, TrainingState) and dst_granule_bytes is None:
            return src_state.param
        if isinstance(src_state, SharedTrainingState) and not src_state.imported and \
                src_state.granule_bytes == dst_granule_bytes:
            return [src_state.tensors[b] for b in src_state.buffers.granules_of(3)]
        return None

    def log_communication_info(self, transfer_time: float, union_world_group=None,
                               logger: Optional[logging.Logger] = None) -> str:
        """The reference's perf line (elastic_manager.py:158-178) plus the payload written on the device.

        ``communication bytes`` keeps the reference's definition (GiB a rank
        would exchange with other ranks, max over ranks); ``payload`` is the
        decimal GB of state written on the device.  The reference reduces the
        line's figures over ``union_world_group``; one process already holds
        every rank's figures, so the group is accepted and unused.
        """
        gib = self.transfer_manager.get_communication_bytes()
        payload = self.transfer_manager.get_payload_bytes()
        bw = 1000 * gib / transfer_time if transfer_time > 0 else float("inf")
        pbw = payload / transfer_time / 1e6 if transfer_time > 0 else float("inf")
        msg = (f"[ElasticMegatron-Perf] : transfer time: {transfer_time:.2f} ms, "
               f"communication bytes: {gib:.2f} GB, bandwidth: {bw:.2f} GB/s "
               f"(payload {payload / 1e9:.2f} GB at {pbw:.1f} GB/s)")
        if logger is not None:
            logger.info(msg)
        return msg

    def clear_meta_state(self, parallel_strategy: StrategyLike) -> int:
        """Forget what a meta-device reshard pre-built for ``parallel_strategy``
        (elastic_manager.py:180-187): here, the cached copy plans into or out of
        it.  The live state's own strategy cannot be cleared.  Returns the
        number of plans dropped."""
        strategy = _as_strategy(parallel_strategy)
        if strategy == self.training_state.parallel_strategy:
            raise AssertionError("the live training state uses this strategy: it is not a meta state")
        return self.transfer_manager.evict(strategy)

    def reshard(self, new_parallel_strategy: StrategyLike, logger: Optional[logging.Logger] = None,
                is_meta_device: bool = False, save_ckpt: bool = False,
                verify: bool = False, lost_ranks=None) -> Optional[TrainingState]:
        """Switch every rank's state to ``new_parallel_strategy``; returns the new state.

        ``is_meta_device=True`` builds and caches the plan, uploads its tables
        to the state's GPU (nothing else: no state is allocated or touched)
        and returns None; the real switch then runs as fast as a repeated one.
        This is the reference's meta-device pre-build, which runs a fake
        transfer to build its NCCL connections (elastic_manager.py:268-304).

        ``verify=True`` compares the new state with the old one on the device
        before the old one is released (the reference's offline checkpoint
        comparison, tools/ckpt/compare_ckpt.py, done in place); the report is
        kept in ``last_verification`` and a mismatch raises RuntimeError.  The
        old state then stays the live state, whole, except after a staged
        (``low_memory``) switch with ``release_source``: each stage's source arena
        is released once that stage has been checked, so a mismatch in a later
        stage leaves the old state without the arenas of the stages before it.

        ``lost_ranks`` (an extension; the reference has no recovery path): ranks of the current
        world whose optimizer state is gone, such as a failed GPU's.  With more than one
        distributed-optimizer instance every instance holds the whole fp32 state, so a
        Group-ZeRO switch reads each shard of a lost rank from another instance's copy and reads
        nothing from the lost ranks (their bf16 params are the model shard's, which every rank of
        its DP group holds).  A shard whose every copy is lost, or any other kind of switch,
        raises ValueError.
        """
        if is_meta_device and save_ckpt:
            raise AssertionError("Can't save checkpoint in meta device")
        if save_ckpt:
            raise NotImplementedError("checkpoint saving is not part of the reshard data path")
        dst_strategy = _as_strategy(new_parallel_strategy)
        src_state = self.training_state
        if src_state.device.type == "meta" and not is_meta_device:
            raise RuntimeError("the manager was built on the meta device and holds no state yet: "
                               "attach_training_state first (or reshard with is_meta_device=True)")
        src_strategy = src_state.parallel_strategy
        space = src_state.layout.space
        backup = ParallelStrategy.is_redundant_backup(src_strategy, dst_strategy)
        dst_space = self.space_for(dst_strategy)
        dst_layout = dst_space.layout(dst_strategy)
        if backup is None and dst_space is space:
            space.register_reshard(src_strategy, dst_strategy)
        gs = _granule_of(src_state)
        gd = self.share_granule_bytes if src_state.device.type != "meta" else None
        # Under Group ZeRO the model-parallel shards are unchanged, so the bf16 params carry over
        # (or are copied, when the new state cannot share them).
        param = self._carried_params(src_state, gd) if backup is not None else None
        kind = "transfer" if backup is None else backup_kind(backup, param is None)
        lost = tuple(lost_ranks or ())
        # ... and instance 0's fp32 granules stay where they are when the new state can take them over.
        adopt = self._adoptable(src_state, dst_layout, kind, gd, param, lost)
        plan = self.transfer_manager.plan_for_states(src_state.layout, dst_layout, gs, gd, kind, adopt_granules=adopt,
                                                     lost_ranks=lost)
        stages = self.transfer_manager.staged_for_states(src_state.layout, dst_layout, gs, gd, kind, lost_ranks=lost) \
            if self.low_memory else ()
        if is_meta_device:
            self._prepare(stages or plan, src_state)
            return None
        report = None
        if self.low_memory:
            if self.share_granule_bytes is not None:
                dst_state = SharedTrainingState.allocate(dst_layout, src_state.device, self.share_granule_bytes,
                                                         param_granules=param, kinds=())
            else:
                dst_state = TrainingState.allocate(dst_layout, src_state.device, param=param, kinds=(),
                                                   granule_bytes=ARENA_GRANULE_BYTES)
            elapsed, checked = self.transfer_staged(src_state, dst_state, kind, verify, lost_ranks=lost)
            if verify:
                report = report_from_stats(*checked)
        else:
            adopted = src_state.leading_fp32_granules(adopt) if adopt else None
            dst_state = self._allocate(dst_layout, src_state.device, param=param, adopted=adopted)
            if backup is None:
                elapsed = self.transfer_params(src_state, dst_state)
            else:
                elapsed = self.redundant_backup(src_state, dst_state, backup, lost_ranks=lost)
            if verify:
                report = self.transfer_manager.verify(src_state, dst_state, kind, lost_ranks=lost)
        self.last_transfer_ms = elapsed
        if verify:
            self.last_verification = report
            if not report.bit_exact:
                lines = report.lines()
                raise RuntimeError(f"reshard verification failed: {report.mismatches} elements differ\n"
                                   + "\n".join(lines[:20]))
        if self.release_source:
            if adopt:
                src_state.hand_over(adopt)
            src_state.release_optimizer()
        self.training_state = dst_state
        msg = self.log_communication_info(elapsed, logger=logger)
        if logger is None and torch.distributed.is_available() and not torch.distributed.is_initialized():
            print(msg)
        return dst_state
