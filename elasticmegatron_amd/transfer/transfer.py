"""Executor of a reshard: one native copy-plan launch.

Replaces ``TransferManager`` of the reference
(elastic_megatron/transfer/transfer.py:23-388).  The reference runs three
Python passes over all parameters with blocking point-to-point messages
(DP gather + SwiGLU shuffle, TP/PP/EP exchange, SwiGLU unshuffle + DP
scatter) and relies on a FIFO for rank-local self copies
(transfer.py:143-269, communicator.py:38-96).  Here the whole switch is
lowered once to a segment table (cached per strategy pair, like the
reference's per-parameter plan cache, virtual_param.py:174-188) and executed
as one launch on the caller's stream.  Rank-local copies and cross-rank
messages are the same operation on one device.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Dict, Optional, Tuple

import numpy as np
import torch

from .. import _native
from ..megatron_manager.parallel_strategy import ParallelStrategy
from ..megatron_manager.training_state import TrainingState
from ..resharding.comm_stats import FP32_TENSORS_BYTES, reference_comm_bytes
from ..resharding.lowering import in_place_prefix, lower_redundant_backup, lower_transfer, payload_bytes, read_bytes
from ..resharding.layout import ARENA_PARAM, SEG_CAST_BF16, SEG_DUP, SEG_ZERO_FILL, StrategyLayout
from ..resharding.shares import destination_rank_shares
from ..resharding.granules import GranuleBuffers
from ..resharding.tensors import TensorBuffers, rebase_on_tensors
from .verify import VerifyReport, report_from_stats


@dataclass
class CompiledPlan:
    segments: np.ndarray
    native: _native.Plan
    payload_bytes: int              # bytes of state written to the destination per execution
    read_bytes: int                 # bytes read per execution
    src: ParallelStrategy
    dst: ParallelStrategy
    reference_comm_bytes: int = 0   # the reference's per-rank cross-rank volume, max over ranks
    src_buf_bytes: Tuple[int, ...] = ()   # arena sizes the plan was checked against
    dst_buf_bytes: Tuple[int, ...] = ()
    src_refs: Tuple[int, ...] = (0, 1, 2, 3)   # arenas the plan reads
    dst_refs: Tuple[int, ...] = (0, 1, 2, 3)   # arenas the plan writes

    @property
    def traffic_bytes(self) -> int:
        """Algorithmic HBM traffic per execution: every byte read once and written once."""
        return self.payload_bytes + self.read_bytes


# Group-ZeRO kinds: (scale-up, bf16 params copied).  Without the copy the new state shares the old
# one's bf16 params; with it the new state holds its own.
BACKUP_KINDS = {"backup_up": (True, False), "backup_down": (False, False),
                "backup_up_bf16": (True, True), "backup_down_bf16": (False, True)}


def backup_kind(scale_up: bool, copy_bf16: bool = False) -> str:
    """The plan kind of a Group-ZeRO switch."""
    return ("backup_up" if scale_up else "backup_down") + ("_bf16" if copy_bf16 else "")


def _lower(src: StrategyLayout, dst: StrategyLayout, kind: str, include_bf16: bool, bf16_source: str,
           with_groups: bool = False, in_place_below: int = 0, lost_ranks: Tuple[int, ...] = (),
           source_instance: int = 0):
    """The segment table of a plan kind (with groups for verification)."""
    if kind == "transfer":
        if in_place_below:
            raise ValueError("only a Group-ZeRO switch can leave part of the new state in place")
        if lost_ranks:
            raise ValueError("only a Group-ZeRO switch has other optimizer instances to read a lost rank's state from")
        return lower_transfer(src, dst, include_bf16=include_bf16, bf16_source=bf16_source, with_groups=with_groups)
    if kind in BACKUP_KINDS:
        up, copy = BACKUP_KINDS[kind]
        return lower_redundant_backup(src, dst, scale_up=up, with_groups=with_groups, copy_bf16=copy,
                                      in_place_below=in_place_below, lost_ranks=lost_ranks,
                                      source_instance=source_instance)
    raise ValueError(kind)


def _lost(lost_ranks) -> Tuple[int, ...]:
    """Lost ranks as a sorted tuple without repeats (a plan-cache key part)."""
    return tuple(sorted({int(r) for r in lost_ranks}))


def _lost_key(lost: Tuple[int, ...]) -> Tuple:
    return (("lost", lost),) if lost else ()


def adoptable_granules(src: StrategyLayout, dst: StrategyLayout, granule_bytes: int, kind: str,
                       lost_ranks=()) -> int:
    """Leading granules of each fp32 arena that the new state of a Group-ZeRO switch can take over
    from the old one instead of copying them, both held in granules of ``granule_bytes``: whole
    granules of the same size on both sides inside :func:`in_place_prefix`.  With PP = 1 that is
    all of instance 0, a third of a scale-up to two instances' traffic and nearly all of a
    scale-down's.  With ``lost_ranks``, only granules that end before the first lost rank's
    state.  0 for any other switch."""
    if kind not in BACKUP_KINDS or granule_bytes is None:
        return 0
    end = in_place_prefix(src, dst, BACKUP_KINDS[kind][0])
    for g in lost_ranks:
        end = min(end, src.rank_fp32_slice(int(g))[0])
    return end * 4 // granule_bytes


def _fixed_padding_space(src: StrategyLayout, dst: StrategyLayout):
    """The model the reference would run a switch in: it keeps the padded vocabulary fixed
    (virtual_param.py:480-481), so a re-padding switch is priced in whichever of the two
    models both TP sizes divide; None when neither does."""
    if src.space is dst.space:
        return src.space
    tps = (src.strategy.tensor_model_parallel_size, dst.strategy.tensor_model_parallel_size)
    for space in (src.space, dst.space):
        if all(space.spec.padded_vocab_size % t == 0 for t in tps):
            return space
    return None


def _arena_refs(table: np.ndarray) -> Tuple[Tuple[int, ...], Tuple[int, ...]]:
    """(source arenas read, destination arenas written) by a segment table."""
    reads = (table["flags"] & SEG_ZERO_FILL) == 0
    second = (table["flags"] & (SEG_CAST_BF16 | SEG_DUP)) != 0
    src = sorted(set(table["src_buf"][reads].tolist()))
    dst = sorted(set(table["dst_buf"].tolist()) | set(table["aux_buf"][second].tolist()))
    return tuple(int(x) for x in src), tuple(int(x) for x in dst)


def _stage_mask(table: np.ndarray, kind: int) -> np.ndarray:
    """Rows of stage ``kind`` of a staged switch: those writing fp32 arena ``kind``, and with the
    first stage the bf16 param rows (the bf16 image rides on the main rows)."""
    d = table["dst_buf"]
    return ((d == kind) | (d == ARENA_PARAM)) if kind == 0 else (d == kind)


def _stage_rows(table: np.ndarray, kind: int) -> np.ndarray:
    return table[_stage_mask(table, kind)]


@dataclass
class CompiledTensorPlan:
    """A switch over per-tensor buffers (one buffer per stored tensor; see resharding.tensors)."""

    segments: np.ndarray
    native: _native.Plan
    src: TensorBuffers
    dst: TensorBuffers
    payload_bytes: int
    read_bytes: int
    buffer_nbytes: list = None   # bytes of every source, then every destination buffer
    reference_comm_bytes: int = 0
    src_refs: Tuple[int, ...] = None   # buffers the plan reads
    dst_refs: Tuple[int, ...] = None   # buffers the plan writes

    @property
    def traffic_bytes(self) -> int:
        """Algorithmic HBM traffic per execution: every byte read once and written once."""
        return self.payload_bytes + self.read_bytes

    def __post_init__(self):
        if self.buffer_nbytes is None:
            self.buffer_nbytes = self.src.nbytes() + self.dst.nbytes()
        if self.src_refs is None:
            self.src_refs, self.dst_refs = _arena_refs(self.segments)


class TransferManager:
    """Builds, caches and runs copy plans between device-resident training states.

    The constructor keeps the reference's ``send_fn`` / ``recv_fn`` /
    ``broadcast_fn`` parameters (transfer.py:23-34) so that existing call
    sites construct it unchanged.  With every rank's state on one device
    every hop is a local copy inside the plan, so they are kept but never
    called.
    """

    def __init__(self, send_fn: Optional[Callable] = None, recv_fn: Optional[Callable] = None,
                 broadcast_fn: Optional[Callable] = None, *, check_disjoint: bool = False,
                 bf16_source: str = "cast"):
        if bf16_source not in ("cast", "copy"):
            raise ValueError(f"bf16_source must be 'cast' or 'copy', not {bf16_source!r}")
        self.send_fn, self.recv_fn, self.broadcast_fn = send_fn, recv_fn, broadcast_fn
        self._plans: Dict[Tuple, CompiledPlan] = {}
        self.check_disjoint = check_disjoint
        self.bf16_source = bf16_source
        self.fake_transfer = False
        self._verify_plans: Dict[Tuple, Tuple] = {}
        self._checked_tensors: Dict[int, Tuple] = {}   # per plan: the pointers last checked
        self._adoptable: Dict[Tuple, int] = {}
        self._payload_bytes = 0
        self._comm_bytes = 0

    def set_fake_transfer(self, fake_transfer: bool) -> None:
        """Plan without moving data (transfer.py:32-34)."""
        self.fake_transfer = fake_transfer

    def evict(self, strategy: Optional[ParallelStrategy] = None) -> int:
        """Drop the cached plans (copy and verification) that switch from or to ``strategy``, or every
        cached plan when it is None; returns how many were dropped.  A dropped plan frees its device
        segment tables once nothing else holds it."""
        n = 0
        for cache in (self._plans, self._verify_plans):
            for key in [k for k in cache if strategy is None or any(x == strategy for x in k)]:
                del cache[key]
                n += 1
        live = {id(p) for p in self._plans.values()}
        self._checked_tensors = {k: v for k, v in self._checked_tensors.items() if k in live}
        self._adoptable = {k: v for k, v in self._adoptable.items()
                           if not (strategy is None or any(x == strategy for x in k))}
        return n

    def adoptable(self, src: StrategyLayout, dst: StrategyLayout, granule_bytes: Optional[int], kind: str, *,
                  lost_ranks=()) -> int:
        """:func:`adoptable_granules`, kept per switch (it walks every parameter's runs)."""
        lost = _lost(lost_ranks)
        key = (src.space.spec, src.strategy, dst.space.spec, dst.strategy, granule_bytes, kind) + _lost_key(lost)
        n = self._adoptable.get(key)
        if n is None:
            n = self._adoptable[key] = adoptable_granules(src, dst, granule_bytes, kind, lost)
        return n

    def compile(self, src: StrategyLayout, dst: StrategyLayout, kind: str = "transfer",
                include_bf16: bool = True, in_place_below: int = 0, *, lost_ranks=(),
                source_instance: int = 0) -> CompiledPlan:
        """The arena plan of a switch; ``in_place_below``, ``lost_ranks`` and ``source_instance``:
        see :func:`lower_redundant_backup`."""
        lost = _lost(lost_ranks)
        key = (src.space.spec, src.strategy, dst.space.spec, dst.strategy, kind, include_bf16, self.bf16_source)
        if in_place_below:
            key += (("in-place", in_place_below),)
        key += _lost_key(lost)
        if source_instance:
            key += (("source-instance", source_instance),)
        cp = self._plans.get(key)
        if cp is not None:
            return cp
        table = _lower(src, dst, kind, include_bf16, self.bf16_source, in_place_below=in_place_below, lost_ranks=lost,
                       source_instance=source_instance)
        sb = [src.fp32_numel * 4] * 3 + [src.bf16_numel * 2]
        db = [dst.fp32_numel * 4] * 3 + [dst.bf16_numel * 2]
        if kind == "transfer":
            space = _fixed_padding_space(src, dst)
            comm = max(reference_comm_bytes(space, src.strategy, dst.strategy).values(), default=0) \
                if space is not None else 0
        elif BACKUP_KINDS[kind][0]:  # every rank joins the broadcast of its whole shard (transfer.py:377-388)
            comm = max(dst.rank_numel) * FP32_TENSORS_BYTES
        else:  # param_migrate is a local copy (training_state.py:40-60)
            comm = 0
        cp = CompiledPlan(table, _native.Plan(table, sb, db, self.check_disjoint), payload_bytes(table),
                          read_bytes(table), src.strategy, dst.strategy, comm, tuple(sb), tuple(db),
                          *_arena_refs(table))
        self._plans[key] = cp
        return cp

    def compile_staged(self, src: StrategyLayout, dst: StrategyLayout, kind: str = "transfer",
                       include_bf16: bool = True, *, lost_ranks=()) -> Tuple[CompiledPlan, CompiledPlan, CompiledPlan]:
        """The switch as three launches, one per optimizer kind: ``main`` (with the bf16 params),
        ``exp_avg``, ``exp_avg_sq``.  Stage k reads source arena k only and writes destination arena
        k only (and the param arena), so a caller can allocate each destination arena just before its
        stage and release the source arena right after it, as the reference releases every
        optimizer tensor once it is sent (transfer.py:182-228, resharding_metadata.py:58-65).  The
        three together write exactly what :meth:`compile` writes."""
        lost = _lost(lost_ranks)
        key = ("staged", src.space.spec, src.strategy, dst.space.spec, dst.strategy, kind, include_bf16,
               self.bf16_source) + _lost_key(lost)
        stages = self._plans.get(key)
        if stages is not None:
            return stages
        full = self.compile(src, dst, kind, include_bf16, lost_ranks=lost)
        out = []
        for k in range(3):
            t = _stage_rows(full.segments, k)
            out.append(CompiledPlan(t, _native.Plan(t, full.src_buf_bytes, full.dst_buf_bytes, self.check_disjoint),
                                    payload_bytes(t), read_bytes(t), full.src, full.dst,
                                    full.reference_comm_bytes if k == 0 else 0, full.src_buf_bytes,
                                    full.dst_buf_bytes, *_arena_refs(t)))
        stages = tuple(out)
        self._plans[key] = stages
        return stages

    def prepare(self, plans, device) -> None:
        """Upload the tables of a compiled plan (or of several, such as the stages of
        :meth:`compile_staged`) to ``device`` now, so that their first execution there runs as fast
        as later ones: the counterpart of the reference's meta-device pass, which builds its NCCL
        connections ahead of the switch (elastic_manager.py:282-304)."""
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError("plans are prepared on a GPU: the reshard has no CPU path")
        if isinstance(plans, (CompiledPlan, CompiledTensorPlan)):
            plans = (plans,)
        with torch.cuda.device(device):
            st = torch.cuda.current_stream(device)
            for p in plans:
                p.native.prepare(st.cuda_stream)

    def compile_shares(self, src: StrategyLayout, dst: StrategyLayout, kind: str = "transfer",
                       include_bf16: bool = True, *, lost_ranks=()) -> Tuple[Tuple[CompiledPlan, ...], CompiledPlan]:
        """The switch split by destination rank (``resharding.shares``): plan g writes rank g's
        fp32 shard, with the bf16 image of its ``main`` pieces, and nothing else; the last plan
        holds the segments whose primary destination is the bf16 param arena (none when the bf16
        params are cast).  With one rank per GPU, plan g is what GPU g would run, its sources then
        partly on peers.  Run in any order on the same arenas, they write what :meth:`compile`
        writes.  ``lost_ranks``: as for :func:`lower_redundant_backup`; no share then pulls from
        them."""
        lost = _lost(lost_ranks)
        key = ("shares", src.space.spec, src.strategy, dst.space.spec, dst.strategy, kind, include_bf16,
               self.bf16_source) + _lost_key(lost)
        got = self._plans.get(key)
        if got is not None:
            return got
        full = self.compile(src, dst, kind, include_bf16, lost_ranks=lost)
        per_rank, bf16 = destination_rank_shares(full.segments, dst)

        def plan_of(t):
            return CompiledPlan(t, _native.Plan(t, full.src_buf_bytes, full.dst_buf_bytes, self.check_disjoint),
                                payload_bytes(t), read_bytes(t), full.src, full.dst, 0, full.src_buf_bytes,
                                full.dst_buf_bytes, *_arena_refs(t))

        got = (tuple(plan_of(t) for t in per_rank), plan_of(bf16))
        self._plans[key] = got
        return got

    def compile_tensors(self, src: StrategyLayout, dst: StrategyLayout, kind: str = "transfer",
                        include_bf16: bool = True, *, lost_ranks=()) -> CompiledTensorPlan:
        """The switch over one buffer per stored tensor, as the reference holds them: the
        ``OptimizerTensorInfo`` tensors of every (rank, parameter) and the bf16 parameter of every
        model-parallel shard.  ``plan.src.keys`` / ``plan.dst.keys`` name the tensors in buffer
        order.  ``lost_ranks``: as for :func:`lower_redundant_backup`; the lost ranks' tensors are
        then not referenced and may be None."""
        lost = _lost(lost_ranks)
        key = ("tensors", src.space.spec, src.strategy, dst.space.spec, dst.strategy, kind, include_bf16,
               self.bf16_source) + _lost_key(lost)
        cp = self._plans.get(key)
        if cp is not None:
            return cp
        arena_plan = self.compile(src, dst, kind, include_bf16, lost_ranks=lost)
        sb, db = TensorBuffers(src), TensorBuffers(dst)
        table = rebase_on_tensors(arena_plan.segments, sb, db)
        cp = CompiledTensorPlan(table, _native.Plan(table, sb.nbytes(), db.nbytes(), self.check_disjoint), sb, db,
                                payload_bytes(table), read_bytes(table))
        self._plans[key] = cp
        return cp

    def compile_share_tensors(self, src: StrategyLayout, dst: StrategyLayout, rank: int, kind: str = "transfer",
                              include_bf16: bool = True, *, lost_ranks=()) -> CompiledTensorPlan:
        """Destination rank ``rank``'s share of the switch (:meth:`compile_shares`) over one buffer
        per stored tensor (:meth:`compile_tensors`).  It reads and writes only some of the tensors:
        ``plan.src_refs`` / ``plan.dst_refs``, the rest may be passed as None to
        :meth:`execute_tensors`.  With one rank per GPU, those are what GPU ``rank`` runs its part
        of the switch on: its own optimizer tensors, its part of its model shard's bf16 params, and
        the source tensors it pulls, which in a multi-GPU job other GPUs hold.  With ``lost_ranks``
        none of those is a lost rank's."""
        lost = _lost(lost_ranks)
        key = ("share-tensors", src.space.spec, src.strategy, dst.space.spec, dst.strategy, kind, include_bf16,
               self.bf16_source, rank) + _lost_key(lost)
        cp = self._plans.get(key)
        if cp is not None:
            return cp
        per_rank, _ = self.compile_shares(src, dst, kind, include_bf16, lost_ranks=lost)
        if not 0 <= rank < len(per_rank):
            raise ValueError(f"rank {rank} is not a destination rank (world {len(per_rank)})")
        sb, db = TensorBuffers(src), TensorBuffers(dst)
        table = rebase_on_tensors(per_rank[rank].segments, sb, db)
        cp = CompiledTensorPlan(table, _native.Plan(table, sb.nbytes(), db.nbytes(), self.check_disjoint), sb, db,
                                payload_bytes(table), read_bytes(table))
        self._plans[key] = cp
        return cp

    def execute_tensors(self, plan: CompiledTensorPlan, src_tensors, dst_tensors,
                        stream: Optional[torch.cuda.Stream] = None) -> None:
        """Run a per-tensor plan; ``src_tensors`` / ``dst_tensors`` follow ``plan.src.keys`` / ``plan.dst.keys``.
        A tensor the plan neither reads nor writes may be None (a share of the switch)."""
        if self.fake_transfer:
            return
        if len(src_tensors) != len(plan.src) or len(dst_tensors) != len(plan.dst):
            raise ValueError("tensor lists do not match the plan's buffers")
        ts = list(src_tensors) + list(dst_tensors)
        if any(t is None for t in ts):
            self._execute_some_tensors(plan, ts, stream)
            return
        # One pass per property in list comprehensions: a per-tensor plan passes thousands of
        # tensors, and this check runs before every launch.  The pointers and sizes are read on
        # every call; the layout and device checks are skipped when both equal those of the last
        # call that passed them (the same tensors again: same storage, offset and size).
        ptrs = [t.data_ptr() for t in ts]
        nbytes = [t.nbytes for t in ts]
        if nbytes != plan.buffer_nbytes:
            raise ValueError("a tensor does not match its buffer (bytes or layout)")
        dev = ts[0].device
        last = self._checked_tensors.get(id(plan))
        if last is None or last[0] is not plan or last[1] != ptrs or last[2] != dev:
            if not all([t.is_contiguous() for t in ts]):
                raise ValueError("a tensor does not match its buffer (bytes or layout)")
            if dev.type != "cuda" or any([t.device != dev for t in ts]):
                raise RuntimeError("tensors must live in GPU memory, on one device: the reshard has no CPU path")
            self._checked_tensors[id(plan)] = (plan, ptrs, dev)
        st = stream if stream is not None else torch.cuda.current_stream(dev)
        ns = len(plan.src)
        with torch.cuda.device(dev):
            plan.native.execute(ptrs[:ns], ptrs[ns:], st.cuda_stream)
        self._payload_bytes += plan.payload_bytes

    def _execute_some_tensors(self, plan: CompiledTensorPlan, ts, stream) -> None:
        """execute_tensors with None for the tensors the plan does not touch: every tensor it reads or
        writes is checked on every call (such a plan is one rank's share, run once per switch)."""
        ns = len(plan.src)
        refs = set(plan.src_refs) | {ns + i for i in plan.dst_refs}
        need = plan.buffer_nbytes
        dev = None
        for i in sorted(refs):
            t = ts[i]
            if t is None:
                raise ValueError(f"the plan reads or writes {(plan.src.keys + plan.dst.keys)[i]}, which is None")
            if t.nbytes != need[i] or not t.is_contiguous():
                raise ValueError("a tensor does not match its buffer (bytes or layout)")
            dev = t.device if dev is None else dev
            if t.device != dev or dev.type != "cuda":
                raise RuntimeError("tensors must live in GPU memory, on one device: the reshard has no CPU path")
        if dev is None:
            return   # nothing to move
        ptrs = [0 if t is None or i not in refs else t.data_ptr() for i, t in enumerate(ts)]
        st = stream if stream is not None else torch.cuda.current_stream(dev)
        with torch.cuda.device(dev):
            plan.native.execute(ptrs[:ns], ptrs[ns:], st.cuda_stream)
        self._payload_bytes += plan.payload_bytes

    def compile_granules(self, src: StrategyLayout, dst: StrategyLayout, src_granule_bytes: Optional[int],
                         dst_granule_bytes: Optional[int], kind: str = "transfer",
                         include_bf16: bool = True, adopt_granules: int = 0, *, lost_ranks=()) -> CompiledTensorPlan:
        """The switch between states whose arenas are cut into granules (``SharedTrainingState``,
        handed between processes; ``None``: whole arenas, a ``TrainingState``).  ``plan.src`` /
        ``plan.dst`` are the :class:`~..resharding.granules.GranuleBuffers` of each side.

        ``adopt_granules``: a Group-ZeRO switch whose new state holds the old one's first
        ``adopt_granules`` granules of every fp32 arena (at most :func:`adoptable_granules`); the
        plan writes nothing there."""
        lost = _lost(lost_ranks)
        key = ("granules", src.space.spec, src.strategy, dst.space.spec, dst.strategy, kind, include_bf16,
               self.bf16_source, src_granule_bytes, dst_granule_bytes, adopt_granules) + _lost_key(lost)
        cp = self._plans.get(key)
        if cp is not None:
            return cp
        if adopt_granules:
            if src_granule_bytes is None or src_granule_bytes != dst_granule_bytes:
                raise ValueError("adopting granules needs both states in granules of one size")
            if not 0 < adopt_granules <= self.adoptable(src, dst, src_granule_bytes, kind, lost_ranks=lost):
                raise ValueError(f"the new state cannot take over {adopt_granules} granules of the old one")
        below = adopt_granules * src_granule_bytes // 4 if adopt_granules else 0
        arena_plan = self.compile(src, dst, kind, include_bf16, in_place_below=below, lost_ranks=lost)
        sb, db = GranuleBuffers(src, src_granule_bytes), GranuleBuffers(dst, dst_granule_bytes)
        table = rebase_on_tensors(arena_plan.segments, sb, db)
        cp = CompiledTensorPlan(table, _native.Plan(table, sb.nbytes(), db.nbytes(), self.check_disjoint), sb, db,
                                payload_bytes(table), read_bytes(table),
                                reference_comm_bytes=arena_plan.reference_comm_bytes)
        self._plans[key] = cp
        return cp

    def staged_for_states(self, src_layout: StrategyLayout, dst_layout: StrategyLayout, src_granule_bytes,
                          dst_granule_bytes, kind: str = "transfer", include_bf16: bool = True, *, lost_ranks=()):
        """The three plans of :meth:`compile_staged`, re-based onto granules when either side is held
        in them (a staged switch from a received state)."""
        lost = _lost(lost_ranks)
        stages = self.compile_staged(src_layout, dst_layout, kind, include_bf16, lost_ranks=lost)
        if src_granule_bytes is None and dst_granule_bytes is None:
            return stages
        key = ("staged-granules", src_layout.space.spec, src_layout.strategy, dst_layout.space.spec,
               dst_layout.strategy, kind, include_bf16, self.bf16_source, src_granule_bytes,
               dst_granule_bytes) + _lost_key(lost)
        got = self._plans.get(key)
        if got is not None:
            return got
        sb, db = GranuleBuffers(src_layout, src_granule_bytes), GranuleBuffers(dst_layout, dst_granule_bytes)
        out = []
        for st in stages:
            table = rebase_on_tensors(st.segments, sb, db)
            out.append(CompiledTensorPlan(table, _native.Plan(table, sb.nbytes(), db.nbytes(), self.check_disjoint),
                                          sb, db, payload_bytes(table), read_bytes(table),
                                          reference_comm_bytes=st.reference_comm_bytes))
        got = tuple(out)
        self._plans[key] = got
        return got

    def plan_for_states(self, src_layout: StrategyLayout, dst_layout: StrategyLayout, src_granule_bytes,
                        dst_granule_bytes, kind: str = "transfer", include_bf16: bool = True,
                        adopt_granules: int = 0, *, lost_ranks=()):
        """The arena plan when both sides are whole arenas, else the granule plan."""
        if src_granule_bytes is None and dst_granule_bytes is None and not adopt_granules:
            return self.compile(src_layout, dst_layout, kind, include_bf16, lost_ranks=lost_ranks)
        return self.compile_granules(src_layout, dst_layout, src_granule_bytes, dst_granule_bytes, kind,
                                     include_bf16, adopt_granules, lost_ranks=lost_ranks)

    def execute_states(self, plan, src, dst, stream: Optional[torch.cuda.Stream] = None) -> None:
        """Run ``plan`` (from :meth:`plan_for_states`) between two states of either kind."""
        if isinstance(plan, CompiledPlan):
            self.execute(plan, src, dst, stream)
            return
        if self.fake_transfer:
            return
        if src.layout.strategy != plan.src.layout.strategy or dst.layout.strategy != plan.dst.layout.strategy:
            raise ValueError("states do not match the plan's strategies")
        if src.device != dst.device or src.device.type != "cuda":
            raise RuntimeError("source and destination states must be on one GPU")
        sp, sn = _buffers_of(src)
        dp, dn = _buffers_of(dst)
        # Buffers the plan does not touch may be empty: a staged switch allocates the destination's
        # arenas and releases the source's one at a time.
        for have, need, refs, side in ((sn, plan.src.nbytes(), plan.src_refs, "source"),
                                       (dn, plan.dst.nbytes(), plan.dst_refs, "destination")):
            if len(have) != len(need) or any(have[i] < need[i] for i in refs):
                raise ValueError(f"the {side} state's buffers do not match the plan (released, not yet "
                                 "allocated, or laid out for another granule size)")
        st = stream if stream is not None else torch.cuda.current_stream(src.device)
        with torch.cuda.device(src.device):
            plan.native.execute(sp, dp, st.cuda_stream)
        self._payload_bytes += plan.payload_bytes
        self._comm_bytes += plan.reference_comm_bytes

    def execute(self, plan: CompiledPlan, src: TrainingState, dst: TrainingState,
                stream: Optional[torch.cuda.Stream] = None) -> None:
        if self.fake_transfer:
            return
        if src.layout.strategy != plan.src or dst.layout.strategy != plan.dst:
            raise ValueError("training states do not match the plan's strategies")
        if src.device != dst.device:
            raise ValueError("source and destination states must be on the same device")
        if src.device.type != "cuda":
            raise RuntimeError("training states must live in GPU memory: the reshard has no CPU path")
        # The kernel trusts the sizes the plan was built for; a state laid out for another model
        # (another padded vocabulary, say) must not reach it.  Arenas the plan does not touch may
        # be empty (a staged switch allocates and releases them one at a time).
        have = src.arena_bytes(), dst.arena_bytes()
        need = plan.src_buf_bytes, plan.dst_buf_bytes
        for side, refs in enumerate((plan.src_refs, plan.dst_refs)):
            for a in refs:
                if need[side] and have[side][a] < need[side][a]:
                    raise ValueError("a training state's arena is smaller than the plan's buffer: it is "
                                     "released, not yet allocated, or laid out for another model")
        st = stream if stream is not None else torch.cuda.current_stream(src.device)
        with torch.cuda.device(src.device):
            plan.native.execute(src.arena_ptrs(), dst.arena_ptrs(), st.cuda_stream)
        self._payload_bytes += plan.payload_bytes
        self._comm_bytes += plan.reference_comm_bytes

    def verify(self, src: TrainingState, dst: TrainingState, kind: str = "transfer",
               include_bf16: bool = True, stream: Optional[torch.cuda.Stream] = None, *,
               lost_ranks=()) -> VerifyReport:
        """Check, on the device, that ``dst`` holds what the switch from ``src`` must produce.

        Replaces the reference's offline checkpoint comparison
        (tools/ckpt/compare_ckpt.py:17-76): per parameter and tensor kind, the
        bits that differ and compare_ckpt's max-abs / max-rel / RMS / relative
        RMS.  ``src`` must still hold the state it was resharded from (with ``lost_ranks``, the
        copies the switch read instead of theirs).
        """
        stats, names = self.verify_stats(src, dst, kind, include_bf16, stream, lost_ranks=lost_ranks)
        return report_from_stats(stats, names)

    def verify_stats(self, src: TrainingState, dst: TrainingState, kind: str = "transfer",
                     include_bf16: bool = True, stream: Optional[torch.cuda.Stream] = None,
                     stage: Optional[int] = None, *, lost_ranks=()):
        """The records behind :meth:`verify` and the parameter names they index; with ``stage`` only
        what stage ``stage`` of :meth:`compile_staged` writes, so that a staged switch can check each
        stage before it releases that stage's source arena (:func:`.verify.merge_stats` adds them)."""
        if src.device.type != "cuda" or dst.device.type != "cuda":
            raise RuntimeError("training states must live in GPU memory: verification has no CPU path")
        sl, dl = src.layout, dst.layout
        gs, gd = _granule_of(src), _granule_of(dst)
        lost = _lost(lost_ranks)
        key = (sl.space.spec, sl.strategy, dl.space.spec, dl.strategy, kind, include_bf16, self.bf16_source, stage,
               gs, gd) + _lost_key(lost)
        vp = self._verify_plans.get(key)
        if vp is None:
            table, groups, aux_groups = _lower(sl, dl, kind, include_bf16, self.bf16_source, with_groups=True,
                                               lost_ranks=lost)
            if stage is not None:
                m = _stage_mask(table, stage)
                table, groups, aux_groups = table[m], groups[m], aux_groups[m]
            if gs is None and gd is None:
                sb = [sl.fp32_numel * 4] * 3 + [sl.bf16_numel * 2]
                db = [dl.fp32_numel * 4] * 3 + [dl.bf16_numel * 2]
            else:   # granules: the groups follow the segments through the cuts
                sgb, dgb = GranuleBuffers(sl, gs), GranuleBuffers(dl, gd)
                table, origin = rebase_on_tensors(table, sgb, dgb, return_origin=True)
                groups, aux_groups = groups[origin], aux_groups[origin]
                sb, db = sgb.nbytes(), dgb.nbytes()
            names = [p.name for p in dl.space.all_virtual_params]
            vp = (_native.Plan(table, sb, db), groups, aux_groups, names)
            self._verify_plans[key] = vp
        plan, groups, aux_groups, names = vp
        st = stream if stream is not None else torch.cuda.current_stream(src.device)
        with torch.cuda.device(src.device):
            stats = plan.compare(_buffers_of(src)[0], _buffers_of(dst)[0], groups, aux_groups, 4 * len(names),
                                 st.cuda_stream)
        return stats, names

    def transfer_optimizer_tensors(self, virtual_param_space, use_block_and_print: bool = False, *,
                                   src: Optional[TrainingState] = None, dst: Optional[TrainingState] = None,
                                   include_bf16: bool = True, stream=None) -> CompiledPlan:
        """Move fp32 optimizer state from ``src`` to ``dst`` and rebuild the bf16 params (transfer.py:291-341).

        By default the destination bf16 params are the bf16 rounding of the
        destination main weights, written in the same pass (the reference's
        cast plus DP all-gather, training_state.py:176-197); with
        ``bf16_source="copy"`` they are copied from the source bf16 shards.

        ``use_block_and_print`` keeps the reference's debugging switch
        (transfer.py:271-289): every parameter's global send and receive
        ranges are printed before the switch runs.  There is nothing to block
        on: the whole switch is one launch.
        """
        src = src if src is not None else virtual_param_space.src_state
        dst = dst if dst is not None else virtual_param_space.dst_state
        if use_block_and_print and virtual_param_space is not None:
            print(plan_dump(virtual_param_space), flush=True)
        plan = self.compile(src.layout, dst.layout, "transfer", include_bf16)
        self.execute(plan, src, dst, stream)
        return plan

    def redundant_backup(self, is_scale_up: bool, src: TrainingState, dst: TrainingState, group_src: int = 0,
                         stream=None) -> CompiledPlan:
        """Group-ZeRO switch (transfer.py:343-388): fp32 shards replicated or dropped.  As in the
        reference, only the optimizer tensors move; ``ElasticMegatronManager`` also copies the bf16
        params when the new state cannot share them.  ``group_src``: on a scale-up, the optimizer
        instance whose copy fills the new ones (the reference's broadcast root in the
        inter-instance group)."""
        plan = self.compile(src.layout, dst.layout, backup_kind(is_scale_up),
                            source_instance=group_src if is_scale_up else 0)
        self.execute(plan, src, dst, stream)
        return plan

    def get_communication_bytes(self) -> float:
        """The reference's communication figure since the last call, in GiB, then reset.

        Max over ranks of fp32 bytes sent to or received from other ranks
        (communicator.py:118-122); see :mod:`..resharding.comm_stats`.
        """
        b = self._comm_bytes
        self._comm_bytes = 0
        return b / 1024 ** 3

    def get_payload_bytes(self) -> int:
        """Bytes of state written to the destination since the last call (each read once), then reset."""
        b = self._payload_bytes
        self._payload_bytes = 0
        return b


def _granule_of(state) -> Optional[int]:
    """Granule size of a shared state's arenas; None for a TrainingState's whole arenas."""
    return None if isinstance(state, TrainingState) else state.granule_bytes


def held_granules(src, dst) -> int:
    """Leading granules of every fp32 arena (the same count in each) that ``dst`` holds in
    ``src``'s memory, both states held in granules of one size: what a Group-ZeRO switch from
    ``src`` into ``dst`` leaves in place (:func:`adoptable_granules`).  0 for whole arenas."""
    gs, gd = _granule_of(src), _granule_of(dst)
    if gs is None or gs != gd:
        return 0
    sp, dp = src.buffer_ptrs(), dst.buffer_ptrs()
    n = None
    for a in range(3):
        si, di = src.buffers.granules_of(a), dst.buffers.granules_of(a)
        k = 0
        while k < min(len(si), len(di)) and sp[si[k]] and sp[si[k]] == dp[di[k]]:
            k += 1
        n = k if n is None else min(n, k)
    return n


def shares_params(src, dst) -> bool:
    """Whether ``dst`` holds its bf16 params in ``src``'s memory, as a state built for a Group-ZeRO
    switch normally does (the switch then leaves them in place)."""
    def param_ptrs(state):
        ptrs = _buffers_of(state)[0]
        if isinstance(state, TrainingState):
            return [ptrs[ARENA_PARAM]]
        return [ptrs[b] for b in state.buffers.granules_of(ARENA_PARAM)]

    return param_ptrs(src) == param_ptrs(dst)


def _buffers_of(state):
    """(base pointers, bytes) of a state's buffers in plan order: arenas or granules."""
    if isinstance(state, TrainingState):
        return state.arena_ptrs(), state.arena_bytes()
    return state.buffer_ptrs(), state.buffer_bytes()


def plan_dump(virtual_param_space) -> str:
    """Every parameter's registered switch as global (rank, range) pairs: who sends what to whom
    and who receives what from whom, in the order the reference walks the parameters."""
    lines = []
    for vp in virtual_param_space.all_virtual_params:
        rp = vp.reshard_plan
        lines.append(f"[reshard plan] {vp.param_position_attr}")
        if rp is None:
            lines.append("  (no switch registered)")
            continue
        for s_rank, per_dst in sorted(rp.global_send_info.items()):
            for d_rank, rng in sorted(per_dst.items()):
                lines.append(f"  send  {s_rank:>4} -> {d_rank:<4} {rng}")
        for d_rank, per_src in sorted(rp.global_recv_info.items()):
            for s_rank, rng in sorted(per_src.items()):
                lines.append(f"  recv  {d_rank:>4} <- {s_rank:<4} {rng}")
    return "\n".join(lines)
