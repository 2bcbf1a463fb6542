"""Device-resident training state of every rank of one parallel strategy.

Stands in for the reference's ``TrainingState`` and ``OptimizerTensorInfo``
(elastic_megatron/megatron_manager/training_state.py:35-366,
elastic_megatron/resharding/resharding_metadata.py:19-96): instead of one
Megatron model and optimizer per process, it owns the four arenas of a
:class:`~elasticmegatron_amd.resharding.layout.StrategyLayout` on one device
(fp32 main / exp_avg / exp_avg_sq of every rank, bf16 params of every
model-parallel shard) and hands out per-(rank, parameter) views with the
reference's names.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch

from .. import _native
from ..resharding.layout import ARENA_NAMES, StrategyLayout, split_vocab_rows
from ..resharding.util import Range


@dataclass
class OptimizerTensorInfo:
    """Views of one rank's piece of one parameter (resharding_metadata.py:19-40)."""

    main_weight: torch.Tensor
    exp_avg: torch.Tensor
    exp_avg_sq: torch.Tensor
    optimizer_tensor_range_in_model_param: Range   # param-local flat range this rank owns
    model_param_shape: Tuple[int, ...]             # TP-local shape

    @property
    def optimizer_tensors(self) -> List[torch.Tensor]:
        return [self.main_weight, self.exp_avg, self.exp_avg_sq]


# Capacity granule of fp32 arenas that are allocated and released one at a time: arenas of two
# layouts of one model differ by a few MB of padding, and rounding both up to this granule lets the
# block a released source arena leaves in torch's caching allocator serve the next destination
# arena, with no call to the driver.
ARENA_GRANULE_BYTES = 1 << 30


class TrainingState:
    def __init__(self, layout: StrategyLayout, main: torch.Tensor, exp_avg: torch.Tensor,
                 exp_avg_sq: torch.Tensor, param: torch.Tensor, granule_bytes: int = 0):
        self.layout = layout
        self.main = main
        self.exp_avg = exp_avg
        self.exp_avg_sq = exp_avg_sq
        self.param = param
        self.granule_bytes = granule_bytes

    @property
    def parallel_strategy(self):
        return self.layout.strategy

    @classmethod
    def allocate(cls, layout: StrategyLayout, device=None, param: Optional[torch.Tensor] = None,
                 kinds: Tuple[int, ...] = (0, 1, 2), granule_bytes: int = 0) -> "TrainingState":
        """Uninitialised arenas for ``layout``; ``param`` may alias an existing bf16 arena.

        ``kinds``: the fp32 arenas to allocate now (0 main, 1 exp_avg,
        2 exp_avg_sq); the others start empty and are allocated later with
        :meth:`allocate_kind`, as a staged switch does.  ``granule_bytes``:
        round each fp32 arena's capacity up to a multiple of it (see
        ``ARENA_GRANULE_BYTES``); the arena itself is a view of the exact size.
        """
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        if param is None:
            param = torch.empty(layout.bf16_numel, dtype=torch.bfloat16, device=dev)
        elif param.numel() != layout.bf16_numel or param.dtype != torch.bfloat16:
            raise ValueError("aliased param arena does not match the layout")
        empty = torch.empty(0, dtype=torch.float32, device=dev)
        st = cls(layout, empty, empty, empty, param, granule_bytes)
        for k in kinds:
            st.allocate_kind(k)
        return st

    _KINDS = ("main", "exp_avg", "exp_avg_sq")

    def allocate_kind(self, kind: int) -> None:
        """Allocate fp32 arena ``kind`` (0 main, 1 exp_avg, 2 exp_avg_sq) if it is empty."""
        name, n = self._KINDS[kind], self.layout.fp32_numel
        if getattr(self, name).numel() == 0 and n:
            g = max(1, self.granule_bytes // 4)
            cap = (n + g - 1) // g * g
            setattr(self, name, torch.empty(cap, dtype=torch.float32, device=self.device)[:n])

    def release_kind(self, kind: int) -> None:
        """Free fp32 arena ``kind``, as the reference releases each optimizer tensor once it has been
        sent (resharding_metadata.py:58-65): its storage is resized to nothing, so the memory goes
        back to torch's caching allocator even where views of it are still held."""
        name = self._KINDS[kind]
        t = getattr(self, name)
        if t.numel():
            t.untyped_storage().resize_(0)
        setattr(self, name, torch.empty(0, dtype=torch.float32, device=self.device))

    # ----- arenas -----
    def arenas(self) -> List[torch.Tensor]:
        return [self.main, self.exp_avg, self.exp_avg_sq, self.param]

    def arena_ptrs(self) -> List[int]:
        return [t.data_ptr() for t in self.arenas()]

    def arena_bytes(self) -> List[int]:
        return [t.numel() * t.element_size() for t in self.arenas()]

    @property
    def device(self) -> torch.device:
        return self.param.device

    def release_optimizer(self) -> None:
        """Drop the fp32 arenas (training_state.py:313-315)."""
        for k in range(3):
            self.release_kind(k)

    # ----- per-(rank, parameter) views -----
    def optimizer_tensor_info(self, vp, rank: int) -> Optional[OptimizerTensorInfo]:
        for h in self.layout.fp32_holders(vp):
            if h.rank == rank:
                sl = slice(h.offset, h.offset + h.hi - h.lo)
                return OptimizerTensorInfo(self.main[sl], self.exp_avg[sl], self.exp_avg_sq[sl],
                                           Range(h.lo, h.hi), vp.local_shape(self.layout.strategy))
        return None

    def model_param(self, vp, tp_rank: int = 0) -> Optional[torch.Tensor]:
        """bf16 TP-local tensor of ``vp`` held by TP rank ``tp_rank`` of its stage."""
        for h in self.layout.bf16_holders(vp):
            if h.tp_rank == tp_rank:
                return self.param[h.offset:h.offset + h.hi - h.lo].view(vp.local_shape(self.layout.strategy))
        return None

    # ----- synthetic workload -----
    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def fill_synthetic(self, seed: int, params=None, fp32: bool = True, bf16: bool = True) -> None:
        """Write the seeded synthetic values of every stored element (see csrc/synth.hip)."""
        pcs = self.layout.pieces(params, include_bf16=bf16, include_fp32=fp32)
        with torch.cuda.device(self.device):
            _native.synth_fill(pcs, self.arena_ptrs(), self.arena_bytes(), seed, self._stream())

    def verify_synthetic(self, seed: int, params=None, fp32: bool = True, bf16: bool = True,
                         vocab_rows: Optional[int] = None):
        """(mismatching elements, first bad element) against the seeded synthetic values.

        ``vocab_rows``: vocabulary rows at and past it must be zero instead
        (new padding rows after a switch to a larger padded vocabulary).
        """
        pcs = self.layout.pieces(params, include_bf16=bf16, include_fp32=fp32)
        zero = []
        if vocab_rows is not None:
            pcs, zero = split_vocab_rows(self.layout, pcs, vocab_rows)
        with torch.cuda.device(self.device):
            bad, first = _native.synth_verify(pcs, self.arena_ptrs(), self.arena_bytes(), seed, self._stream())
            arenas = self.arenas()
            for buf, off, n in zero:
                a = arenas[buf]
                bits = a.view(torch.int16 if a.dtype == torch.bfloat16 else torch.int32)[off:off + n]
                bad += int(torch.count_nonzero(bits))
        if first is not None:
            p = pcs[first[0]]
            first = dict(arena=ARENA_NAMES[int(p["buf"])], param_id=int(p["param_id"]), kind=int(p["kind"]),
                         element=int(first[1]), piece_offset=int(p["buf_off"]))
        return bad, first
