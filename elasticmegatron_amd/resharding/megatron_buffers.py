"""Megatron's flat buffers as the caller's tensors of a per-tensor plan.

A Megatron job does not hold its state in this library's arenas.  Each
model-parallel shard owns, per (pipeline stage, dense or expert) buffer, one
flat bf16 ``param_data`` tensor of its ``_ParamAndGradBuffer``: parameters in
reverse order, each start padded to 64 elements, each bucket end padded to a
multiple of lcm(dp, 128) (the rules restated in :mod:`.ddp_layout`;
reference: elastic_megatron/resharding/resharding_dp.py:224-315).  Each rank
of the distributed optimizer owns its DP shard of every bucket of those
buffers, and its fp32 ``main`` / ``exp_avg`` / ``exp_avg_sq`` of that shard.

:class:`MegatronBuffers` names those flat tensors for one layout, with their
sizes, and hands out the per-tensor views a per-tensor plan
(:meth:`~elasticmegatron_amd.transfer.transfer.TransferManager.compile_tensors`)
reads or writes: every (rank, parameter, kind) piece at its offset inside its
rank's shard, every parameter's bf16 tensor at its ``param_index_map`` start
inside its shard's ``param_data``.  Padding lies between the views; no plan
reads or writes it.

Keys:

* ``("param", shard_key)``: the flat bf16 param buffer of a model-parallel
  shard, ``shard_key`` being ``("dense", stage, tp)`` or
  ``("expert", stage, ep, etp)``; ``BufferLayout.numel`` elements.
* ``(kind, rank, "dense" | "expert")``: the flat fp32 DP shard of a global
  rank's dense or expert buffer, ``BufferLayout.rank_shard_numel`` elements.
"""

from __future__ import annotations

from typing import Dict, List, Tuple

import numpy as np

from .layout import ARENA_PARAM, FP32_KINDS, StrategyLayout
from .tensors import TensorBuffers


class MegatronBuffers:
    """The flat buffers of every rank and shard of one layout."""

    def __init__(self, layout: StrategyLayout):
        self.layout = layout
        self.specs: List[Tuple[Tuple, str, int]] = []   # (key, "bf16" | "fp32", numel)
        for k, key in enumerate(layout.shard_keys):
            self.specs.append((("param", key), "bf16", layout.shard_numel[k]))
        for kind in FP32_KINDS:
            for g in range(layout.strategy.world_size):
                dn = layout.rank_dense_numel[g]
                en = layout.rank_numel[g] - dn
                if dn:
                    self.specs.append(((kind, g, "dense"), "fp32", dn))
                if en:
                    self.specs.append(((kind, g, "expert"), "fp32", en))
        self.numel: Dict[Tuple, int] = {key: n for key, _, n in self.specs}

    def keys(self) -> List[Tuple]:
        return [key for key, _, _ in self.specs]

    def allocate(self, device) -> Dict[Tuple, "torch.Tensor"]:
        """One uninitialised tensor per buffer (a stand-in for a job's own buffers)."""
        import torch

        dt = {"bf16": torch.bfloat16, "fp32": torch.float32}
        return {key: torch.empty(n, dtype=dt[d], device=device) for key, d, n in self.specs}

    def locate(self, arena: int, offset: int, numel: int) -> Tuple[Tuple, int]:
        """(buffer key, element offset) of arena elements [offset, offset + numel)."""
        lay = self.layout
        if arena == ARENA_PARAM:
            k = _last_at_or_below(lay.shard_base, offset)
            key, local = ("param", lay.shard_keys[k]), offset - lay.shard_base[k]
        else:
            g = _last_at_or_below(lay.rank_base, offset)
            local = offset - lay.rank_base[g]
            dn = lay.rank_dense_numel[g]
            part = "dense" if local < dn else "expert"
            key, local = (FP32_KINDS[arena], g, part), (local if local < dn else local - dn)
        if local + numel > self.numel.get(key, -1):
            raise ValueError(f"elements [{offset}, {offset + numel}) of arena {arena} leave buffer {key}")
        return key, local

    def rank_keys(self, rank: int) -> List[Tuple]:
        """The buffers global rank ``rank`` holds in a job with one rank per GPU: its fp32 DP shards
        and the bf16 ``param_data`` of the model shards it belongs to (dense, and expert with MoE)."""
        st = self.layout.strategy
        pp, _, tp = st.dense_rank_coords(rank)
        epp, _, ep, etp = st.expert_rank_coords(rank)
        wanted = [(kind, rank, part) for kind in FP32_KINDS for part in ("dense", "expert")]
        wanted += [("param", ("dense", pp, tp)), ("param", ("expert", epp, ep, etp))]
        return [key for key in wanted if key in self.numel]

    def tensor_views(self, tb: TensorBuffers, buffers: Dict[Tuple, "torch.Tensor"], partial: bool = False) -> list:
        """The tensors of ``tb`` (one side of a per-tensor plan of this layout), in buffer order, as
        views of the caller's flat ``buffers``.  With ``partial`` only the buffers given are needed
        (one rank's own, :meth:`rank_keys`), and the tensors of any other buffer come back as None."""
        if tb.layout is not self.layout and (tb.layout.space.spec, tb.layout.strategy) != \
                (self.layout.space.spec, self.layout.strategy):
            raise ValueError("the per-tensor buffers belong to another layout")
        for key, _, n in self.specs:
            t = buffers.get(key)
            if t is None and partial:
                continue
            if t is None or t.numel() != n or not t.is_contiguous():
                raise ValueError(f"buffer {key} is missing or is not a contiguous tensor of {n} elements")
        out = []
        for a, off, n in zip(tb.arena, tb.offset, tb.numel):
            key, local = self.locate(a, off, n)
            t = buffers.get(key)
            out.append(None if t is None else t[local:local + n])
        return out

    def remap_pieces(self, pieces: np.ndarray) -> np.ndarray:
        """The layout's ``emrs_piece`` records (arena ids and offsets, from ``layout.pieces()``)
        re-expressed over these buffers: buffer ids in ``specs`` order, offsets inside each buffer.
        A piece is one holder's run of a parameter, so it lies in one buffer."""
        index = {key: i for i, (key, _, _) in enumerate(self.specs)}
        out = pieces.copy()
        for r in out:
            key, local = self.locate(int(r["buf"]), int(r["buf_off"]), int(r["len"]))
            r["buf"] = index[key]
            r["buf_off"] = local
        return out

    def byte_sizes(self) -> List[int]:
        """Bytes of every buffer, in ``specs`` order."""
        return [n * (2 if d == "bf16" else 4) for _, d, n in self.specs]


def _last_at_or_below(starts: List[int], x: int) -> int:
    """Index of the last start <= x (starts ascending)."""
    lo, hi = 0, len(starts) - 1
    while lo < hi:
        mid = (lo + hi + 1) // 2
        if starts[mid] <= x:
            lo = mid
        else:
            hi = mid - 1
    return lo
