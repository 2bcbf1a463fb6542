"""Device-memory layout of every rank's state under one parallel strategy.

All ranks of a layout live in one device's HBM, in four arenas:

* ``main``, ``exp_avg``, ``exp_avg_sq`` (fp32): the concatenation, over global
  ranks, of each rank's flat optimizer shard.  A rank's shard is its DP shard
  of every bucket of its stage's dense buffer, then of its expert buffer, in
  bucket order -- the view Megatron's distributed optimizer has of the grad
  buffer.  A parameter piece sits at its offset inside the bucket shard;
  padding is never read or written.
* ``param`` (bf16): one full Megatron param buffer per model-parallel shard,
  dense shards keyed (stage, tp) and expert shards keyed (stage, ep, etp).
  Data-parallel replicas of a shard are one buffer; the reference replicates
  them with an all-gather after casting main to bf16
  (elastic_megatron/megatron_manager/training_state.py:176-197).

The reference keeps one tensor per (parameter, rank) instead
(elastic_megatron/resharding/resharding_metadata.py:19-40); the pieces and
their contents are the same.

Every TP-local tensor is viewed as 2-D ``(rows, cols)`` and mapped onto the
full (TP = 1) tensor by :class:`Geometry`: a row offset per band of local
rows and one column offset.  Row splits use one band, the fused SwiGLU fc1
``[W_t; V_t]`` two bands, column splits a column offset.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import numpy as np

from ..megatron_manager.parallel_strategy import ParallelStrategy, global_rank_of
from .ddp_layout import BufferLayout, dp_distribution, piece_offset_in_rank_shard
from .resharding_dp import stage_buffer_layouts

FP32_KINDS = ("main", "exp_avg", "exp_avg_sq")
ARENA_MAIN, ARENA_EXP_AVG, ARENA_EXP_AVG_SQ, ARENA_PARAM = 0, 1, 2, 3
ARENA_NAMES = ("main", "exp_avg", "exp_avg_sq", "param")
_RANK_ALIGN = 64     # fp32 elements (256 bytes)
_SHARD_ALIGN = 128   # bf16 elements (256 bytes)

# Record layouts shared with include/emrs.h.
SEGMENT_DTYPE = np.dtype([
    ("src_buf", "<u4"), ("dst_buf", "<u4"), ("elem_bytes", "<u4"), ("flags", "<u4"),
    ("src_off", "<u8"), ("dst_off", "<u8"), ("len", "<u8"), ("rows", "<u8"),
    ("src_stride", "<u8"), ("dst_stride", "<u8"),
    ("aux_buf", "<u4"), ("reserved", "<u4"), ("aux_off", "<u8"), ("aux_stride", "<u8"),
])
SEG_CAST_BF16 = 1
SEG_ZERO_FILL = 2
SEG_DUP = 4
PIECE_DTYPE = np.dtype([
    ("buf", "<u4"), ("param_id", "<u4"), ("kind", "<u4"), ("reserved", "<u4"),
    ("buf_off", "<u8"), ("len", "<u8"), ("local_start", "<u8"), ("local_cols", "<u8"),
    ("full_cols", "<u8"), ("band_rows", "<u8"), ("row_off", "<u8"), ("row_off2", "<u8"),
    ("col_off", "<u8"),
])
assert SEGMENT_DTYPE.itemsize == 88 and PIECE_DTYPE.itemsize == 88


def _align(n: int, a: int) -> int:
    return -(-n // a) * a


def view2d(shape: Tuple[int, ...], partition_dim: int) -> Tuple[int, int]:
    """2-D view of a parameter shape: 1-D tensors split along dim 0 are columns of width 1."""
    if len(shape) == 2:
        return shape[0], shape[1]
    if partition_dim == 0:
        return shape[0], 1
    return 1, shape[0]


@dataclass(frozen=True)
class Geometry:
    """Placement of one TP rank's local tensor inside the full tensor."""

    rows: int                 # local rows
    cols: int                 # local cols
    full_cols: int
    band_rows: int            # local rows of the first band (== rows for one band)
    row_off: int              # full row of local row 0
    row_off2: int             # full row of local row band_rows (second band)
    col_off: int              # full col of local col 0

    def bands(self):
        """(local_row_lo, local_row_hi, full_row_of_local_row_lo)."""
        if self.band_rows >= self.rows:
            return [(0, self.rows, self.row_off)]
        return [(0, self.band_rows, self.row_off), (self.band_rows, self.rows, self.row_off2)]


def geometry(vp, tp_size: int, tp_rank: int) -> Geometry:
    tpa = vp.tensor_parallel_attr
    R, C = view2d(vp.full_shape, tpa.partition_dim)
    if not tpa.tensor_model_parallel or tp_size == 1:
        return Geometry(R, C, C, R, 0, 0, 0)
    pdim = tpa.partition_dim
    if len(vp.full_shape) == 1:
        pdim = 0
    if pdim == 0:
        rl = R // tp_size
        if vp.is_swiglu_fc:
            half, f = rl // 2, R // 2
            return Geometry(rl, C, C, half, tp_rank * half, f + tp_rank * half, 0)
        return Geometry(rl, C, C, rl, tp_rank * rl, 0, 0)
    cl = C // tp_size
    return Geometry(R, cl, C, R, 0, 0, tp_rank * cl)


@dataclass(frozen=True)
class Holder:
    """A contiguous run of one parameter's local elements in an arena."""

    rank: int                 # global rank (fp32) or shard index (bf16)
    tp_rank: int
    lo: int                   # local flat range [lo, hi)
    hi: int
    offset: int               # arena element offset of local element lo
    instance: int = 0         # distributed-optimizer instance (Group ZeRO)


@dataclass
class _ParamPlace:
    stage: int
    expert_ep: Optional[int]          # EP rank holding the expert, None for dense
    index: int                        # position in its buffer's parameter list
    dist: Dict[int, Tuple[int, int]]  # dp rank -> local (lo, hi)


class StrategyLayout:
    def __init__(self, space, strategy: ParallelStrategy):
        spec = space.spec
        self.space = space
        self.strategy = strategy
        self.spec = spec
        strategy.validate_for(spec.num_layers, spec.num_experts)
        if spec.is_moe and strategy.num_distributed_optimizer_instances > 1:
            raise NotImplementedError("Group ZeRO with expert parallelism is not supported")
        pp = strategy.pipeline_model_parallel_size
        self.stage_dense: List[Optional[BufferLayout]] = []
        self.stage_expert: List[Optional[BufferLayout]] = []
        self.place: Dict[int, _ParamPlace] = {}
        for sid, params in enumerate(space.stages(pp)):
            disable = sid > 0 or spec.overlap_param_gather_with_optimizer_step
            dense, dl, experts, el = stage_buffer_layouts(params, strategy, spec, disable)
            self.stage_dense.append(dl)
            self.stage_expert.append(el)
            if dl is not None:
                dd = dp_distribution(dl)
                for i, p in enumerate(dense):
                    self.place[p.global_index] = _ParamPlace(sid, None, i, dd[i])
            if el is not None:
                ed = dp_distribution(el)
                for ep, lst in experts.items():
                    for i, p in enumerate(lst):
                        self.place[p.global_index] = _ParamPlace(sid, ep, i, ed[i])

        W = strategy.world_size
        # fp32 arena: one flat shard per global rank.
        self.rank_dense_numel: List[int] = []
        self.rank_numel: List[int] = []
        self.rank_base: List[int] = []
        acc = 0
        for g in range(W):
            pp_d, _, _ = strategy.dense_rank_coords(g)
            dl, el = self.stage_dense[pp_d], self.stage_expert[pp_d]
            dn = dl.rank_shard_numel if dl is not None else 0
            en = el.rank_shard_numel if el is not None else 0
            self.rank_dense_numel.append(dn)
            self.rank_numel.append(dn + en)
            self.rank_base.append(acc)
            acc += _align(dn + en, _RANK_ALIGN)
        self.fp32_numel = max(acc, _RANK_ALIGN)

        # bf16 arena: one full param buffer per model-parallel shard.
        self.shard_keys: List[Tuple] = []
        self.shard_base: List[int] = []
        self.shard_numel: List[int] = []
        self._shard_index: Dict[Tuple, int] = {}
        acc = 0
        tp, etp, ep = (strategy.tensor_model_parallel_size, strategy.expert_tensor_parallel_size,
                       strategy.expert_model_parallel_size)
        for sid in range(pp):
            if self.stage_dense[sid] is not None:
                for t in range(tp):
                    acc = self._add_shard(("dense", sid, t), self.stage_dense[sid].numel, acc)
            if self.stage_expert[sid] is not None:
                for e in range(ep):
                    for t in range(etp):
                        acc = self._add_shard(("expert", sid, e, t), self.stage_expert[sid].numel, acc)
        self.bf16_numel = max(acc, _SHARD_ALIGN)

    def _add_shard(self, key, numel: int, acc: int) -> int:
        self._shard_index[key] = len(self.shard_keys)
        self.shard_keys.append(key)
        self.shard_base.append(acc)
        self.shard_numel.append(numel)
        return acc + _align(numel, _SHARD_ALIGN)

    # ----- queries -----
    @property
    def payload_numel(self) -> int:
        """Elements of model state held once (no replicas)."""
        return sum(self.space.all_virtual_params[g].numel() for g in self.place)

    def tp_size_of(self, vp) -> int:
        return vp.tp_size_at(self.strategy)

    def geometry(self, vp, tp_rank: int) -> Geometry:
        return geometry(vp, self.tp_size_of(vp), tp_rank)

    def has_param(self, vp) -> bool:
        return vp.global_index in self.place

    def stage_of(self, vp) -> int:
        return self.place[vp.global_index].stage

    def dp_distribution(self, vp) -> Dict[int, Tuple[int, int]]:
        return self.place[vp.global_index].dist

    def fp32_holders(self, vp) -> List[Holder]:
        """Every (rank, piece) holding fp32 state of ``vp``, replicas included."""
        pl = self.place[vp.global_index]
        st = self.strategy
        out: List[Holder] = []
        if pl.expert_ep is None:
            dl = self.stage_dense[pl.stage]
            part = st.optimizer_data_parallel_size
            for inst in range(st.num_distributed_optimizer_instances):
                for t in range(st.tensor_model_parallel_size):
                    for r, (lo, hi) in pl.dist.items():
                        g = self._dense_rank(pl.stage, inst * part + r, t)
                        off = self.rank_base[g] + piece_offset_in_rank_shard(dl, pl.index, r, lo)
                        out.append(Holder(g, t, lo, hi, off, inst))
            return out
        el = self.stage_expert[pl.stage]
        for t in range(st.expert_tensor_parallel_size):
            for r, (lo, hi) in pl.dist.items():
                g = global_rank_of(st, pl.stage, r, pl.expert_ep, t)
                off = self.rank_base[g] + self.rank_dense_numel[g] + piece_offset_in_rank_shard(el, pl.index, r, lo)
                out.append(Holder(g, t, lo, hi, off))
        return out

    def _dense_rank(self, stage: int, dp_full: int, tp_rank: int) -> int:
        """Global rank of a dense shard; equals resharding.py:19-51 with one optimizer instance."""
        st = self.strategy
        tp = st.tensor_model_parallel_size
        return stage * (st.data_parallel_size * st.context_parallel_size * tp) + dp_full * tp + tp_rank

    def bf16_holders(self, vp) -> List[Holder]:
        """Every model-parallel shard holding the whole local bf16 tensor of ``vp``."""
        pl = self.place[vp.global_index]
        st = self.strategy
        out: List[Holder] = []
        n = vp.numel_at(st)
        if pl.expert_ep is None:
            start = self.stage_dense[pl.stage].param_index_map[pl.index][0]
            for t in range(st.tensor_model_parallel_size):
                k = self._shard_index[("dense", pl.stage, t)]
                out.append(Holder(k, t, 0, n, self.shard_base[k] + start))
            return out
        start = self.stage_expert[pl.stage].param_index_map[pl.index][0]
        for t in range(st.expert_tensor_parallel_size):
            k = self._shard_index[("expert", pl.stage, pl.expert_ep, t)]
            out.append(Holder(k, t, 0, n, self.shard_base[k] + start))
        return out

    def rank_fp32_slice(self, g: int) -> Tuple[int, int]:
        return self.rank_base[g], self.rank_base[g] + self.rank_numel[g]

    # ----- synthetic-data descriptors -----
    def pieces(self, params=None, include_bf16: bool = True, include_fp32: bool = True) -> np.ndarray:
        """emrs_piece records covering every stored element of ``params``.

        A tied output layer is described with the word embedding's id: it
        holds the same values.
        """
        rows = []
        vps = params if params is not None else [self.space.all_virtual_params[g] for g in sorted(self.place)]
        for vp in vps:
            vid = self.space.value_source(vp).global_index
            if include_fp32:
                for h in self.fp32_holders(vp):
                    geo = self.geometry(vp, h.tp_rank)
                    for kind in (1, 2, 3):
                        rows.append(_piece_row(kind - 1, vid, kind, h, geo))
            if include_bf16:
                for h in self.bf16_holders(vp):
                    geo = self.geometry(vp, h.tp_rank)
                    rows.append(_piece_row(ARENA_PARAM, vid, 0, h, geo))
        arr = np.zeros(len(rows), dtype=PIECE_DTYPE)
        if rows:
            arr[:] = rows
        return arr


VOCAB_PARAM_NAMES = ("embedding.word_embeddings.weight", "output_layer.weight")


def split_vocab_rows(layout: "StrategyLayout", pieces: np.ndarray, vocab_rows: int):
    """Cut the pieces of the vocabulary parameters at full row ``vocab_rows``.

    Returns (pieces holding rows below it, [(buf, offset, len)] of the
    elements at or past it): after a switch to a larger padded vocabulary,
    the first keep their values and the second are new padding rows.
    """
    vocab_ids = {vp.global_index for vp in layout.space.all_virtual_params if vp.name in VOCAB_PARAM_NAMES}
    keep, zero = [], []
    for p in pieces:
        n = int(p["len"])
        if int(p["param_id"]) not in vocab_ids or int(p["band_rows"]):
            keep.append(p)
            continue
        # Row-split vocabulary shards: full row = local row + row_off.
        cut = max(0, vocab_rows - int(p["row_off"])) * int(p["local_cols"]) - int(p["local_start"])
        cut = min(max(cut, 0), n)
        if cut:
            q = p.copy()
            q["len"] = cut
            keep.append(q)
        if cut < n:
            zero.append((int(p["buf"]), int(p["buf_off"]) + cut, n - cut))
    arr = np.zeros(len(keep), dtype=PIECE_DTYPE)
    if keep:
        arr[:] = keep
    return arr, zero


def _piece_row(buf: int, pid: int, kind: int, h: Holder, geo: Geometry):
    return (buf, pid, kind, 0, h.offset, h.hi - h.lo, h.lo, geo.cols, geo.full_cols,
            geo.band_rows if geo.band_rows < geo.rows else 0, geo.row_off, geo.row_off2, geo.col_off)
