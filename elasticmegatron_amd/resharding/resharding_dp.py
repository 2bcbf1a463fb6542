"""Data- and expert-parallel resharding info.

Mirrors elastic_megatron/resharding/resharding_dp.py:
``ExpertParallelReshardingInfo`` (:21-34), ``DataParallelReshardingInfo``
(:37-133), ``intersect_range`` / ``intersect_sub_ranges`` (:136-152) and
``get_params_dp_distribution`` (:318-386).  The Megatron buffer layout the
reference obtains from a mocked ``_ParamAndGradBuffer`` comes from
:mod:`.ddp_layout`.
"""

from __future__ import annotations

from typing import TYPE_CHECKING, Any, Dict, List, Optional

from ..megatron_manager.parallel_strategy import ParallelStrategy, global_rank_of
from .ddp_layout import build_buffer_layout, dp_distribution
from .resharding_pp import PipelineParallelReshardingInfo
from .util import Range

if TYPE_CHECKING:
    from .model_spec import ModelSpec
    from .virtual_param import VirtualParam


class ExpertParallelReshardingInfo:
    def __init__(self, expert_id: int, src: ParallelStrategy, dst: ParallelStrategy, num_experts: int):
        self.expert_id = expert_id
        self.src_expert_parallel_rank = expert_id // src.expert_num_per_ep_rank(num_experts)
        self.dst_expert_parallel_rank = expert_id // dst.expert_num_per_ep_rank(num_experts)


def intersect_range(main: Range, sub: Range) -> Optional[Range]:
    lo, hi = max(main.start, sub.start), min(main.end, sub.end)
    return Range(lo, hi) if lo < hi else None


def intersect_sub_ranges(main: Range, subs: Dict[Any, Range]) -> Dict[Any, Range]:
    out = {}
    for k, r in subs.items():
        x = intersect_range(main, r)
        if x is not None:
            out[k] = x
    return out


class DataParallelReshardingInfo:
    """DP distributions of one parameter keyed by global rank, and the aligned ranks.

    The reference converts DP ranks to global ranks with the *caller's* TP
    rank (resharding_dp.py:100); with every rank simulated here the TP rank
    is an argument.  The aligned rank is the lowest DP rank holding a piece
    (resharding_dp.py:120-133).
    """

    def __init__(self, src_dp_distribution: Dict[int, Range], dst_dp_distribution: Dict[int, Range],
                 src: ParallelStrategy, dst: ParallelStrategy,
                 pp_info: PipelineParallelReshardingInfo,
                 ep_info: Optional[ExpertParallelReshardingInfo],
                 src_tp_rank: int = 0, dst_tp_rank: int = 0):
        self.src_dp_distribution = src_dp_distribution
        self.dst_dp_distribution = dst_dp_distribution
        self.src_pp_rank = pp_info.src_pp_rank
        self.dst_pp_rank = pp_info.dst_pp_rank
        self.is_expert = ep_info is not None
        self.src_ep_rank = ep_info.src_expert_parallel_rank if ep_info else None
        self.dst_ep_rank = ep_info.dst_expert_parallel_rank if ep_info else None
        self.src_dp_distribution_with_global_rank = {
            global_rank_of(src, self.src_pp_rank, dp, self.src_ep_rank, src_tp_rank): r
            for dp, r in src_dp_distribution.items()
        }
        self.dst_dp_distribution_with_global_rank = {
            global_rank_of(dst, self.dst_pp_rank, dp, self.dst_ep_rank, dst_tp_rank): r
            for dp, r in dst_dp_distribution.items()
        }
        self.src_aligned_dp_rank = next(iter(src_dp_distribution))
        self.dst_aligned_dp_rank = next(iter(dst_dp_distribution))
        self.src_aligned_global_rank = next(iter(self.src_dp_distribution_with_global_rank), None)
        self.dst_aligned_global_rank = next(iter(self.dst_dp_distribution_with_global_rank), None)


def bucket_size_for(spec: "ModelSpec", strategy: ParallelStrategy, disable_bucketing: bool) -> Optional[int]:
    """resharding_dp.py:332-336."""
    size = spec.ddp_bucket_size
    if size is None:
        size = max(40_000_000, 1_000_000 * strategy.optimizer_data_parallel_size)
    if not spec.overlap_grad_reduce or disable_bucketing:
        return None
    return size


def stage_buffer_layouts(params: List["VirtualParam"], strategy: ParallelStrategy, spec: "ModelSpec",
                         disable_bucketing: bool):
    """Megatron buffers of one pipeline stage.

    Returns ``(dense_params, dense_layout, expert_params_by_ep, expert_layout)``;
    the expert layout is computed for EP rank 0's experts and shared by every
    EP rank, whose experts map onto it in order (resharding_dp.py:354-375).
    """
    bucket_size = bucket_size_for(spec, strategy, disable_bucketing)
    dense = [p for p in params if not p.is_expert]
    experts: Dict[int, List["VirtualParam"]] = {}
    if spec.is_moe:
        per_rank = strategy.expert_num_per_ep_rank(spec.num_experts)
        for p in params:
            if p.is_expert:
                experts.setdefault(p.expert_id // per_rank, []).append(p)
    dense_layout = None
    if dense:
        dense_layout = build_buffer_layout(
            [p.numel_at(strategy) for p in dense], strategy.optimizer_data_parallel_size, bucket_size,
            [p.shared_embedding for p in dense], spec.use_distributed_optimizer)
    expert_layout = None
    if experts:
        ep0 = experts[0]
        for r, lst in experts.items():
            assert len(lst) == len(ep0), "EP ranks hold different expert parameter lists"
        expert_layout = build_buffer_layout(
            [p.numel_at(strategy) for p in ep0], strategy.expert_data_parallel_size, bucket_size,
            None, spec.use_distributed_optimizer)
    return dense, dense_layout, experts, expert_layout


def get_params_dp_distribution(params: List["VirtualParam"], strategy: ParallelStrategy, spec: "ModelSpec",
                               disable_bucketing: bool = False) -> Dict["VirtualParam", Dict[int, Range]]:
    """param -> {dp_rank: param-local Range}, dp ranks ascending (resharding_dp.py:318-386)."""
    dense, dl, experts, el = stage_buffer_layouts(params, strategy, spec, disable_bucketing)
    out: Dict["VirtualParam", Dict[int, Range]] = {}
    if dl is not None:
        for i, d in dp_distribution(dl).items():
            out[dense[i]] = {r: Range(lo, hi) for r, (lo, hi) in d.items()}
    if el is not None:
        dist = dp_distribution(el)
        for lst in experts.values():
            for i, p in enumerate(lst):
                out[p] = {r: Range(lo, hi) for r, (lo, hi) in dist[i].items()}
    assert len(out) == len(params)
    return out
