"""Per-parameter reshard plan: global send/recv maps.

Mirrors ``get_global_rank`` and ``ReshardPlan`` of the reference
(elastic_megatron/resharding/resharding.py:19-162): the TP send/recv maps are
lifted from TP ranks to global ranks at the parameter's pipeline stage, its
expert-parallel rank, and the aligned (lowest) data-parallel rank.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Optional

from ..megatron_manager.parallel_strategy import ParallelStrategy, global_rank_of
from .resharding_dp import DataParallelReshardingInfo, ExpertParallelReshardingInfo
from .resharding_pp import PipelineParallelReshardingInfo
from .resharding_tp import TensorParallelReshardingInfo
from .util import ParamRange


def get_global_rank(pipeline_model_parallel_rank: int, data_parallel_rank: int,
                    expert_model_parallel_rank: Optional[int], tensor_model_parallel_rank: int,
                    parallel_strategy: ParallelStrategy) -> int:
    """Order TP -> EP -> DP -> PP (resharding.py:19-51)."""
    return global_rank_of(parallel_strategy, pipeline_model_parallel_rank, data_parallel_rank,
                          expert_model_parallel_rank, tensor_model_parallel_rank)


@dataclass
class ReshardPlan:
    tensor_parallel_resharding_info: TensorParallelReshardingInfo
    pipeline_parallel_resharding_info: PipelineParallelReshardingInfo
    data_parallel_resharding_info: DataParallelReshardingInfo
    expert_parallel_reshardign_info: Optional[ExpertParallelReshardingInfo]
    src_parallel_strategy: ParallelStrategy
    dst_parallel_strategy: ParallelStrategy
    global_send_info: Optional[Dict[int, Dict[int, ParamRange]]] = field(init=False, default=None)
    global_recv_info: Optional[Dict[int, Dict[int, ParamRange]]] = field(init=False, default=None)

    def __post_init__(self):
        ep = self.expert_parallel_reshardign_info
        if ep is not None:  # resharding.py:64-79
            assert self.src_parallel_strategy.get_tensor_model_parallel_size(True) == 1
            assert self.dst_parallel_strategy.get_tensor_model_parallel_size(True) == 1
            assert len(self.tensor_parallel_resharding_info.send_info) == 1
            assert len(self.tensor_parallel_resharding_info.recv_info) == 1
            self.src_ep_rank = ep.src_expert_parallel_rank
            self.dst_ep_rank = ep.dst_expert_parallel_rank
        else:
            self.src_ep_rank = None
            self.dst_ep_rank = None
        self.src_pp_rank = self.pipeline_parallel_resharding_info.src_pp_rank
        self.dst_pp_rank = self.pipeline_parallel_resharding_info.dst_pp_rank
        if self.src_pp_rank == -1 or self.dst_pp_rank == -1:
            return
        self.src_dp_rank = self.data_parallel_resharding_info.src_aligned_dp_rank
        self.dst_dp_rank = self.data_parallel_resharding_info.dst_aligned_dp_rank
        self.global_send_info = self._lift(self.tensor_parallel_resharding_info.send_info, send=True)
        self.global_recv_info = self._lift(self.tensor_parallel_resharding_info.recv_info, send=False)

    def _src_global(self, tp_rank: int) -> int:
        return get_global_rank(self.src_pp_rank, self.src_dp_rank, self.src_ep_rank, tp_rank,
                               self.src_parallel_strategy)

    def _dst_global(self, tp_rank: int) -> int:
        return get_global_rank(self.dst_pp_rank, self.dst_dp_rank, self.dst_ep_rank, tp_rank,
                               self.dst_parallel_strategy)

    def _lift(self, tp_map: Dict[int, Dict[int, ParamRange]], send: bool) -> Dict[int, Dict[int, ParamRange]]:
        outer = self._src_global if send else self._dst_global
        inner = self._dst_global if send else self._src_global
        return {outer(a): {inner(b): r for b, r in peers.items()} for a, peers in tp_map.items()}
