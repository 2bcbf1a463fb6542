"""Parallel strategy: sizes and rank arithmetic of one TP/PP/CP/DP/EP layout.

Mirrors ``ParallelStrategy`` of the reference
(elastic_megatron/megatron_manager/parallel_strategy.py:10-147, :234-263)
without its process-group side: the reference reads the caller's rank and
Megatron's ``parallel_state`` to learn its own coordinates, while here every
rank of the layout is simulated on one device, so coordinates are computed
from a global rank with the rank order ``tp-cp-ep-dp-pp``
(parallel_strategy.py:21; elastic_megatron/megatron_manager/rank_generator.py:9-36).
Model-dependent checks (layers divisible by PP, experts divisible by EP) run
in :meth:`ParallelStrategy.validate_for` instead of reading global args.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Optional, Tuple


@dataclass(frozen=True)
class ParallelStrategy:
    world_size: int
    tensor_model_parallel_size: int
    pipeline_model_parallel_size: int
    context_parallel_size: int = 1
    num_distributed_optimizer_instances: int = 1
    expert_model_parallel_size: int = 1
    expert_tensor_parallel_size: Optional[int] = None
    # The fields below are not part of a strategy's identity: the reference
    # compares and hashes str(self), which prints only the seven sizes above
    # (parallel_strategy.py:223-232).  Strategies that differ only here are
    # equal, hash alike and share every plan and layout cache.
    sequence_parallel: Optional[bool] = field(default=None, compare=False)
    order: str = field(default="tp-cp-ep-dp-pp", compare=False)
    ranks: Optional[Tuple[int, ...]] = field(default=None, compare=False)

    def __post_init__(self):
        # parallel_strategy.py:24-47
        if self.world_size <= 0:
            raise ValueError("world_size must be positive")
        tp, pp, cp = (
            self.tensor_model_parallel_size,
            self.pipeline_model_parallel_size,
            self.context_parallel_size,
        )
        if min(tp, pp, cp, self.num_distributed_optimizer_instances, self.expert_model_parallel_size) < 1:
            raise ValueError("parallel sizes must be >= 1")
        if self.world_size % tp or self.world_size % pp:
            raise ValueError(f"world_size {self.world_size} not divisible by TP {tp} and PP {pp}")
        if self.world_size % (tp * pp * cp):
            raise ValueError(f"world_size {self.world_size} not divisible by TP*PP*CP {tp * pp * cp}")
        if tp == 1 and self.sequence_parallel:
            raise ValueError("Sequence parallel is not supported with tensor model parallel size 1")
        if self.sequence_parallel is None:
            object.__setattr__(self, "sequence_parallel", tp > 1)
        if self.expert_tensor_parallel_size is None:  # parallel_strategy.py:108-110
            object.__setattr__(self, "expert_tensor_parallel_size", tp)
        # Group ZeRO (parallel_strategy.py:99-106).  The reference also demands
        # CP > 1 there; that precondition concerns Megatron's group building,
        # not the data movement, and is not required here.
        if self.data_parallel_size % self.num_distributed_optimizer_instances:
            raise ValueError("data parallel size not divisible by num_distributed_optimizer_instances")
        etmp = self.expert_tensor_parallel_size * self.expert_model_parallel_size * pp
        if self.world_size % etmp:  # parallel_strategy.py:116-122
            raise RuntimeError(
                f"decoder world_size ({self.world_size}) is not divisible by "
                f"expert_tensor_model_pipeline_parallel size ({etmp})"
            )
        if self.order != "tp-cp-ep-dp-pp":
            raise ValueError("only the rank order tp-cp-ep-dp-pp is supported")

    # ----- sizes (parallel_strategy.py:31-36, :108-147) -----
    @property
    def model_parallel_size(self) -> int:
        return self.tensor_model_parallel_size * self.pipeline_model_parallel_size

    @property
    def total_model_size(self) -> int:
        return self.model_parallel_size * self.context_parallel_size

    @property
    def data_parallel_size(self) -> int:
        return self.world_size // self.total_model_size

    @property
    def expert_data_parallel_size(self) -> int:
        return self.world_size // (
            self.expert_tensor_parallel_size * self.expert_model_parallel_size * self.pipeline_model_parallel_size
        )

    def get_data_parallel_world_size(self, with_context_parallel: bool = False, partial_data_parallel: bool = False) -> int:
        if with_context_parallel:
            if partial_data_parallel:
                return (
                    self.data_parallel_size
                    * self.context_parallel_size
                    // self.num_distributed_optimizer_instances
                )
            return self.data_parallel_size * self.context_parallel_size
        if partial_data_parallel:
            raise AssertionError("Partial DP for Optimizer needs to include CP")
        return self.data_parallel_size

    @property
    def optimizer_data_parallel_size(self) -> int:
        """DP size over which the distributed optimizer shards dense params."""
        return self.get_data_parallel_world_size(with_context_parallel=True, partial_data_parallel=True)

    def get_tensor_model_parallel_size(self, is_expert: bool) -> int:
        return self.expert_tensor_parallel_size if is_expert else self.tensor_model_parallel_size

    def expert_num_per_ep_rank(self, num_experts: int) -> int:
        if num_experts % self.expert_model_parallel_size:
            raise AssertionError("num_experts must be divisible by expert_model_parallel_size")
        return num_experts // self.expert_model_parallel_size

    def transformer_layer_num_per_stage(self, num_layers: int) -> int:
        if num_layers < 1 or num_layers % self.pipeline_model_parallel_size:
            raise AssertionError("num_layers must be divisible by pipeline_model_parallel_size")
        return num_layers // self.pipeline_model_parallel_size

    def validate_for(self, num_layers: int, num_experts: Optional[int]) -> None:
        """Model-dependent checks of the reference (parallel_strategy.py:51-77)."""
        self.transformer_layer_num_per_stage(num_layers)
        if num_experts:
            self.expert_num_per_ep_rank(num_experts)
            if self.expert_tensor_parallel_size != 1:
                raise AssertionError("Only support TPE==1 for MoE resharding")

    # ----- rank arithmetic (resharding/resharding.py:19-51) -----
    def dense_rank_coords(self, global_rank: int) -> Tuple[int, int, int]:
        """(pp_rank, dp_rank, tp_rank) of a global rank; dp indexes the whole DP-CP group.

        With Group ZeRO the DP-CP group is cut into contiguous blocks of
        ``optimizer_data_parallel_size`` ranks, one per optimizer instance:
        the instance is ``dp_rank // optimizer_data_parallel_size`` and the
        shard index ``dp_rank % optimizer_data_parallel_size``.
        """
        tp = self.tensor_model_parallel_size
        dp = self.data_parallel_size * self.context_parallel_size
        return global_rank // (tp * dp), (global_rank // tp) % dp, global_rank % tp

    def expert_rank_coords(self, global_rank: int) -> Tuple[int, int, int, int]:
        """(pp_rank, expert_dp_rank, ep_rank, etp_rank) of a global rank."""
        etp = self.expert_tensor_parallel_size
        ep = self.expert_model_parallel_size
        edp = self.expert_data_parallel_size
        return (
            global_rank // (etp * ep * edp),
            (global_rank // (etp * ep)) % edp,
            (global_rank // etp) % ep,
            global_rank % etp,
        )

    def __str__(self):  # parallel_strategy.py:223-224
        return (
            f"self.world_size={self.world_size}, self.tensor_model_parallel_size={self.tensor_model_parallel_size}, "
            f"self.pipeline_model_parallel_size={self.pipeline_model_parallel_size}, "
            f"self.context_parallel_size={self.context_parallel_size}, "
            f"self.num_distributed_optimizer_instances={self.num_distributed_optimizer_instances}, "
            f"self.expert_model_parallel_size={self.expert_model_parallel_size}, "
            f"self.expert_tensor_parallel_size={self.expert_tensor_parallel_size}"
        )

    @staticmethod
    def from_dict(d: Dict[str, int]) -> "ParallelStrategy":
        return ParallelStrategy(**d)

    @staticmethod
    def is_redundant_backup(src: "ParallelStrategy", dst: "ParallelStrategy") -> Optional[bool]:
        """None for a normal reshard, True for a Group-ZeRO scale-up, False for a scale-down.

        parallel_strategy.py:234-263.
        """
        g_src = src.num_distributed_optimizer_instances
        g_dst = dst.num_distributed_optimizer_instances
        if g_src == g_dst:
            if g_src != 1:
                raise ValueError(f"Resharding within a group is not supported, current group size is {g_src}")
            return None
        if src.model_parallel_size != dst.model_parallel_size:
            raise AssertionError("Group-ZeRO switch needs equal model-parallel sizes")
        if src.context_parallel_size != dst.context_parallel_size:
            raise AssertionError("Group-ZeRO switch needs equal CP sizes")
        if src.world_size == dst.world_size:
            raise AssertionError("Group-ZeRO switch needs a world-size change")
        if src.world_size * g_dst != dst.world_size * g_src:
            raise AssertionError("Group-ZeRO switch needs W_src * g_dst == W_dst * g_src")
        return g_src < g_dst


def global_rank_of(
    strategy: ParallelStrategy,
    pipeline_model_parallel_rank: int,
    data_parallel_rank: int,
    expert_model_parallel_rank: Optional[int],
    tensor_model_parallel_rank: int,
) -> int:
    """Global rank with order TP -> EP -> DP -> PP (resharding.py:19-51)."""
    if expert_model_parallel_rank is not None:
        dp_size = strategy.expert_data_parallel_size
        ep_size = strategy.expert_model_parallel_size
        ep_rank = expert_model_parallel_rank
    else:
        dp_size = strategy.optimizer_data_parallel_size
        ep_size = 1
        ep_rank = 0
    tp_size = strategy.get_tensor_model_parallel_size(expert_model_parallel_rank is not None)
    return (
        pipeline_model_parallel_rank * dp_size * ep_size * tp_size
        + data_parallel_rank * ep_size * tp_size
        + ep_rank * tp_size
        + tensor_model_parallel_rank
    )
