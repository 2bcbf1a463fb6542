"""Global virtual parameter space (every parallel size = 1).

Mirrors ``VirtualParam``, ``VirtualParamSpace`` and ``build_virtual_model`` of
the reference (elastic_megatron/resharding/virtual_param.py:48-802).  The
reference derives the per-layer parameter list from the first local layer of a
live Megatron model; here it comes from a :class:`~.model_spec.ModelSpec`
(same names, order and TP attributes).  Per-strategy results are cached like
the reference's ``_dp_distribution_cache`` / ``_reshard_plan_cache``
(virtual_param.py:88-94, :151-188).
"""

from __future__ import annotations

from typing import Dict, List, Optional, Tuple

from ..megatron_manager.parallel_strategy import ParallelStrategy
from .model_spec import ModelSpec, ParamDef
from .resharding import ReshardPlan
from .resharding_dp import (DataParallelReshardingInfo, ExpertParallelReshardingInfo,
                            get_params_dp_distribution)
from .resharding_pp import LayerType, ParamPositionAttr
from .resharding_tp import TensorParallelAttr
from .util import Range


class VirtualParam:
    """A parameter of the model with every parallel size equal to 1."""

    def __init__(self, position: ParamPositionAttr, pdef: ParamDef):
        self.param_position_attr = position
        self.param_def = pdef
        self.tensor_parallel_attr = TensorParallelAttr(pdef.shape, pdef.tensor_model_parallel, pdef.partition_dim)
        self.shared_embedding = position.shared_embedding
        # virtual_param.py:83-86: SwiGLU handling only applies to a TP-split fc1.
        self.is_swiglu_fc = position.is_swiglu_fc and self.tensor_parallel_attr.tensor_model_parallel
        self._dp_cache: Dict[ParallelStrategy, Dict[int, Range]] = {}
        self._plan_cache: Dict[Tuple[ParallelStrategy, ParallelStrategy], ReshardPlan] = {}
        self.current_reshard_plan: Optional[ReshardPlan] = None

    @property
    def global_index(self) -> int:
        return self.param_position_attr.global_index

    @property
    def is_expert(self) -> bool:
        return self.param_position_attr.expert_id is not None

    @property
    def expert_id(self) -> Optional[int]:
        return self.param_position_attr.expert_id

    @property
    def full_shape(self) -> Tuple[int, ...]:
        return self.tensor_parallel_attr.full_shape

    def numel(self) -> int:
        n = 1
        for s in self.full_shape:
            n *= s
        return n

    def tp_size_at(self, strategy: ParallelStrategy) -> int:
        return strategy.get_tensor_model_parallel_size(self.is_expert)

    def local_shape(self, strategy: ParallelStrategy) -> Tuple[int, ...]:
        return self.tensor_parallel_attr.local_shape(self.tp_size_at(strategy))

    def numel_at(self, strategy: ParallelStrategy) -> int:
        n = 1
        for s in self.local_shape(strategy):
            n *= s
        return n

    def get_model_param_stage_id(self, pp_size: int) -> int:
        return self.param_position_attr.get_model_param_stage_id(pp_size)

    @property
    def name(self) -> str:
        pos = self.param_position_attr
        if pos.layer_type == LayerType.TRANSFORMER_LAYER:
            return f"decoder.layers.{pos.transformer_layer_id}.{self.param_def.name}"
        return self.param_def.name

    def get_dp_distribution(self, strategy: ParallelStrategy) -> Dict[int, Range]:
        d = self._dp_cache.get(strategy)
        assert d is not None, f"DP distribution of {self.name} at {strategy} not built"
        return d

    def set_dp_distribution(self, strategy: ParallelStrategy, dist: Dict[int, Range]) -> None:
        self._dp_cache[strategy] = dist

    def apply_reshard_plan(self, src: ParallelStrategy, dst: ParallelStrategy, num_experts: Optional[int]) -> ReshardPlan:
        key = (src, dst)
        plan = self._plan_cache.get(key)
        if plan is None:
            plan = self._generate_reshard_plan(src, dst, num_experts)
            self._plan_cache[key] = plan
        self.current_reshard_plan = plan
        return plan

    @property
    def reshard_plan(self) -> Optional[ReshardPlan]:
        return self.current_reshard_plan

    def _generate_reshard_plan(self, src: ParallelStrategy, dst: ParallelStrategy,
                               num_experts: Optional[int]) -> ReshardPlan:
        """virtual_param.py:194-259."""
        tp_info = self.tensor_parallel_attr.reshard(self.tp_size_at(src), self.tp_size_at(dst))
        pp_info = self.param_position_attr.reshard(src.pipeline_model_parallel_size,
                                                   dst.pipeline_model_parallel_size)
        ep_info = (ExpertParallelReshardingInfo(self.expert_id, src, dst, num_experts)
                   if self.is_expert else None)
        dp_info = None
        if pp_info.src_pp_rank != -1 and pp_info.dst_pp_rank != -1:
            dp_info = DataParallelReshardingInfo(self.get_dp_distribution(src), self.get_dp_distribution(dst),
                                                 src, dst, pp_info, ep_info)
        return ReshardPlan(tp_info, pp_info, dp_info, ep_info, src, dst)

    def __repr__(self):
        return f"VirtualParam({self.global_index}: {self.name} {self.full_shape})"


class VirtualParamSpace:
    def __init__(self, spec: ModelSpec, embedding_layer_virtual_params: List[VirtualParam],
                 transformer_layers_virtual_params: List[List[VirtualParam]],
                 output_layer_virtual_params: List[VirtualParam]):
        self.spec = spec
        self.embedding_layer_virtual_params = embedding_layer_virtual_params
        self.transformer_layers_virtual_params = transformer_layers_virtual_params
        self.output_layer_virtual_params = output_layer_virtual_params
        self.all_virtual_params: List[VirtualParam] = list(embedding_layer_virtual_params)
        for layer in transformer_layers_virtual_params:
            self.all_virtual_params += layer
        self.all_virtual_params += output_layer_virtual_params
        assert all(p.global_index == i for i, p in enumerate(self.all_virtual_params)), \
            "Global index of virtual params is not correct"
        self._stages: Dict[int, List[List[VirtualParam]]] = {}
        self._built: set = set()
        self._layouts: Dict[ParallelStrategy, "object"] = {}
        # The training states of a transfer in progress, read by
        # TransferManager.transfer_optimizer_tensors(space); None between transfers.
        self.src_state = None
        self.dst_state = None

    @property
    def tied_embeddings(self) -> bool:
        return not self.spec.untie_embeddings_and_output_weights

    def value_source(self, vp: VirtualParam) -> VirtualParam:
        """The parameter whose values ``vp`` carries.

        A tied output layer carries the word embedding: the reference skips it
        in the transfer and then broadcasts the new word-embedding state to it
        over the embedding group (transfer.py:103-141, :324-330).
        """
        if self.tied_embeddings and vp.param_position_attr.layer_type == LayerType.OUTPUT_LAYER:
            return self.embedding_layer_virtual_params[0]
        return vp

    def stages(self, pp_size: int) -> List[List[VirtualParam]]:
        """virtual_param.py:295-316."""
        st = self._stages.get(pp_size)
        if st is None:
            st = [[] for _ in range(pp_size)]
            for p in self.all_virtual_params:
                sid = p.get_model_param_stage_id(pp_size)
                if sid != -1:
                    st[sid].append(p)
            self._stages[pp_size] = st
        return st

    def build_model_virtual_params(self, strategy: ParallelStrategy) -> None:
        """DP distributions of every parameter at ``strategy`` (virtual_param.py:324-375)."""
        if strategy in self._built:
            return
        spec = self.spec
        if not spec.use_distributed_optimizer:
            raise AssertionError("non-zero DP is not supported yet")
        strategy.validate_for(spec.num_layers, spec.num_experts)
        for idx, stage in enumerate(self.stages(strategy.pipeline_model_parallel_size)):
            disable = idx > 0 or spec.overlap_param_gather_with_optimizer_step
            dist = get_params_dp_distribution(stage, strategy, spec, disable)
            for p in stage:
                p.set_dp_distribution(strategy, dist[p])
        self._built.add(strategy)

    def register_reshard(self, src: ParallelStrategy, dst: ParallelStrategy) -> None:
        """Build both strategies and every parameter's ReshardPlan (virtual_param.py:377-410)."""
        self.build_model_virtual_params(src)
        self.build_model_virtual_params(dst)
        for p in self.all_virtual_params:
            p.apply_reshard_plan(src, dst, self.spec.num_experts)

    def layout(self, strategy: ParallelStrategy):
        """Device-memory layout of every rank's state at ``strategy`` (cached)."""
        from .layout import StrategyLayout

        lay = self._layouts.get(strategy)
        if lay is None:
            lay = StrategyLayout(self, strategy)
            self._layouts[strategy] = lay
        return lay


def build_virtual_model(spec: ModelSpec) -> VirtualParamSpace:
    """virtual_param.py:769-802 with the inventory taken from ``spec``."""
    L = spec.num_layers
    shared = not spec.untie_embeddings_and_output_weights
    gi = 0
    emb: List[VirtualParam] = []
    for k, pd in enumerate(spec.embedding_params()):
        lt = LayerType.WORD_EMBEDDING if k == 0 else LayerType.POSITION_EMBEDDING
        emb.append(VirtualParam(ParamPositionAttr(lt, L, pd.name, global_index=gi, layer_index=k,
                                                  shared_embedding=shared and k == 0), pd))
        gi += 1
    layers: List[List[VirtualParam]] = []
    defs = spec.layer_params()
    for lid in range(L):
        layer: List[VirtualParam] = []
        dense_idx = 0
        for pd in defs:
            is_expert = pd.expert_local is not None
            pos = ParamPositionAttr(
                LayerType.TRANSFORMER_LAYER, L, pd.name, global_index=gi, transformer_layer_id=lid,
                layer_index=-1 if is_expert else dense_idx,
                is_swiglu_fc=pd.is_swiglu_fc,
                expert_id=pd.expert_local if is_expert else None,
                expert_param_layer_id=(0 if "linear_fc1" in pd.name else 1) if is_expert else -1)
            if not is_expert:
                dense_idx += 1
            layer.append(VirtualParam(pos, pd))
            gi += 1
        layers.append(layer)
    out: List[VirtualParam] = []
    for k, pd in enumerate(spec.output_params()):
        lt = LayerType.OUTPUT_LAYER if pd.name == "output_layer.weight" else LayerType.FINAL_LAYERNORM
        out.append(VirtualParam(ParamPositionAttr(lt, L, pd.name, global_index=gi, layer_index=k,
                                                  shared_embedding=shared and lt == LayerType.OUTPUT_LAYER), pd))
        gi += 1
    return VirtualParamSpace(spec, emb, layers, out)
