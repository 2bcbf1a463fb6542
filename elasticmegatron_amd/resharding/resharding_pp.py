"""Pipeline-stage placement of a parameter.

Mirrors ``LayerType``, ``ParamPositionAttr`` and
``PipelineParallelReshardingInfo`` of the reference
(elastic_megatron/resharding/resharding_pp.py:1-173):
embeddings live on stage 0, the final norm and output layer on the last
stage (the output layer on no stage when it shares the embedding and PP is
1), and transformer layer l on stage ``l // (num_layers / pp)``.
The reference reads ``num_layers`` from Megatron's global args; here it is a
field of the attribute.
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum
from typing import Dict, Optional, Tuple


@dataclass
class PipelineParallelReshardingInfo:
    src_pp_rank: int
    dst_pp_rank: int


class LayerType(Enum):
    WORD_EMBEDDING = "word_embedding"
    POSITION_EMBEDDING = "position_embedding"
    TRANSFORMER_LAYER = "transformer_layer"
    FINAL_LAYERNORM = "final_layernorm"
    OUTPUT_LAYER = "output_layer"


class ParamPositionAttr:
    def __init__(self, layer_type: LayerType, num_layers: int, module_name: str = "",
                 global_index: int = -1, transformer_layer_id: int = -1, layer_index: int = -1,
                 is_swiglu_fc: bool = False, shared_embedding: bool = False,
                 expert_id: Optional[int] = None, expert_param_layer_id: int = -1):
        self.layer_type = layer_type
        self.num_layers = num_layers
        self.module_name = module_name
        self.global_index = global_index
        self.transformer_layer_id = transformer_layer_id
        self.layer_index = layer_index
        self.is_swiglu_fc = is_swiglu_fc
        self.shared_embedding = shared_embedding
        self.expert_id = expert_id
        self.expert_param_layer_id = expert_param_layer_id
        self._stage_cache: Dict[int, int] = {}
        self._cache: Dict[Tuple[int, int], PipelineParallelReshardingInfo] = {}

    @property
    def is_expert(self) -> bool:
        return self.expert_id is not None

    def get_model_param_stage_id(self, pp_size: int) -> int:
        assert pp_size >= 1
        sid = self._stage_cache.get(pp_size)
        if sid is not None:
            return sid
        if self.layer_type in (LayerType.WORD_EMBEDDING, LayerType.POSITION_EMBEDDING):
            sid = 0
        elif self.layer_type == LayerType.FINAL_LAYERNORM:
            sid = pp_size - 1
        elif self.layer_type == LayerType.OUTPUT_LAYER:
            sid = -1 if (self.shared_embedding and pp_size == 1) else pp_size - 1
        else:
            assert self.transformer_layer_id != -1
            assert self.num_layers % pp_size == 0
            sid = self.transformer_layer_id // (self.num_layers // pp_size)
        self._stage_cache[pp_size] = sid
        return sid

    def reshard(self, src_pp: int, dst_pp: int) -> PipelineParallelReshardingInfo:
        key = (src_pp, dst_pp)
        info = self._cache.get(key)
        if info is None:
            info = PipelineParallelReshardingInfo(self.get_model_param_stage_id(src_pp),
                                                  self.get_model_param_stage_id(dst_pp))
            self._cache[key] = info
        return info

    def __str__(self):
        where = (f"layer {self.transformer_layer_id}" if self.transformer_layer_id != -1
                 else self.layer_type.value)
        slot = (f"expert {self.expert_id} param {self.expert_param_layer_id}" if self.is_expert
                else f"param {self.layer_index}")
        return f"#{self.global_index} {where} {slot} {self.module_name}".rstrip()

    __repr__ = __str__
