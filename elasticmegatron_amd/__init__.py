"""MI355X-native reshard repack of ElasticMegatron.

Public API (names follow elastic_megatron):
  ElasticMegatronManager   reshard(new_parallel_strategy=...)      elastic_manager.py
  ParallelStrategy         TP/PP/CP/DP/EP sizes, rank arithmetic   megatron_manager/parallel_strategy.py
  TrainingState            device-resident state of every rank     megatron_manager/training_state.py
  TransferManager          native copy-plan executor               transfer/transfer.py
  build_virtual_model      planner over a ModelSpec                resharding/virtual_param.py
"""

from .elastic_manager import ElasticMegatronManager
from .megatron_manager.parallel_strategy import ParallelStrategy
from .megatron_manager.training_state import OptimizerTensorInfo, TrainingState
from .resharding.model_spec import ModelSpec, llama2_7b, llama3_8b, mixtral_8x7b_slice, tiny_llama2
from .resharding.virtual_param import VirtualParamSpace, build_virtual_model
from .transfer.transfer import TransferManager

__all__ = [
    "ElasticMegatronManager", "ParallelStrategy", "TrainingState", "OptimizerTensorInfo", "TransferManager",
    "ModelSpec", "VirtualParamSpace", "build_virtual_model", "tiny_llama2", "llama2_7b", "llama3_8b",
    "mixtral_8x7b_slice",
]
