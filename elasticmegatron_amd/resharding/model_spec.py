"""Model description that stands in for Megatron's global args and module tree.

The reference learns a model's parameter inventory from the first local
transformer layer of a live Megatron model and from ``get_args()``
(elastic_megatron/resharding/virtual_param.py:472-802,
elastic_megatron/resharding/resharding_metadata.py:322-386).  Here the same
inventory is generated from explicit hyper-parameters, following the mcore GPT
model with the Transformer-Engine layer spec:

  per dense layer   self_attention.linear_proj.weight             [h, nq*d]        TP dim 1
                    self_attention.linear_qkv.layer_norm_weight   [h]
                    self_attention.linear_qkv.weight              [(nq+2g)*d, h]   TP dim 0
                    mlp.linear_fc1.layer_norm_weight              [h]
                    mlp.linear_fc1.weight                         [2F, h] (SwiGLU [W; V])  TP dim 0
                    mlp.linear_fc2.weight                         [h, F]           TP dim 1
  per MoE layer     linear_proj, linear_qkv.layer_norm_weight, linear_qkv (as above)
                    pre_mlp_layernorm.weight                      [h]
                    mlp.router.weight                             [E, h]
                    mlp.experts.linear_fc1.weight{e}              [2F, h] per expert, TP dim 0
                    mlp.experts.linear_fc2.weight{e}              [h, F]  per expert, TP dim 1
  model             embedding.word_embeddings.weight [Vp, h] TP dim 0, the layers,
                    decoder.final_layernorm.weight (+ .bias for LayerNorm),
                    output_layer.weight [Vp, h] TP dim 0 (absent when tied)

QKV rows are grouped by KV group ([g][nq/g q heads, k, v][d]), so contiguous
row chunks keep whole groups on a TP rank; fused SwiGLU fc1 is [W; V] on every
rank (the reference re-interleaves it around the exchange,
resharding_metadata.py:98-178).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Tuple


@dataclass(frozen=True)
class ParamDef:
    name: str                      # module path within a layer, or a model-level name
    shape: Tuple[int, ...]         # full (TP = 1) shape
    tensor_model_parallel: bool
    partition_dim: int             # -1 when not tensor-parallel
    is_swiglu_fc: bool = False
    expert_local: Optional[int] = None  # expert index within the layer (EP = 1)


@dataclass(frozen=True)
class ModelSpec:
    name: str
    num_layers: int
    hidden_size: int
    num_attention_heads: int
    ffn_hidden_size: int
    padded_vocab_size: int
    num_query_groups: Optional[int] = None      # None: multi-head attention
    kv_channels: Optional[int] = None           # None: hidden / heads
    swiglu: bool = True
    normalization: str = "RMSNorm"
    untie_embeddings_and_output_weights: bool = True
    position_embedding_type: str = "rope"
    max_position_embeddings: int = 4096
    num_experts: Optional[int] = None
    moe_ffn_hidden_size: Optional[int] = None
    moe_grouped_gemm: bool = True
    # true vocabulary and Megatron's padding rule (only used to re-pad the vocabulary)
    vocab_size: Optional[int] = None
    make_vocab_size_divisible_by: int = 128
    # distributed-data-parallel / optimizer settings read by the planner
    ddp_bucket_size: Optional[int] = None
    overlap_grad_reduce: bool = False
    overlap_param_gather_with_optimizer_step: bool = False
    use_distributed_optimizer: bool = True

    @property
    def head_dim(self) -> int:
        return self.kv_channels or self.hidden_size // self.num_attention_heads

    @property
    def query_groups(self) -> int:
        return self.num_query_groups or self.num_attention_heads

    @property
    def is_moe(self) -> bool:
        return bool(self.num_experts)

    def layer_params(self) -> List[ParamDef]:
        h, d = self.hidden_size, self.head_dim
        nq, g = self.num_attention_heads, self.query_groups
        out = [
            ParamDef("self_attention.linear_proj.weight", (h, nq * d), True, 1),
            ParamDef("self_attention.linear_qkv.layer_norm_weight", (h,), False, -1),
        ]
        if self.normalization != "RMSNorm":
            out.append(ParamDef("self_attention.linear_qkv.layer_norm_bias", (h,), False, -1))
        out.append(ParamDef("self_attention.linear_qkv.weight", ((nq + 2 * g) * d, h), True, 0))
        if not self.is_moe:
            f = self.ffn_hidden_size
            out.append(ParamDef("mlp.linear_fc1.layer_norm_weight", (h,), False, -1))
            if self.normalization != "RMSNorm":
                out.append(ParamDef("mlp.linear_fc1.layer_norm_bias", (h,), False, -1))
            out.append(ParamDef("mlp.linear_fc1.weight", ((2 if self.swiglu else 1) * f, h), True, 0,
                                is_swiglu_fc=self.swiglu))
            out.append(ParamDef("mlp.linear_fc2.weight", (h, f), True, 1))
            return out
        e_n = self.num_experts
        f = self.moe_ffn_hidden_size or self.ffn_hidden_size
        out.append(ParamDef("pre_mlp_layernorm.weight", (h,), False, -1))
        if self.normalization != "RMSNorm":
            out.append(ParamDef("pre_mlp_layernorm.bias", (h,), False, -1))
        out.append(ParamDef("mlp.router.weight", (e_n, h), False, -1))
        fc1 = [ParamDef(f"mlp.experts.linear_fc1.weight{e}", ((2 if self.swiglu else 1) * f, h), True, 0,
                        is_swiglu_fc=self.swiglu, expert_local=e) for e in range(e_n)]
        fc2 = [ParamDef(f"mlp.experts.linear_fc2.weight{e}", (h, f), True, 1, expert_local=e) for e in range(e_n)]
        if self.moe_grouped_gemm:  # grouped_gemm_order (virtual_param.py:611-686)
            out += fc1 + fc2
        else:  # expert_id_order
            for a, b in zip(fc1, fc2):
                out += [a, b]
        return out

    def embedding_params(self) -> List[ParamDef]:
        out = [ParamDef("embedding.word_embeddings.weight", (self.padded_vocab_size, self.hidden_size), True, 0)]
        if self.position_embedding_type == "learned_absolute":
            out.append(ParamDef("embedding.position_embeddings.weight",
                                (self.max_position_embeddings, self.hidden_size), False, -1))
        return out

    def output_params(self) -> List[ParamDef]:
        out = [ParamDef("decoder.final_layernorm.weight", (self.hidden_size,), False, -1)]
        if self.normalization != "RMSNorm":
            out.append(ParamDef("decoder.final_layernorm.bias", (self.hidden_size,), False, -1))
        out.append(ParamDef("output_layer.weight", (self.padded_vocab_size, self.hidden_size), True, 0))
        return out

    def padded_vocab_for_tp(self, tp: int) -> int:
        """Megatron's padded vocabulary at TP size ``tp`` (multiple of divisible_by * tp)."""
        if self.vocab_size is None:
            raise ValueError("vocab_size is not set")
        return _pad_vocab(self.vocab_size, self.make_vocab_size_divisible_by * tp)

    def with_padded_vocab(self, padded_vocab_size: int) -> "ModelSpec":
        from dataclasses import replace

        if self.vocab_size is not None and padded_vocab_size < self.vocab_size:
            raise ValueError("padded vocabulary smaller than the vocabulary")
        return replace(self, padded_vocab_size=padded_vocab_size)

    def num_params(self) -> int:
        tot = 0
        for p in self.embedding_params() + self.output_params():
            if p.name == "output_layer.weight" and not self.untie_embeddings_and_output_weights:
                continue
            tot += _numel(p.shape)
        tot += self.num_layers * sum(_numel(p.shape) for p in self.layer_params())
        return tot


def _numel(shape) -> int:
    n = 1
    for s in shape:
        n *= s
    return n


def _pad_vocab(v: int, multiple: int) -> int:
    return -(-v // multiple) * multiple


# Model shapes of the reshard workloads.  bucket sizes follow Megatron's
# default max(4e7, 1e6 * dp) when overlap_grad_reduce is on.
def tiny_llama2() -> ModelSpec:
    """2 layers, hidden 512, 8 heads, SwiGLU FFN 1376, vocab 32000 (single bucket)."""
    return ModelSpec(name="tiny-llama2", num_layers=2, hidden_size=512, num_attention_heads=8,
                     ffn_hidden_size=1376, padded_vocab_size=32000, overlap_grad_reduce=False)


def llama2_7b() -> ModelSpec:
    return ModelSpec(name="llama2-7b", num_layers=32, hidden_size=4096, num_attention_heads=32,
                     ffn_hidden_size=11008, padded_vocab_size=32000, ddp_bucket_size=40_000_000,
                     overlap_grad_reduce=True)


def llama2_13b() -> ModelSpec:
    """40 layers, hidden 5120, 40 heads, SwiGLU FFN 13824, vocab 32000: 13.0e9 parameters, whose
    state (182 GB) does not fit twice in one GPU's HBM."""
    return ModelSpec(name="llama2-13b", num_layers=40, hidden_size=5120, num_attention_heads=40,
                     ffn_hidden_size=13824, padded_vocab_size=32000, ddp_bucket_size=40_000_000,
                     overlap_grad_reduce=True)


def llama2_70b() -> ModelSpec:
    """80 layers, hidden 8192, 64 heads with 8 KV groups, SwiGLU FFN 28672, vocab 32000: 69.0e9
    parameters, 966 GB of state, which no single GPU holds; one destination rank's share of a
    switch fits."""
    return ModelSpec(name="llama2-70b", num_layers=80, hidden_size=8192, num_attention_heads=64,
                     num_query_groups=8, ffn_hidden_size=28672, padded_vocab_size=32000,
                     ddp_bucket_size=40_000_000, overlap_grad_reduce=True)


def llama3_8b() -> ModelSpec:
    return ModelSpec(name="llama3-8b", num_layers=32, hidden_size=4096, num_attention_heads=32,
                     num_query_groups=8, ffn_hidden_size=14336, vocab_size=128256,
                     padded_vocab_size=_pad_vocab(128256, 128 * 2), overlap_grad_reduce=True)


def mixtral_8x7b_slice(num_layers: int = 4) -> ModelSpec:
    return ModelSpec(name=f"mixtral-8x7b-{num_layers}l", num_layers=num_layers, hidden_size=4096,
                     num_attention_heads=32, num_query_groups=8, ffn_hidden_size=14336,
                     padded_vocab_size=32000, num_experts=8, moe_ffn_hidden_size=14336,
                     overlap_grad_reduce=True)
