"""Parameter inventory of a model, from its hyper-parameters (test infrastructure).

Follows the mcore GPT + Transformer-Engine parameter order the reference's
virtual model reproduces (elastic_megatron/resharding/virtual_param.py:472-802;
names per resharding_metadata.py:335-386).  ``hp`` is any object with the
hyper-parameter attributes (num_layers, hidden_size, num_attention_heads,
num_query_groups, kv_channels, ffn_hidden_size, padded_vocab_size, swiglu,
normalization, untie_embeddings_and_output_weights, position_embedding_type,
max_position_embeddings, num_experts, moe_ffn_hidden_size, moe_grouped_gemm).
"""


def _p(name, shape, tp, pdim, where, layer=-1, swiglu=False, expert=None):
    return dict(name=name, shape=tuple(shape), tp=tp, pdim=pdim if tp else -1, where=where,
                layer=layer, swiglu=swiglu and tp, expert=expert)


def inventory(hp):
    h = hp.hidden_size
    nq = hp.num_attention_heads
    g = hp.num_query_groups or nq
    d = hp.kv_channels or h // nq
    ln = hp.normalization != "RMSNorm"
    out = [_p("embedding.word_embeddings.weight", (hp.padded_vocab_size, h), True, 0, "emb")]
    if hp.position_embedding_type == "learned_absolute":
        out.append(_p("embedding.position_embeddings.weight", (hp.max_position_embeddings, h), False, -1, "emb"))
    for l in range(hp.num_layers):
        pre = f"decoder.layers.{l}."
        out.append(_p(pre + "self_attention.linear_proj.weight", (h, nq * d), True, 1, "layer", l))
        out.append(_p(pre + "self_attention.linear_qkv.layer_norm_weight", (h,), False, -1, "layer", l))
        if ln:
            out.append(_p(pre + "self_attention.linear_qkv.layer_norm_bias", (h,), False, -1, "layer", l))
        out.append(_p(pre + "self_attention.linear_qkv.weight", ((nq + 2 * g) * d, h), True, 0, "layer", l))
        mult = 2 if hp.swiglu else 1
        if not hp.num_experts:
            f = hp.ffn_hidden_size
            out.append(_p(pre + "mlp.linear_fc1.layer_norm_weight", (h,), False, -1, "layer", l))
            if ln:
                out.append(_p(pre + "mlp.linear_fc1.layer_norm_bias", (h,), False, -1, "layer", l))
            out.append(_p(pre + "mlp.linear_fc1.weight", (mult * f, h), True, 0, "layer", l, swiglu=hp.swiglu))
            out.append(_p(pre + "mlp.linear_fc2.weight", (h, f), True, 1, "layer", l))
            continue
        E = hp.num_experts
        f = hp.moe_ffn_hidden_size or hp.ffn_hidden_size
        out.append(_p(pre + "pre_mlp_layernorm.weight", (h,), False, -1, "layer", l))
        if ln:
            out.append(_p(pre + "pre_mlp_layernorm.bias", (h,), False, -1, "layer", l))
        out.append(_p(pre + "mlp.router.weight", (E, h), False, -1, "layer", l))
        fc1 = [_p(pre + f"mlp.experts.linear_fc1.weight{e}", (mult * f, h), True, 0, "layer", l,
                  swiglu=hp.swiglu, expert=e) for e in range(E)]
        fc2 = [_p(pre + f"mlp.experts.linear_fc2.weight{e}", (h, f), True, 1, "layer", l, expert=e)
               for e in range(E)]
        if hp.moe_grouped_gemm:
            out += fc1 + fc2
        else:
            for a, b in zip(fc1, fc2):
                out += [a, b]
    out.append(_p("decoder.final_layernorm.weight", (h,), False, -1, "final"))
    if ln:
        out.append(_p("decoder.final_layernorm.bias", (h,), False, -1, "final"))
    out.append(_p("output_layer.weight", (hp.padded_vocab_size, h), True, 0, "out"))
    for i, p in enumerate(out):
        p["id"] = i
        p["shared"] = (not hp.untie_embeddings_and_output_weights) and p["where"] in ("emb", "out") and \
            p["name"] != "embedding.position_embeddings.weight"
    return out


def numel(shape):
    n = 1
    for s in shape:
        n *= s
    return n
