"""Re-padding the vocabulary across a TP switch (an extension: the reference keeps it fixed).

The reference keeps ``padded_vocab_size`` constant across switches
(elastic_megatron/resharding/virtual_param.py:480-481).  With re-padding the
destination uses Megatron's padded size for its own TP size; the plan copies
the rows both sizes hold and writes zeros into new padding rows in all four
tensors.  There is no reference output to match, so the plan is checked
against an invariant stated independently of it: row r of the embedding and
output layer carries the generator's values for (r, c) while r is below the
source's padded size, and is zero past it (the canonical oracle with
``vocab_rows``).  Everything else must equal the fixed-padding result.
"""

from dataclasses import replace

import numpy as np
import pytest

from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy as PS
from elasticmegatron_amd.resharding import model_spec as ms
from elasticmegatron_amd.resharding.layout import SEG_CAST_BF16, SEG_ZERO_FILL, VOCAB_PARAM_NAMES, split_vocab_rows
from elasticmegatron_amd.resharding.lowering import lower_transfer, payload_bytes, read_bytes
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from oracle import canonical, model
from tests.helpers import (REPAD_CASES, SEED, compare, execute_numpy, extract, new_arenas, piece_fill_numpy,
                           repad_spaces, small_llama3, strat)


def test_padding_rule():
    """Smallest multiple of divisible_by * TP not below the vocabulary (Megatron's rule)."""
    spec = ms.llama3_8b()
    assert spec.padded_vocab_size == 128256
    assert [spec.padded_vocab_for_tp(t) for t in (1, 2, 4, 8)] == [128256, 128256, 128512, 129024]
    for v in (1, 127, 128, 129, 32000, 50257):
        s = replace(ms.tiny_llama2(), vocab_size=v)
        for t in (1, 2, 3, 4, 8):
            m = 128 * t
            p = s.padded_vocab_for_tp(t)
            assert p % m == 0 and v <= p < v + m
    with pytest.raises(ValueError):
        ms.tiny_llama2().padded_vocab_for_tp(2)
    with pytest.raises(ValueError):
        replace(ms.tiny_llama2(), vocab_size=32000).with_padded_vocab(31999)


@pytest.mark.parametrize("factory,vocab,src,dst", REPAD_CASES)
@pytest.mark.parametrize("bf16_source", ["cast", "copy"])
def test_repad_matches_invariant(factory, vocab, src, dst, bf16_source):
    spec = replace(factory(), vocab_size=vocab)
    sa, sb = repad_spaces(spec, (src.tensor_model_parallel_size, dst.tensor_model_parallel_size))
    ls, ld = sa.layout(src), sb.layout(dst)
    table = lower_transfer(ls, ld, bf16_source=bf16_source)
    a, b = new_arenas(ls), new_arenas(ld)
    piece_fill_numpy(ls.pieces(), a, SEED)
    execute_numpy(table, a, b)
    got32, gotbf = extract(ld, b)
    want32, wantbf = canonical.world(model.inventory(sb.spec), sb.spec, strat(dst), SEED,
                                     vocab_rows=sa.spec.padded_vocab_size)
    assert compare(got32, gotbf, want32, wantbf) == []

    zero = (table["flags"] & SEG_ZERO_FILL) != 0
    grow = sb.spec.padded_vocab_size - sa.spec.padded_vocab_size
    assert zero.any() == (grow > 0)
    if grow > 0:
        # New rows are written once per kind and never read.
        h = sb.spec.hidden_size
        n_vocab = sum(1 for vp in sb.all_virtual_params if vp.name in VOCAB_PARAM_NAMES and ld.has_param(vp))
        units = table["len"].astype(np.int64) * table["rows"].astype(np.int64)
        fp32_zero = units[zero & (table["elem_bytes"] == 4)].sum()
        assert fp32_zero == 3 * n_vocab * grow * h
        assert read_bytes(table) == read_bytes(table[~zero])
        if bf16_source == "cast":
            assert (table["flags"][zero & (table["src_buf"] == 0)] & SEG_CAST_BF16).all()
    # Every element read is written once (dropped padding rows are not read).
    assert read_bytes(table) <= payload_bytes(table)


def test_repad_round_trip_is_identity():
    """Grow then shrink the padding: every element of the source comes back."""
    spec = replace(small_llama3(), vocab_size=2300)
    src, mid = PS(8, 2, 2), PS(8, 4, 1)
    sa, sb = repad_spaces(spec, (2, 4))
    la, lb = sa.layout(src), sb.layout(mid)
    a = new_arenas(la)
    piece_fill_numpy(la.pieces(), a, SEED)
    b = new_arenas(lb)
    execute_numpy(lower_transfer(la, lb), a, b)
    c = new_arenas(la)
    execute_numpy(lower_transfer(lb, la), b, c)
    want = new_arenas(la)
    piece_fill_numpy(la.pieces(), want, SEED)
    assert compare(*extract(la, c), *extract(la, want)) == []


def test_split_vocab_rows_partitions_pieces():
    spec = replace(small_llama3(), vocab_size=2300)
    _, sb = repad_spaces(spec, (2, 4))
    lay = sb.layout(PS(8, 4, 1))
    pcs = lay.pieces()
    keep, zero = split_vocab_rows(lay, pcs, 2304)
    assert int(keep["len"].sum()) + sum(n for _, _, n in zero) == int(pcs["len"].sum())
    # 256 new rows of 256 columns in 2 vocabulary params, each held once per fp32 kind (the DP
    # shards partition it) and once in the bf16 arena (DP replicas share one buffer).
    assert sum(n for _, _, n in zero) == 256 * 256 * 2 * (3 + 1)


def test_incompatible_models_rejected():
    a = build_virtual_model(small_llama3())
    b = build_virtual_model(replace(small_llama3(), hidden_size=512))
    with pytest.raises(ValueError):
        lower_transfer(a.layout(PS(8, 2, 1)), b.layout(PS(8, 2, 1)))


def test_manager_repad_plans():
    """ElasticMegatronManager(repad_vocab=True) lays each strategy out at its own padded size."""
    from elasticmegatron_amd import ElasticMegatronManager

    spec = replace(small_llama3(), vocab_size=2300)
    seq = [dict(world_size=8, tensor_model_parallel_size=2, pipeline_model_parallel_size=2),
           dict(world_size=8, tensor_model_parallel_size=4, pipeline_model_parallel_size=1)]
    mgr = ElasticMegatronManager(seq, spec, device="meta", repad_vocab=True)
    assert mgr.virtual_param_space.spec.padded_vocab_size == 2304
    assert mgr.space_for(PS(8, 4, 1)).spec.padded_vocab_size == 2560
    assert mgr.reshard(new_parallel_strategy=seq[1], is_meta_device=True) is None
    with pytest.raises(ValueError):
        ElasticMegatronManager(seq, small_llama3(), device="meta", repad_vocab=True)
