"""Oracle-2: destination pieces regenerated from full-tensor indices (test infrastructure).

Independent of any plan: a TP-local element's full-tensor index follows from
Megatron's partitioning (contiguous chunks along the partition dim; a fused
SwiGLU fc1 holds [W_t; V_t], resharding_metadata.py:98-178), and its value
from the seeded generator.

Re-padding the vocabulary (a switch between two padded vocabulary sizes,
which the reference does not have: virtual_param.py:480-481 keeps it fixed)
is pinned by an invariant rather than by the reference: row r of the
embedding and output layer keeps its values while r is below the source's
padded size, and rows past it are zero in every tensor.
"""

import numpy as np

from . import synth
from .plan import dp_distributions, ep_rank, global_rank, local_shape, stage, tp_size


def full_index(p, T, t, local_idx):
    idx = np.asarray(local_idx, dtype=np.int64)
    if not p["tp"] or T == 1:
        return idx
    shape = p["shape"]
    if len(shape) == 1:
        return t * (shape[0] // T) + idx
    R, C = shape
    if p["pdim"] == 0:
        rl = R // T
        r, c = np.divmod(idx, C)
        if p["swiglu"]:
            half, F = rl // 2, R // 2
            fr = np.where(r < half, t * half + r, F + t * half + (r - half))
        else:
            fr = t * rl + r
        return fr * C + c
    cl = C // T
    r, c = np.divmod(idx, cl)
    return r * C + t * cl + c


def value_id(p):
    """Generator stream of a parameter: a tied output layer carries the word embedding (id 0)."""
    return 0 if (p["shared"] and p["where"] == "out") else p["id"]


VOCAB_PARAMS = ("embedding.word_embeddings.weight", "output_layer.weight")


def _values(seed, p, kind, f, vocab_rows):
    v = synth.values(seed, value_id(p), kind, f)
    if vocab_rows is not None and p["name"] in VOCAB_PARAMS:
        v = np.where(f // p["shape"][1] < vocab_rows, v, np.zeros((), dtype=v.dtype))
    return v


def piece_values(seed, p, T, t, lo, hi, vocab_rows=None):
    """{kind: array} for local elements [lo, hi) of TP rank t at TP size T.

    ``vocab_rows``: rows of the vocabulary parameters at and past it are zero
    (the new padding rows of a re-padded destination).
    """
    f = full_index(p, T, t, np.arange(lo, hi))
    return {k: _values(seed, p, k, f, vocab_rows) for k in ("main", "exp_avg", "exp_avg_sq")}


def shard_key(p, strat, hp, t):
    s = stage(p, strat.pp, hp.num_layers)
    if p["expert"] is None:
        return ("dense", s, t)
    return ("expert", s, ep_rank(p, strat, hp.num_experts), t)


def world(inv, hp, strat, seed, params=None, vocab_rows=None):
    """({(rank, pid): {kind: array}}, {(shard key, pid): bf16 bits}) of a layout."""
    dist = dp_distributions(inv, strat, hp)
    fp32, bf16 = {}, {}
    for p in inv:
        if params is not None and p["id"] not in params:
            continue
        if p["id"] not in dist:
            continue
        s = stage(p, strat.pp, hp.num_layers)
        T = tp_size(strat, p)
        e = ep_rank(p, strat, hp.num_experts) if p["expert"] is not None else None
        for t in range(T):
            for r, (lo, hi) in dist[p["id"]].items():
                for inst in range(strat.inst):
                    if e is None:
                        g = s * (strat.dp * strat.cp * strat.tp) + (inst * strat.pdp + r) * strat.tp + t
                    else:
                        g = global_rank(strat, s, r, e, t)
                    fp32[(g, p["id"])] = piece_values(seed, p, T, t, lo, hi, vocab_rows)
            n = int(np.prod(local_shape(p, T)))
            bf16[(shard_key(p, strat, hp, t), p["id"])] = _values(
                seed, p, "param", full_index(p, T, t, np.arange(n)), vocab_rows)
    return fp32, bf16
