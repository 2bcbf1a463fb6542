"""Shared test utilities: small model shapes, numpy executors and comparisons."""

import numpy as np

from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy as PS
from elasticmegatron_amd.resharding import model_spec as ms
from elasticmegatron_amd.resharding.layout import ARENA_PARAM
from oracle import synth
from oracle.plan import Strat

SEED = 1234


# Small models with the structure of each reshard workload (GQA, MoE, buckets, PP).
def small_llama2():
    return ms.ModelSpec(name="small-llama2", num_layers=4, hidden_size=256, num_attention_heads=4,
                        ffn_hidden_size=688, padded_vocab_size=1024, ddp_bucket_size=150_000,
                        overlap_grad_reduce=True)


def small_llama3():
    return ms.ModelSpec(name="small-llama3", num_layers=4, hidden_size=256, num_attention_heads=8,
                        num_query_groups=2, kv_channels=32, ffn_hidden_size=896, padded_vocab_size=2048,
                        ddp_bucket_size=200_000, overlap_grad_reduce=True)


def small_mixtral():
    return ms.ModelSpec(name="small-mixtral", num_layers=2, hidden_size=256, num_attention_heads=8,
                        num_query_groups=2, kv_channels=32, ffn_hidden_size=512, padded_vocab_size=1024,
                        num_experts=8, moe_ffn_hidden_size=512, ddp_bucket_size=300_000,
                        overlap_grad_reduce=True)


# (name, spec factory, [strategies]) -- consecutive strategies are switched.
SMALL_CASES = [
    ("tiny_tp2dp4_tp1dp8_tp4dp2", ms.tiny_llama2, [PS(8, 2, 1), PS(8, 1, 1), PS(8, 4, 1)]),
    ("llama2_tp1dp8_tp4dp2", small_llama2, [PS(8, 1, 1), PS(8, 4, 1)]),
    ("llama3_tp2pp2dp2_tp4pp1dp2", small_llama3, [PS(8, 2, 2), PS(8, 4, 1)]),
    ("mixtral_ep4_ep8", small_mixtral, [PS(8, 1, 1, expert_model_parallel_size=4),
                                        PS(8, 1, 1, expert_model_parallel_size=8)]),
    ("llama2_dp8_dp6", small_llama2, [PS(8, 1, 1), PS(6, 1, 1)]),
    ("llama2_pp4_tp2", small_llama2, [PS(8, 1, 4), PS(8, 2, 1), PS(8, 2, 2)]),
    ("llama3_tp4_tp1pp2", small_llama3, [PS(8, 4, 1), PS(8, 1, 2)]),
    # Context parallelism: the distributed optimizer shards over DP x CP ranks.
    ("llama2_cp2tp2_cp2tp1_cp1tp2", small_llama2, [PS(8, 2, 1, context_parallel_size=2),
                                                   PS(8, 1, 1, context_parallel_size=2), PS(8, 2, 1)]),
]


def piece_fill_numpy(pieces, arenas, seed):
    """Restatement of emrs_synth_fill on numpy arenas (uint32 fp32 bits / uint16 bf16 bits)."""
    for p in pieces:
        n = int(p["len"])
        if n == 0:
            continue
        li = int(p["local_start"]) + np.arange(n, dtype=np.int64)
        r, c = np.divmod(li, int(p["local_cols"]))
        br = int(p["band_rows"])
        if br:
            row = np.where(r < br, r + int(p["row_off"]), r - br + int(p["row_off2"]))
        else:
            row = r + int(p["row_off"])
        f = row * int(p["full_cols"]) + c + int(p["col_off"])
        kind = int(p["kind"])
        name = ("param", "main", "exp_avg", "exp_avg_sq")[kind]
        v = synth.values(seed, int(p["param_id"]), name, f)
        off = int(p["buf_off"])
        arenas[int(p["buf"])][off:off + n] = v.view(np.uint16) if kind == 0 else v.view(np.uint32)


def new_arenas(layout, fill=0xFFFFFFFF):
    f32 = [np.full(layout.fp32_numel, fill, dtype=np.uint32) for _ in range(3)]
    return f32 + [np.full(layout.bf16_numel, fill & 0xFFFF, dtype=np.uint16)]


def bf16_rne_bits(u32):
    """fp32 bits -> bf16 bits, nearest-even; NaN -> 0x7FC0 (torch's float -> bfloat16 rounding)."""
    u = u32.astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)).astype(np.uint16)
    return np.where((u32 & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000), np.uint16(0x7FC0), r)


def _view(arr, off, rows, n, stride):
    if rows == 1:
        return arr[off:off + n]
    return np.lib.stride_tricks.as_strided(arr[off:], shape=(rows, n), strides=(stride * arr.itemsize, arr.itemsize))


def execute_numpy(table, src, dst):
    """Reference semantics of emrs_plan_execute on numpy arenas (fp32 arenas as uint32 bits)."""
    for s in table:
        a, b = src[int(s["src_buf"])], dst[int(s["dst_buf"])]
        so, do, n, rows = int(s["src_off"]), int(s["dst_off"]), int(s["len"]), int(s["rows"])
        if int(s["flags"]) & 2:  # zero fill
            vals = np.zeros((rows, n) if rows > 1 else n, dtype=b.dtype)
        else:
            vals = _view(a, so, rows, n, int(s["src_stride"])).copy()
        _view(b, do, rows, n, int(s["dst_stride"]))[...] = vals
        if int(s["flags"]) & 1:
            aux = dst[int(s["aux_buf"])]
            _view(aux, int(s["aux_off"]), rows, n, int(s["aux_stride"]))[...] = bf16_rne_bits(vals)
        if int(s["flags"]) & 4:  # duplicate
            _view(dst[int(s["aux_buf"])], int(s["aux_off"]), rows, n, int(s["aux_stride"]))[...] = vals


def extract(layout, arenas, params=None):
    """({(rank, pid): {kind: uint32 bits}}, {(shard key, pid): uint16 bits}) from product arenas."""
    space = layout.space
    fp32, bf16 = {}, {}
    vps = [space.all_virtual_params[g] for g in sorted(layout.place)]
    for vp in vps:
        if params is not None and vp.global_index not in params:
            continue
        for h in layout.fp32_holders(vp):
            n = h.hi - h.lo
            fp32[(h.rank, vp.global_index)] = {
                k: arenas[i][h.offset:h.offset + n] for i, k in enumerate(("main", "exp_avg", "exp_avg_sq"))}
        for h in layout.bf16_holders(vp):
            n = h.hi - h.lo
            bf16[(layout.shard_keys[h.rank], vp.global_index)] = arenas[ARENA_PARAM][h.offset:h.offset + n]
    return fp32, bf16


def compare(got32, gotbf, want32, wantbf):
    """Returns a list of mismatch descriptions (empty when bit-exact and complete)."""
    errs = []
    if set(got32) != set(want32):
        errs.append(f"fp32 piece keys differ: {sorted(set(got32) ^ set(want32))[:5]}")
    for k in set(got32) & set(want32):
        for kind in ("main", "exp_avg", "exp_avg_sq"):
            g = np.asarray(got32[k][kind]).view(np.uint32)
            w = np.asarray(want32[k][kind]).view(np.uint32)
            if g.shape != w.shape or not np.array_equal(g, w):
                bad = np.flatnonzero(g != w) if g.shape == w.shape else []
                errs.append(f"fp32 {k} {kind}: {len(bad)} differ, first {bad[:3]}")
    if set(gotbf) != set(wantbf):
        errs.append(f"bf16 keys differ: {sorted(set(gotbf) ^ set(wantbf))[:5]}")
    for k in set(gotbf) & set(wantbf):
        if not np.array_equal(np.asarray(gotbf[k]).view(np.uint16), np.asarray(wantbf[k]).view(np.uint16)):
            errs.append(f"bf16 {k} differs")
    return errs


def strat(ps):
    return Strat.of(ps)


def small_llama2_tied():
    return ms.ModelSpec(name="small-llama2-tied", num_layers=4, hidden_size=256, num_attention_heads=4,
                        ffn_hidden_size=688, padded_vocab_size=1024, ddp_bucket_size=150_000,
                        overlap_grad_reduce=True, untie_embeddings_and_output_weights=False)


SMALL_CASES.append(("llama2_tied_pp1_pp2_pp4_tp2pp1",
                    small_llama2_tied, [PS(8, 1, 1), PS(8, 1, 2), PS(8, 2, 4), PS(8, 2, 1)]))


def small_ragged():
    """Shapes that are not multiples of 64 or 8 (hidden 200, FFN 520, vocabulary 1000) and small
    buckets: parameter starts, bucket ends and DP shards land on padding, rows on odd offsets."""
    return ms.ModelSpec(name="small-ragged", num_layers=2, hidden_size=200, num_attention_heads=4,
                        ffn_hidden_size=520, padded_vocab_size=1000, ddp_bucket_size=40_000,
                        overlap_grad_reduce=True)


SMALL_CASES.append(("ragged_tp2dp4_dp6_tp4dp2_tp2dp3",
                    small_ragged, [PS(8, 2, 1), PS(6, 1, 1), PS(8, 4, 1), PS(6, 2, 1)]))


# Vocabulary re-padding switches: (spec factory, vocab size, src strategy, dst strategy).
REPAD_CASES = [
    (small_llama3, 2300, PS(8, 2, 2), PS(8, 4, 1)),        # 2304 -> 2560, PP merge
    (small_llama3, 2300, PS(8, 4, 1), PS(8, 2, 2)),        # 2560 -> 2304, dropped rows not read
    (small_llama3, 1100, PS(8, 1, 1), PS(8, 2, 1)),        # 1152 -> 1280
    (small_llama2_tied, 900, PS(8, 1, 2), PS(8, 4, 1)),    # tied output layer, 1024 at both sizes
    (small_llama2_tied, 1100, PS(8, 2, 2), PS(8, 4, 2)),   # tied, 1280 -> 1536, output at PP 1
]


def repad_spaces(spec, tps):
    """Virtual models of ``spec`` at Megatron's padded vocabulary for each TP size."""
    from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
    return [build_virtual_model(spec.with_padded_vocab(spec.padded_vocab_for_tp(t))) for t in tps]


def compare_numpy(table, groups, aux_groups, n_groups, src, dst):
    """Reference semantics of emrs_plan_compare on host arrays (any integer dtype; viewed per segment).

    Returns ``n_groups`` records of _native.COMPARE_DTYPE.  fp32 and bf16
    differences are taken in fp32, squared in fp64, as compare_ckpt.py's
    figures define them (tools/ckpt/compare_ckpt.py:52-66).  A group with no
    mismatching element reports 0 in every figure, its sum of squares of the
    expected values included (its RMS and relative RMS are 0 either way).
    """
    from elasticmegatron_amd._native import COMPARE_DTYPE

    out = np.zeros(n_groups, dtype=COMPARE_DTYPE)
    udt = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}

    def acc(g, e, a, eb):
        r = out[g]
        r["elements"] += e.size
        mism = e != a
        r["mismatches"] += int(mism.sum())
        if eb not in (2, 4):
            return
        if eb == 2:
            e32 = (e.astype(np.uint32) << np.uint32(16)).view(np.float32)
            a32 = (a.astype(np.uint32) << np.uint32(16)).view(np.float32)
        else:
            e32, a32 = e.view(np.float32), a.view(np.float32)
        with np.errstate(all="ignore"):
            fe = np.isfinite(e32)
            r["sum_sq_expected"] += float(np.sum(e32[fe].astype(np.float64) ** 2))
            d = np.abs(a32 - e32)
            fin = np.isfinite(d)
            r["nonfinite"] += int((mism & ~fin).sum())
            sel = mism & fin
            if sel.any():
                r["sum_sq_diff"] += float(np.sum(d[sel].astype(np.float64) ** 2))
                r["max_abs_diff"] = max(float(r["max_abs_diff"]), float(d[sel].max()))
                rel = (d / (np.abs(e32) + np.float32(1e-12))).astype(np.float32)
                r["max_rel_diff"] = max(float(r["max_rel_diff"]), float(rel[sel].max()))

    for s, g, ga in zip(table, groups, aux_groups):
        eb = int(s["elem_bytes"])
        n, rows = int(s["len"]), int(s["rows"])
        if n == 0:
            continue
        d_arr = dst[int(s["dst_buf"])].view(udt[eb])
        act = _view(d_arr, int(s["dst_off"]), rows, n, int(s["dst_stride"])).reshape(-1)
        if int(s["flags"]) & 2:
            exp = np.zeros(act.shape, dtype=act.dtype)
        else:
            s_arr = src[int(s["src_buf"])].view(udt[eb])
            exp = _view(s_arr, int(s["src_off"]), rows, n, int(s["src_stride"])).reshape(-1)
        acc(int(g), exp, act, eb)
        if int(s["flags"]) & 1:
            aux = dst[int(s["aux_buf"])].view(np.uint16)
            act_a = _view(aux, int(s["aux_off"]), rows, n, int(s["aux_stride"])).reshape(-1)
            acc(int(ga), bf16_rne_bits(exp.view(np.uint32)), act_a, 2)
        if int(s["flags"]) & 4:
            aux = dst[int(s["aux_buf"])].view(udt[eb])
            acc(int(ga), exp, _view(aux, int(s["aux_off"]), rows, n, int(s["aux_stride"])).reshape(-1), eb)
    out["sum_sq_expected"][out["mismatches"] == 0] = 0.0
    return out


# Bit patterns written into destination arenas before a switch: every element the layout does not
# store (rank alignment, bucket and parameter-start padding, shard alignment) must still hold them
# afterwards.  Neither is a value the generator produces for its kind.
CANARY32 = -559038737     # 0xDEADBEEF as int32
CANARY16 = -16657         # 0xBEEF as int16


def stored_runs(layout):
    """([start, end) runs of the fp32 arenas, runs of the bf16 arena) holding state, merged and sorted.

    The three fp32 arenas share one layout.  Everything outside the runs is padding."""
    space = layout.space
    r32, r16 = [], []
    for g in sorted(layout.place):
        vp = space.all_virtual_params[g]
        r32 += [(h.offset, h.offset + h.hi - h.lo) for h in layout.fp32_holders(vp)]
        r16 += [(h.offset, h.offset + h.hi - h.lo) for h in layout.bf16_holders(vp)]

    def merge(runs):
        out = []
        for a, b in sorted(runs):
            if b <= a:
                continue
            if out and a <= out[-1][1]:
                assert a == out[-1][1], "two holders overlap"
                out[-1][1] = max(out[-1][1], b)
            else:
                out.append([a, b])
        return [tuple(r) for r in out]

    return merge(r32), merge(r16)


def fill_canaries(state):
    """Write the canary into every element of a state's arenas (torch tensors, any device)."""
    import torch

    for t in (state.main, state.exp_avg, state.exp_avg_sq):
        t.view(torch.int32).fill_(CANARY32)
    state.param.view(torch.int16).fill_(CANARY16)


def padding_gaps(runs, n):
    """The [start, end) ranges of [0, n) outside the sorted, merged ``runs``."""
    gaps, at = [], 0
    for a, b in runs:
        if a > at:
            gaps.append((at, a))
        at = b
    if at < n:
        gaps.append((at, n))
    return gaps


def padding_damage(state, bf16=True):
    """Number of padding elements of a state's arenas (the bf16 one only with ``bf16``) that no
    longer hold the canary.  Only the gaps are read, so full-size arenas need no mask."""
    import torch

    r32, r16 = stored_runs(state.layout)
    bad = 0
    checks = [((state.main, state.exp_avg, state.exp_avg_sq), r32, CANARY32, torch.int32)]
    if bf16:
        checks.append(((state.param,), r16, CANARY16, torch.int16))
    for arenas, runs, canary, dt in checks:
        for a, b in padding_gaps(runs, arenas[0].numel()):
            for t in arenas:
                bad += int(torch.count_nonzero(t.view(dt)[a:b] != canary))
    return bad


def perturb_per_rank(state_or_world, layout=None):
    """Make every rank's fp32 shard distinct: XOR the low mantissa bits of rank g's elements of kind k
    with (g * 3 + k + 1) & 0x7F.  Takes a TrainingState (device arenas, in place) or an Oracle-1 world
    ({pid: {rank: OptInfo}}, in place), so that both sides start from the same per-rank values."""
    import torch

    def mask(g, k):
        return (g * 3 + k + 1) & 0x7F

    if isinstance(state_or_world, dict):
        for infos in state_or_world.values():
            for g, info in infos.items():
                info.tensors = [(t.view(torch.int32) ^ mask(g, k)).view(torch.float32)
                                for k, t in enumerate(info.tensors)]
                info.orig = info.tensors
        return
    st = state_or_world
    lay = st.layout
    for g in range(lay.strategy.world_size):
        a, b = lay.rank_fp32_slice(g)
        for k, t in enumerate((st.main, st.exp_avg, st.exp_avg_sq)):
            v = t.view(torch.int32)[a:b]
            v.bitwise_xor_(mask(g, k))
