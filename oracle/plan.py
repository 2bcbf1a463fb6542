"""The reference's per-parameter reshard plan, restated (test infrastructure).

Follows elastic_megatron/resharding/: TP maps resharding_tp.py:94-191,
stages resharding_pp.py:96-122, EP ranks resharding_dp.py:21-34, DP
distributions resharding_dp.py:224-409 (Megatron layout via
oracle.megatron_buffer), global ranks resharding.py:19-51, aligned ranks
resharding_dp.py:120-133, global send/recv maps resharding.py:54-162.
Ranges are tuples of (start, end) per dimension of the TP-local shape.
"""

from . import megatron_buffer
from .model import numel


class Strat:
    def __init__(self, W, tp, pp, cp=1, inst=1, ep=1, etp=None):
        self.W, self.tp, self.pp, self.cp, self.inst, self.ep = W, tp, pp, cp, inst, ep
        self.etp = tp if etp is None else etp
        self.dp = W // (tp * pp * cp)
        self.pdp = self.dp * cp // inst
        self.edp = W // (self.etp * ep * pp)

    @classmethod
    def of(cls, s):
        return cls(s.world_size, s.tensor_model_parallel_size, s.pipeline_model_parallel_size,
                   s.context_parallel_size, s.num_distributed_optimizer_instances,
                   s.expert_model_parallel_size, s.expert_tensor_parallel_size)


def tp_size(strat, p):
    return strat.etp if p["expert"] is not None else strat.tp


def local_shape(p, T):
    shape = list(p["shape"])
    if p["tp"] and T > 1:
        shape[p["pdim"]] //= T
    return tuple(shape)


def stage(p, pp, L):
    w = p["where"]
    if w == "emb":
        return 0
    if w == "final":
        return pp - 1
    if w == "out":
        return -1 if (p["shared"] and pp == 1) else pp - 1
    return p["layer"] // (L // pp)


def ep_rank(p, strat, E):
    return None if p["expert"] is None else p["expert"] // (E // strat.ep)


def _chunk(rng, k, dim):
    a, b = rng[dim]
    n = (b - a) // k
    assert n * k == b - a
    out = []
    for i in range(k):
        r = list(rng)
        r[dim] = (a + i * n, a + (i + 1) * n)
        out.append(tuple(r))
    return out


def tp_maps(p, Ts, Td):
    """(send {s: {d: range}}, recv {d: {s: range}}) in TP-local coordinates."""
    whole_s = tuple((0, n) for n in local_shape(p, Ts))
    whole_d = tuple((0, n) for n in local_shape(p, Td))
    send, recv = {}, {}
    if not p["tp"]:
        send[0] = {d: whole_s for d in range(Td)}
        for d in range(Td):
            recv[d] = {0: whole_s}
        return send, recv
    dim = p["pdim"]
    if Ts < Td:
        k = Td // Ts
        ch = _chunk(whole_s, k, dim)
        for s in range(Ts):
            for i in range(k):
                send.setdefault(s, {})[s * k + i] = ch[i]
                recv[s * k + i] = {s: ch[0]}
        return send, recv
    k = Ts // Td
    ch = _chunk(whole_d, k, dim)
    for d in range(Td):
        for i in range(k):
            recv.setdefault(d, {})[d * k + i] = ch[i]
            send[d * k + i] = {d: ch[0]}
    return send, recv


def global_rank(strat, pp, dp, ep, tp):
    if ep is None:
        dps, eps, ep, tps = strat.pdp, 1, 0, strat.tp
    else:
        dps, eps, tps = strat.edp, strat.ep, strat.etp
    return pp * dps * eps * tps + dp * eps * tps + ep * tps + tp


def dp_distributions(inv, strat, hp):
    """{param id: {dp rank: (lo, hi)}} for every parameter placed at ``strat``."""
    out = {}
    L = hp.num_layers
    for sid in range(strat.pp):
        on = [p for p in inv if stage(p, strat.pp, L) == sid]
        no_buckets = (not hp.overlap_grad_reduce) or sid > 0 or hp.overlap_param_gather_with_optimizer_step
        bucket = None if no_buckets else (hp.ddp_bucket_size or max(40_000_000, 1_000_000 * strat.pdp))
        dense = [p for p in on if p["expert"] is None]
        if dense:
            d = megatron_buffer.distribution([numel(local_shape(p, strat.tp)) for p in dense], strat.pdp, bucket,
                                             [p["shared"] for p in dense])
            for i, p in enumerate(dense):
                out[p["id"]] = d[i]
        experts = [p for p in on if p["expert"] is not None]
        if experts:
            by_ep = {}
            for p in experts:
                by_ep.setdefault(ep_rank(p, strat, hp.num_experts), []).append(p)
            d = megatron_buffer.distribution([numel(local_shape(p, strat.etp)) for p in by_ep[0]], strat.edp,
                                             bucket)
            for lst in by_ep.values():
                for i, p in enumerate(lst):
                    out[p["id"]] = d[i]
    return out


class ParamPlan:
    def __init__(self, p, src, dst, src_dist, dst_dist, hp):
        L = hp.num_layers
        self.p = p
        self.src, self.dst = src, dst
        self.src_pp, self.dst_pp = stage(p, src.pp, L), stage(p, dst.pp, L)
        self.src_ep = ep_rank(p, src, hp.num_experts) if p["expert"] is not None else None
        self.dst_ep = ep_rank(p, dst, hp.num_experts) if p["expert"] is not None else None
        self.Ts, self.Td = tp_size(src, p), tp_size(dst, p)
        self.send, self.recv = tp_maps(p, self.Ts, self.Td)
        self.src_dist, self.dst_dist = src_dist, dst_dist
        self.skip = self.src_pp == -1 or self.dst_pp == -1
        if self.skip:
            return
        sa, da = next(iter(src_dist)), next(iter(dst_dist))
        g_s = lambda t: global_rank(src, self.src_pp, sa, self.src_ep, t)
        g_d = lambda t: global_rank(dst, self.dst_pp, da, self.dst_ep, t)
        self.global_send = {g_s(s): {g_d(d): r for d, r in m.items()} for s, m in self.send.items()}
        self.global_recv = {g_d(d): {g_s(s): r for s, r in m.items()} for d, m in self.recv.items()}

    def src_dist_g(self, tp):
        return {global_rank(self.src, self.src_pp, r, self.src_ep, tp): v for r, v in self.src_dist.items()}

    def dst_dist_g(self, tp):
        return {global_rank(self.dst, self.dst_pp, r, self.dst_ep, tp): v for r, v in self.dst_dist.items()}

    def src_holders(self):
        """[(global rank, tp rank, (lo, hi))] of every source rank holding a piece."""
        return [(g, t, v) for t in range(self.Ts) for g, v in self.src_dist_g(t).items()]

    def dst_holders(self):
        return [(g, t, v) for t in range(self.Td) for g, v in self.dst_dist_g(t).items()]
