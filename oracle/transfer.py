"""Oracle-1: the reference's three-pass executor on CPU torch tensors (test infrastructure).

Restates elastic_megatron/transfer/transfer.py:36-341 for a whole simulated
world in one process.  Point-to-point messages go through a FIFO mailbox per
(sender, receiver) pair, which is also how the reference's communicator
serves a rank's messages to itself (communicator.py:38-44, :61-96).  The
ranks of the world run each pass in lock step: for every parameter all sends
of a pass are posted before any receive of that pass is taken, which is the
ordering the blocking collectives of the reference enforce.

Storage release/rebuild (resharding_metadata.py:58-65) only manages memory and
is not modelled; staging tensors are filled with NaN so that an element that
is never written shows up in comparisons.
"""

from collections import defaultdict, deque

import numpy as np
import torch

from .canonical import piece_values, shard_key
from .model import numel
from .plan import ParamPlan, dp_distributions, ep_rank, global_rank, local_shape, stage, tp_size

KINDS = ("main", "exp_avg", "exp_avg_sq")


class OptInfo:
    """One rank's OptimizerTensorInfo of one parameter (resharding_metadata.py:19-96)."""

    def __init__(self, tensors, rng, model_shape):
        self.tensors = tensors          # current optimizer_tensors
        self.orig = tensors
        self.rng = rng                  # (lo, hi) owned by this rank
        self.model_shape = model_shape  # TP-local shape
        self.padded = False

    @property
    def model_numel(self):
        return numel(self.model_shape)

    def create_padded(self):  # resharding_metadata.py:67-88
        assert self.rng[0] == 0, "the aligned rank owns the start of the parameter"
        if self.rng[1] - self.rng[0] == self.model_numel:
            return
        self.tensors = [torch.full((self.model_numel,), float("nan"), dtype=torch.float32) for _ in range(3)]
        self.padded = True

    def release_padded(self):  # resharding_metadata.py:90-96
        if self.padded:
            self.tensors = self.orig
            self.padded = False

    def shuffle_swiglu(self, k):  # resharding_metadata.py:98-138
        if k <= 1:
            return
        for t in self.tensors:
            n = t.numel()
            w, v = torch.chunk(t.view(-1), 2)
            ws, vs = torch.chunk(w, k), torch.chunk(v, k)
            new = torch.empty(n, dtype=t.dtype)
            pos, step = 0, n // 2 // k
            for a, b in zip(ws, vs):
                new[pos:pos + step].copy_(a)
                pos += step
                new[pos:pos + step].copy_(b)
                pos += step
            assert pos == n
            t.copy_(new)

    def unshuffle_swiglu(self, k):  # resharding_metadata.py:140-178
        if k <= 1:
            return
        for t in self.tensors:
            n = t.numel()
            new = torch.empty(n, dtype=t.dtype)
            w, v = torch.chunk(new, 2)
            ws, vs = torch.chunk(w, k), torch.chunk(v, k)
            pos, step = 0, n // 2 // k
            for a, b in zip(ws, vs):
                a.copy_(t[pos:pos + step])
                pos += step
                b.copy_(t[pos:pos + step])
                pos += step
            assert pos == n
            t.copy_(new)


def _slices(shape, rng):
    """ParamRange.get_sub_range_slices of the whole local shape (util.py:174-189)."""
    return tuple(slice(a, b) for a, b in rng)


class Mailbox:
    def __init__(self):
        self.q = defaultdict(deque)
        self.cross_rank_bytes = defaultdict(int)

    def send(self, frm, to, t):
        self.q[(frm, to)].append(t.detach().clone().contiguous())
        if frm != to:
            self.cross_rank_bytes[frm] += t.numel() * t.element_size()

    def recv(self, frm, to, out):
        t = self.q[(frm, to)].popleft()
        out.copy_(t.view(out.shape))
        if frm != to:
            self.cross_rank_bytes[to] += t.numel() * t.element_size()

    def empty(self):
        return all(len(v) == 0 for v in self.q.values())


def holders(inv, hp, strat, p, dist):
    """[(global rank, tp rank, (lo, hi))] of every rank holding a piece of ``p`` (all instances)."""
    s = stage(p, strat.pp, hp.num_layers)
    T = tp_size(strat, p)
    out = []
    if p["expert"] is None:
        for inst in range(strat.inst):
            for t in range(T):
                for r, v in dist.items():
                    out.append((s * (strat.dp * strat.cp * strat.tp) + (inst * strat.pdp + r) * strat.tp + t, t, v))
        return out
    e = ep_rank(p, strat, hp.num_experts)
    return [(global_rank(strat, s, r, e, t), t, v) for t in range(T) for r, v in dist.items()]


def build_src_world(inv, hp, src, seed, params=None):
    """{pid: {rank: OptInfo}} with the seeded synthetic values."""
    dist = dp_distributions(inv, src, hp)
    world = {}
    for p in inv:
        if (params is not None and p["id"] not in params) or p["id"] not in dist:
            continue
        T = tp_size(src, p)
        shp = local_shape(p, T)
        for g, t, (lo, hi) in holders(inv, hp, src, p, dist[p["id"]]):
            v = piece_values(seed, p, T, t, lo, hi)
            world.setdefault(p["id"], {})[g] = OptInfo([torch.from_numpy(v[k].copy()) for k in KINDS], (lo, hi), shp)
    return world


def transfer(inv, hp, src, dst, src_world, params=None, dists=None):
    """Run transfer.py:291-341 over the simulated world; returns (dst fp32 world, dst bf16, mailbox).

    ``dists``: the (source, destination) DP distributions of every parameter, when the caller has
    them already (the reference computes them when it plans, outside its timed executor)."""
    sd, dd = dists if dists is not None else (dp_distributions(inv, src, hp), dp_distributions(inv, dst, hp))
    mb = Mailbox()
    plans, dst_world = {}, {}
    for p in inv:
        pid = p["id"]
        if (params is not None and pid not in params) or pid not in sd or pid not in dd:
            continue
        if p["shared"] and p["where"] == "out":  # transfer.py:324-330
            continue
        plan = ParamPlan(p, src, dst, sd[pid], dd[pid], hp)
        if plan.skip:
            continue
        plans[pid] = plan
        shp = local_shape(p, plan.Td)
        dst_world[pid] = {g: OptInfo([torch.full((hi - lo,), float("nan"), dtype=torch.float32) for _ in KINDS],
                                     (lo, hi), shp)
                          for g, t, (lo, hi) in plan.dst_holders()}
    tp_of_src = {pid: {g: t for g, t, _ in pl.src_holders()} for pid, pl in plans.items()}
    tp_of_dst = {pid: {g: t for g, t, _ in pl.dst_holders()} for pid, pl in plans.items()}

    # Pass 1: DP gather onto the aligned rank, then SwiGLU shuffle (transfer.py:143-180).
    for pid, plan in plans.items():
        infos = src_world[pid]
        for g, info in infos.items():
            dist = plan.src_dist_g(tp_of_src[pid][g])
            aligned = next(iter(dist))
            if len(dist) > 1:
                for t in info.tensors:
                    mb.send(g, aligned, t.view(-1))
        for g, info in infos.items():
            dist = plan.src_dist_g(tp_of_src[pid][g])
            aligned = next(iter(dist))
            if len(dist) > 1 and g == aligned:
                info.create_padded()
                for r, (lo, hi) in dist.items():
                    for t in info.tensors:
                        mb.recv(r, g, t.view(-1)[lo:hi])
            if plan.p["swiglu"] and g == aligned:
                k = len(plan.global_send[g])
                assert k >= 1
                info.shuffle_swiglu(k)

    # Pass 2: exchange between aligned ranks (transfer.py:182-228); sends before receives.
    for pid, plan in plans.items():
        infos = src_world[pid]
        for g, peers in plan.global_send.items():
            info = infos[g]
            for d, rng in peers.items():
                for t in info.tensors:
                    mb.send(g, d, t.view(info.model_shape)[_slices(info.model_shape, rng)])
            info.release_padded()
        for g, info in dst_world[pid].items():
            aligned = next(iter(plan.dst_dist_g(tp_of_dst[pid][g])))
            if g != aligned:
                continue
            info.create_padded()
            for s, rng in plan.global_recv[g].items():
                for t in info.tensors:
                    mb.recv(s, g, t.view(info.model_shape)[_slices(info.model_shape, rng)])

    # Pass 3: SwiGLU unshuffle, DP scatter from the aligned rank (transfer.py:230-269).
    for pid, plan in plans.items():
        infos = dst_world[pid]
        for g, info in infos.items():
            dist = plan.dst_dist_g(tp_of_dst[pid][g])
            aligned = next(iter(dist))
            if plan.p["swiglu"] and g == aligned:
                k = len(plan.global_recv[g])
                assert k >= 1
                info.unshuffle_swiglu(k)
        for g, info in infos.items():
            dist = plan.dst_dist_g(tp_of_dst[pid][g])
            if len(dist) > 1 and g == next(iter(dist)):
                for r, (lo, hi) in dist.items():
                    for t in info.tensors:
                        mb.send(g, r, t.view(-1)[lo:hi])
        for g, info in infos.items():
            dist = plan.dst_dist_g(tp_of_dst[pid][g])
            aligned = next(iter(dist))
            if len(dist) > 1:
                if g == aligned:
                    info.release_padded()
                for t in info.tensors:
                    mb.recv(aligned, g, t.view(-1))
            elif g == aligned:
                info.release_padded()
    assert mb.empty(), "unmatched messages"
    tie_output_layer(inv, hp, dst, dd, dst_world, tp_of_dst, mb, params)
    return dst_world, rebuild_bf16(inv, hp, dst, dst_world, plans, tp_of_dst), mb


def tie_output_layer(inv, hp, dst, dd, dst_world, tp_of_dst, mb, params=None):
    """Broadcast the word embedding's new state to a tied output layer (transfer.py:103-141).

    Only with tied embeddings and destination PP > 1: in every embedding
    group (first- and last-stage ranks of one (dp, tp) position) the
    first-stage rank broadcasts its three optimizer tensors.
    """
    out = [p for p in inv if p["shared"] and p["where"] == "out"]
    if not out or dst.pp == 1:
        return
    p_out, p_emb = out[0], inv[0]
    if (params is not None and p_out["id"] not in params) or p_out["id"] not in dd:
        return
    infos = {}
    for g, t, (lo, hi) in holders(inv, hp, dst, p_out, dd[p_out["id"]]):
        r = next(r for r, v in dd[p_out["id"]].items() if v == (lo, hi))
        g0 = global_rank(dst, 0, r, None, t)
        src_info = dst_world[p_emb["id"]][g0]
        assert src_info.rng == (lo, hi), "tied parameters must share their DP distribution"
        info = OptInfo([torch.empty_like(x) for x in src_info.tensors], (lo, hi), src_info.model_shape)
        for a, b in zip(src_info.tensors, info.tensors):
            mb.send(g0, g, a)
            mb.recv(g0, g, b)
        infos[g] = info
    dst_world[p_out["id"]] = infos
    tp_of_dst[p_out["id"]] = {g: t for g, t, _ in holders(inv, hp, dst, p_out, dd[p_out["id"]])}


def rebuild_bf16(inv, hp, dst, dst_world, plans, tp_of_dst):
    """Cast main to bf16 and gather the DP pieces into each model shard (training_state.py:176-197)."""
    out = {}
    for pid, infos in dst_world.items():
        p = inv[pid]
        for g, info in infos.items():
            t = tp_of_dst[pid][g]
            key = (shard_key(p, dst, hp, t), pid)
            buf = out.get(key)
            if buf is None:
                buf = out[key] = np.zeros(info.model_numel, dtype=np.uint16)
            lo, hi = info.rng
            buf[lo:hi] = info.tensors[0].to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    return out


def redundant_backup(inv, hp, src, dst, src_world, scale_up, params=None, dist=None, group_src=0):
    """Group-ZeRO switch (transfer.py:343-388): migrate on the master, broadcast to the instances.

    ``params``: the parameter ids to move (default: all); ``src_world`` must hold them.
    ``dist``: the destination's DP distributions, when the caller has them already.
    ``group_src``: on a scale-up, the master is the ``group_src``-th rank of each inter-instance
    group (transfer.py:360-371), so instance ``group_src``'s shard is what every instance gets."""
    dist = dist if dist is not None else dp_distributions(inv, dst, hp)
    out = {}
    for p in inv:
        pid = p["id"]
        if pid not in dist or (params is not None and pid not in params):
            continue
        T = dst.tp
        for t in range(T):
            for r, (lo, hi) in dist[pid].items():
                for inst in range(dst.inst):
                    s = stage(p, dst.pp, hp.num_layers)
                    g = s * (dst.dp * dst.cp * dst.tp) + (inst * dst.pdp + r) * dst.tp + t
                    src_inst = group_src if scale_up else inst
                    gs = s * (src.dp * src.cp * src.tp) + (src_inst * src.pdp + r) * src.tp + t
                    info = src_world[pid][gs]
                    assert info.rng == (lo, hi)
                    out.setdefault(pid, {})[g] = OptInfo([x.clone() for x in info.tensors], (lo, hi),
                                                         info.model_shape)
    return out


def flatten(world_fp32):
    """{(rank, pid): {kind: numpy array}} from {pid: {rank: OptInfo}}."""
    out = {}
    for pid, infos in world_fp32.items():
        for g, info in infos.items():
            out[(g, pid)] = {k: info.tensors[i].numpy() for i, k in enumerate(KINDS)}
    return out
