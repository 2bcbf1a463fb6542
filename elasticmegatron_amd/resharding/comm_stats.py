"""The reference's communication-volume figure for a switch.

The reference logs ``communication bytes`` as each rank's count of fp32
optimizer bytes it sent to, or received from, *other* ranks (self copies
excluded), maxed over ranks and printed in GiB
(elastic_megatron/transfer/communicator.py:61-122,
elastic_megatron/elastic_manager.py:158-178).  On one device every hop is a
local copy, so the figure is derived from the plan: the DP gather onto the
aligned rank of every source TP rank (transfer.py:143-180), the exchange
between aligned ranks (transfer.py:182-228) and the DP scatter from the
aligned destination rank (transfer.py:230-269), plus, for tied embeddings at
destination PP > 1, the broadcast of the word embedding's state to the
output layer over the embedding group (transfer.py:103-141).
"""

from __future__ import annotations

from collections import defaultdict
from typing import Dict

from ..megatron_manager.parallel_strategy import ParallelStrategy, global_rank_of

FP32_TENSORS_BYTES = 12  # main, exp_avg, exp_avg_sq


def reference_comm_bytes(space, src: ParallelStrategy, dst: ParallelStrategy) -> Dict[int, int]:
    """Per global rank: bytes sent to and received from other ranks."""
    space.register_reshard(src, dst)
    per_rank: Dict[int, int] = defaultdict(int)
    for vp in space.all_virtual_params:
        plan = vp.reshard_plan
        if vp.shared_embedding and vp.param_position_attr.layer_type.value == "output_layer":
            if dst.pipeline_model_parallel_size > 1:
                stage = vp.get_model_param_stage_id(dst.pipeline_model_parallel_size)
                for t in range(vp.tp_size_at(dst)):
                    for r, rng in vp.get_dp_distribution(dst).items():
                        n = rng.size * FP32_TENSORS_BYTES
                        per_rank[global_rank_of(dst, 0, r, None, t)] += n      # first stage sends
                        per_rank[global_rank_of(dst, stage, r, None, t)] += n  # last stage receives
            continue
        if plan is None or plan.global_send_info is None:
            continue
        dpi = plan.data_parallel_resharding_info
        ts, td = vp.tp_size_at(src), vp.tp_size_at(dst)
        for strat, dist, pp, ep, tps, gather in ((src, dpi.src_dp_distribution, plan.src_pp_rank, plan.src_ep_rank,
                                                   ts, True),
                                                  (dst, dpi.dst_dp_distribution, plan.dst_pp_rank, plan.dst_ep_rank,
                                                   td, False)):
            if len(dist) <= 1:
                continue
            for t in range(tps):
                ranks = {global_rank_of(strat, pp, r, ep, t): rng for r, rng in dist.items()}
                aligned = next(iter(ranks))
                for g, rng in ranks.items():
                    if g == aligned:
                        continue
                    n = rng.size * FP32_TENSORS_BYTES
                    per_rank[g] += n        # gather: g sends; scatter: g receives
                    per_rank[aligned] += n
        for s, peers in plan.global_send_info.items():
            for d, rng in peers.items():
                if s != d:
                    n = rng.size * FP32_TENSORS_BYTES
                    per_rank[s] += n
                    per_rank[d] += n
    return dict(per_rank)
