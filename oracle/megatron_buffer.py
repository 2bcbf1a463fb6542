"""Megatron-core DDP buffer layout (test infrastructure; parity unpinned).

Restates the published layout algorithm of megatron/core/distributed/
param_and_grad_buffer.py (core_r0.11.0), which the reference obtains by
instantiating ``_ParamAndGradBuffer`` under mocks
(elastic_megatron/resharding/resharding_dp.py:155-315).  Megatron-core is not
available here, so this restatement is checked by invariants and by known
answers derived by hand from the published algorithm (parity unpinned).
"""

import math


def layout(numels, dp, bucket_size, shared=None, dist_opt=True):
    """Returns (param_ranges {i: (start, end)}, buckets [(start, end, [i, ...])]).

    Parameters are placed last-to-first; starts padded to 64 elements; a
    bucket is closed once it spans >= bucket_size elements (or around a
    shared-embedding parameter) and its end padded to lcm(dp, 128).
    """
    shared = shared or [False] * len(numels)
    q = math.lcm(dp, 128) if dist_opt else 1
    a = 64 if dist_opt else 1
    up = lambda x, m: (x + m - 1) // m * m
    ranges, buckets = {}, []
    b_start, cur, members = 0, 0, []
    end = 0
    for i in range(len(numels) - 1, -1, -1):
        cur = up(cur, a)
        if shared[i] and dist_opt:
            if cur % dp:
                cur = up(cur, q)
            if members:
                e = up(cur, q)
                buckets.append((b_start, e, members))
                b_start, members = e, []
        end = cur + numels[i]
        ranges[i] = (cur, end)
        members = members + [i]
        if (bucket_size is not None and end - b_start >= bucket_size) or (shared[i] and dist_opt):
            e = up(end, q)
            buckets.append((b_start, e, members))
            b_start, members = e, []
            cur = e
        else:
            cur = end
    if members:
        buckets.append((b_start, up(end, q), members))
    return ranges, buckets


def distribution(numels, dp, bucket_size, shared=None, dist_opt=True):
    """{i: {dp_rank: (lo, hi)}} in param-local coordinates, dp ranks ascending."""
    ranges, buckets = layout(numels, dp, bucket_size, shared, dist_opt)
    out = {i: {} for i in ranges}
    for bs, be, members in buckets:
        # resharding_dp.py:276-278 makes each member's range relative to its bucket start, which
        # Range.normalize (util.py:65-69) refuses for a member starting before it.
        assert all(ranges[i][0] >= bs for i in members), "a parameter starts before its bucket"
        s = (be - bs) // dp
        for r in range(dp):
            lo_r, hi_r = bs + r * s, bs + (r + 1) * s
            for i in members:
                ps, pe = ranges[i]
                lo, hi = max(ps, lo_r), min(pe, hi_r)
                if lo < hi:
                    out[i][r] = (lo - ps, hi - ps)
    return {i: dict(sorted(d.items())) for i, d in out.items()}
